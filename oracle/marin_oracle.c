/*
 * CPU oracle: a C restatement of Marin's CPU arithmetic for the quantized decode path.
 *
 * TEST INFRASTRUCTURE. Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, always as the
 * checker or as the timed host baseline; the HIP product path never calls it. Built with -ffp-contract=off so that a
 * plain `a * b + c` rounds twice, as Rust does, and fmaf() marks the places where the reference uses a fused
 * mul_add. Every function names the reference file:line it restates; which test pins it is in marin_oracle.h.
 */
#include "marin_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static int g_threads = 1;
void or_set_threads(int n) { g_threads = n > 0 ? n : 1; }

static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* tensor/src/matrix.rs:31 */
float or_bf16_to_f32(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

uint16_t or_f32_to_bf16(float value) {
    uint32_t u = f32_bits(value);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* cuda/tests/kv_round/mod.rs:3-18 (saturating f16 rounding of the store kernel), as bits. */
uint16_t or_f32_to_f16_sat(float x) {
    uint32_t u = f32_bits(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    float m = fabsf(x);
    if (m != m) return (uint16_t)(sign | 0x7e00u);
    if (m >= 65504.0f) return (uint16_t)(sign | 0x7bffu);
    if (m < 6.103515625e-05f) { /* subnormal: multiples of 2^-24 */
        float q = nearbyintf(m * 16777216.0f); /* exact scaling, ties to even (default mode) */
        return (uint16_t)(sign | (uint16_t)q);
    }
    int e = (int)((u >> 23) & 0xff) - 127; /* -14..15 */
    uint32_t mant = u & 0x7fffffu;
    uint32_t keep = mant >> 13, rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u))) keep++;
    uint32_t h = ((uint32_t)(e + 15) << 10) + keep; /* carry into exponent is correct rounding */
    if (h >= 0x7c00u) h = 0x7bffu;
    return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

/* ---- a1: tensor/src/quant.rs:181-234 ---- */
long or_quantize(const uint16_t *weights, size_t rows, size_t cols, int bits, size_t group, uint8_t *codes,
                 float *scales) {
    if (group == 0 || group % 32 != 0 || cols == 0 || rows == 0 || cols % group != 0) return -2;
    if (bits != 8 && bits != 4) return -2;
    const int max = bits == 8 ? 127 : 7;
    const size_t groups = cols / group;
    const size_t row_bytes = bits == 8 ? cols : (cols + 1) / 2;
    for (size_t r = 0; r < rows; ++r) {
        const uint16_t *row = weights + r * cols;
        for (size_t g = 0; g < groups; ++g) {
            const uint16_t *grp = row + g * group;
            float largest = 0.0f;
            for (size_t i = 0; i < group; ++i) {
                float v = or_bf16_to_f32(grp[i]);
                if (!isfinite(v)) return (long)r;
                float a = fabsf(v);
                largest = a > largest ? a : largest; /* f32::max */
            }
            const float scale = largest / (float)max;
            scales[r * groups + g] = scale;
            for (size_t i = 0; i < group; ++i) {
                int code = 0;
                if (scale > 0.0f) {
                    float q = roundf(or_bf16_to_f32(grp[i]) / scale); /* f32::round: half away from zero */
                    long c = q >= 2147483647.0f ? 2147483647L : (q <= -2147483648.0f ? -2147483648L : (long)q);
                    code = (int)(c < -max ? -max : (c > max ? max : c));
                }
                const size_t col = g * group + i;
                if (bits == 8) {
                    codes[r * row_bytes + col] = (uint8_t)(int8_t)code;
                } else {
                    uint8_t nib = (uint8_t)(code + 8);
                    uint8_t *slot = &codes[r * row_bytes + col / 2];
                    if (col % 2 == 0) *slot = (uint8_t)((*slot & 0xf0u) | nib);
                    else *slot = (uint8_t)((*slot & 0x0fu) | (uint8_t)(nib << 4));
                }
            }
        }
    }
    return -1;
}

/* ---- a2: tensor/src/quant.rs:259-299 ---- */
void or_dequantize_row(const uint8_t *codes, const float *scales, size_t cols, int bits, size_t group, size_t row,
                       float *out) {
    const size_t groups = cols / group;
    const size_t row_bytes = bits == 8 ? cols : (cols + 1) / 2;
    const uint8_t *c = codes + row * row_bytes;
    const float *s = scales + row * groups;
    for (size_t i = 0; i < cols; ++i) {
        int code;
        if (bits == 8) code = (int)(int8_t)c[i];
        else code = (int)((i % 2 == 0) ? (c[i / 2] & 0xfu) : (c[i / 2] >> 4)) - 8;
        out[i] = (float)code * s[i / group];
    }
}

/* pulp's 8-lane horizontal sum: halves, then quarters, then the pair. */
static inline float reduce8(const float t[8]) {
    float a0 = t[0] + t[4], a1 = t[1] + t[5], a2 = t[2] + t[6], a3 = t[3] + t[7];
    float b0 = a0 + a2, b1 = a1 + a3;
    return b0 + b1;
}

/* ---- a5 CPU order: tensor/src/q8_gemv.rs:28-76 (8 f32 lanes, AVX2) ---- */
static void q8_gemv_rows(const uint8_t *codes, const float *scales, const float *x, float *out, size_t r0, size_t r1,
                         size_t cols, size_t group) {
    const size_t groups = cols / group;
    const size_t words_per_group = group / 4;
    /* x packed as planes: for every 32 inputs, plane p lane i = x[4i + p] (q8_gemv.rs:40-52). */
    const size_t chunks = (cols + 31) / 32;
    float *planes = (float *)calloc(chunks * 32, sizeof(float));
    for (size_t c = 0; c < chunks; ++c)
        for (size_t i = 0; i < 8; ++i)
            for (size_t p = 0; p < 4; ++p) {
                size_t idx = c * 32 + 4 * i + p;
                planes[c * 32 + p * 8 + i] = idx < cols ? x[idx] : 0.0f;
            }
    for (size_t r = r0; r < r1; ++r) {
        const uint8_t *row = codes + r * cols;
        float total[8] = {0};
        for (size_t g = 0; g < groups; ++g) {
            const uint8_t *gc = row + g * group;
            const float *gx = planes + (g * group / 32) * 32;
            float a[8] = {0}, b[8] = {0}, c[8] = {0}, d[8] = {0};
            for (size_t v = 0; v < words_per_group / 8; ++v) {
                const uint8_t *w = gc + v * 32;
                const float *xv = gx + v * 32;
                for (int i = 0; i < 8; ++i) {
                    a[i] = fmaf((float)(int8_t)w[4 * i + 0], xv[0 * 8 + i], a[i]);
                    b[i] = fmaf((float)(int8_t)w[4 * i + 1], xv[1 * 8 + i], b[i]);
                    c[i] = fmaf((float)(int8_t)w[4 * i + 2], xv[2 * 8 + i], c[i]);
                    d[i] = fmaf((float)(int8_t)w[4 * i + 3], xv[3 * 8 + i], d[i]);
                }
            }
            const float scale = scales[r * groups + g];
            for (int i = 0; i < 8; ++i) {
                float sum = (a[i] + b[i]) + (c[i] + d[i]);
                total[i] = fmaf(sum, scale, total[i]);
            }
        }
        out[r] = reduce8(total);
    }
    free(planes);
}

void or_q8_gemv(const uint8_t *codes, const float *scales, const float *x, float *out, size_t rows, size_t cols,
                size_t group) {
    if (g_threads <= 1) {
        q8_gemv_rows(codes, scales, x, out, 0, rows, cols, group);
        return;
    }
    /* Rows are independent, so splitting them changes no bit of the result. */
    const long chunk = 64;
#pragma omp parallel for schedule(dynamic, 1) num_threads(g_threads)
    for (long r0 = 0; r0 < (long)rows; r0 += chunk) {
        size_t r1 = (size_t)r0 + chunk < rows ? (size_t)r0 + chunk : rows;
        q8_gemv_rows(codes, scales, x, out, (size_t)r0, r1, cols, group);
    }
}

/* ---- tensor/src/ops.rs:5-21 ---- */
float or_dot(const float *a, const float *b, size_t n) {
    double acc[8] = {0};
    size_t full = n / 8 * 8;
    double tail = 0.0;
    for (size_t i = full; i < n; ++i) tail += (double)a[i] * (double)b[i];
    for (size_t i = 0; i < full; i += 8)
        for (int j = 0; j < 8; ++j) acc[j] += (double)a[i + j] * (double)b[i + j];
    double s = 0.0;
    for (int j = 0; j < 8; ++j) s += acc[j];
    return (float)(s + tail);
}

/* q8.rs:117-128: decode a row, then the f64 dot against every token. */
void or_matmul_dot(const uint8_t *codes, const float *scales, const float *x, float *out, size_t rows, size_t cols,
                   int bits, size_t group, size_t tokens) {
#pragma omp parallel for schedule(dynamic, 16) num_threads(g_threads)
    for (long r = 0; r < (long)rows; ++r) {
        float *row = (float *)malloc(cols * sizeof(float));
        or_dequantize_row(codes, scales, cols, bits, group, (size_t)r, row);
        for (size_t t = 0; t < tokens; ++t) out[t * rows + (size_t)r] = or_dot(row, x + t * cols, cols);
        free(row);
    }
}

static void dense_matmul(const float *w, const float *x, float *out, size_t rows, size_t cols, size_t tokens) {
#pragma omp parallel for schedule(dynamic, 16) num_threads(g_threads)
    for (long r = 0; r < (long)rows; ++r)
        for (size_t t = 0; t < tokens; ++t) out[t * rows + (size_t)r] = or_dot(w + (size_t)r * cols, x + t * cols, cols);
}

/* ---- tensor/src/kernel.rs:73-98 ---- */
float or_exp(float x) {
    x = fminf(fmaxf(x, -87.3f), 88.0f);
    const float magic = 12582912.0f;
    const float rounded = fmaf(x, 1.44269504088896340736f, magic);
    const float n = rounded - magic;
    float r = fmaf(-n, 0.6933594f, x);
    r = fmaf(-n, -2.1219444e-4f, r);
    float y = 1.9875691e-4f;
    const float coeff[5] = {1.3981999e-3f, 8.333452e-3f, 4.1665796e-2f, 1.6666665e-1f, 0.5f};
    for (int i = 0; i < 5; ++i) y = fmaf(y, r, coeff[i]);
    y = fmaf(y, r * r, r + 1.0f);
    const uint32_t exponent = f32_bits(rounded) + (127u - 0x4B400000u);
    return y * bits_f32(exponent << 23);
}

/* ---- tensor/src/norm.rs:6-58 (SIMD path) ---- */
void or_rms_norm_rows(float *x, size_t len, const float *weight, size_t dim, float eps) {
    for (size_t r = 0; r < len / dim; ++r) {
        float *row = x + r * dim;
        float sum[8] = {0};
        size_t full = dim / 8 * 8;
        for (size_t i = 0; i < full; i += 8)
            for (int j = 0; j < 8; ++j) sum[j] = fmaf(row[i + j], row[i + j], sum[j]);
        for (size_t i = full; i < dim; ++i) sum[i - full] = fmaf(row[i], row[i], sum[i - full]);
        const float mean_sq = reduce8(sum) / (float)dim;
        const float scale = 1.0f / sqrtf(mean_sq + eps);
        for (size_t i = 0; i < dim; ++i) row[i] = (row[i] * scale) * weight[i];
    }
}

/* ---- tensor/src/ops.rs:56-95 ---- */
void or_rope_tokens(float *x, size_t len, size_t token_dim, size_t head_size, size_t start, float theta) {
    const size_t half = head_size / 2;
    float *cosv = (float *)malloc(half * sizeof(float)), *sinv = (float *)malloc(half * sizeof(float));
    float *freq = (float *)malloc(half * sizeof(float));
    for (size_t i = 0; i < half; ++i) freq[i] = powf(theta, -((float)i * 2.0f / (float)head_size));
    for (size_t t = 0; t < len / token_dim; ++t) {
        const float position = (float)(start + t);
        for (size_t i = 0; i < half; ++i) {
            const float angle = position * freq[i];
            sinv[i] = sinf(angle);
            cosv[i] = cosf(angle);
        }
        for (size_t h = 0; h < token_dim / head_size; ++h) {
            float *head = x + t * token_dim + h * head_size;
            for (size_t i = 0; i < half; ++i) {
                const float a = head[i], b = head[i + half];
                head[i] = a * cosv[i] - b * sinv[i];
                head[i + half] = b * cosv[i] + a * sinv[i];
            }
        }
    }
    free(cosv);
    free(sinv);
    free(freq);
}

/* ---- tensor/src/silu.rs:48-53 ---- */
void or_silu_mul(float *gate, const float *up, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float e = or_exp(0.0f - gate[i]);
        gate[i] = (gate[i] / (1.0f + e)) * up[i];
    }
}

/* ---- tensor/src/ops.rs:23-33 ---- */
void or_softmax(float *x, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; ++i) max = x[i] > max ? x[i] : (max != max ? x[i] : max);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    for (size_t i = 0; i < n; ++i) x[i] /= sum;
}

/* attention_one.rs:84-101: four 8-lane accumulators over quads of vectors. */
static float dot4acc(const float *a, const float *b, size_t n) {
    float acc[4][8] = {{0}};
    const size_t vecs = n / 8, quads = vecs / 4;
    for (size_t q = 0; q < quads; ++q)
        for (int k = 0; k < 4; ++k)
            for (int j = 0; j < 8; ++j) {
                size_t idx = (q * 4 + k) * 8 + j;
                acc[k][j] = fmaf(a[idx], b[idx], acc[k][j]);
            }
    for (size_t v = quads * 4, k = 0; v < vecs; ++v, ++k)
        for (int j = 0; j < 8; ++j) acc[k][j] = fmaf(a[v * 8 + j], b[v * 8 + j], acc[k][j]);
    float s[8];
    for (int j = 0; j < 8; ++j) s[j] = (acc[0][j] + acc[1][j]) + (acc[2][j] + acc[3][j]);
    return reduce8(s);
}

/* attention_one.rs:103-112: vector exp over whole vectors and the padded tail. */
static void softmax_vec(float *s, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; ++i) max = s[i] > max ? s[i] : max;
    const size_t full = n / 8 * 8;
    float sum[8] = {0};
    for (size_t i = 0; i < full; i += 8)
        for (int j = 0; j < 8; ++j) {
            s[i + j] = or_exp(s[i + j] - max);
            sum[j] = sum[j] + s[i + j];
        }
    float tail = 0.0f;
    for (size_t i = full; i < n; ++i) {
        s[i] = or_exp(s[i] - max);
        tail += s[i];
    }
    const float total = reduce8(sum) + tail;
    for (size_t i = 0; i < n; ++i) s[i] = s[i] / total;
}

void or_attention(const float *queries, const float *keys, const float *values, float *out, size_t heads,
                  size_t kv_heads, size_t head_dim, size_t start, size_t tokens) {
    const size_t group = heads / kv_heads, kv_dim = kv_heads * head_dim, q_dim = heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const int vectorizable = head_dim % 8 == 0 && (tokens == 1 || 8 % group == 0);
    if (tokens == 1 && vectorizable) { /* AttendOne */
        const size_t positions = start + 1;
        float *scores = (float *)malloc(heads * positions * sizeof(float));
        for (size_t p = 0; p < positions; ++p)
            for (size_t h = 0; h < heads; ++h)
                scores[h * positions + p] =
                    dot4acc(queries + h * head_dim, keys + p * kv_dim + (h / group) * head_dim, head_dim) * scale;
        for (size_t h = 0; h < heads; ++h) softmax_vec(scores + h * positions, positions);
        memset(out, 0, q_dim * sizeof(float));
        for (size_t p = 0; p < positions; ++p)
            for (size_t h = 0; h < heads; ++h) {
                const float w = scores[h * positions + p];
                const float *v = values + p * kv_dim + (h / group) * head_dim;
                for (size_t d = 0; d < head_dim; ++d) out[h * head_dim + d] = fmaf(w, v[d], out[h * head_dim + d]);
            }
        free(scores);
        return;
    }
    /* attend_scalar (attention.rs:139-173) */
    float *scores = (float *)malloc((start + tokens) * sizeof(float));
    for (size_t t = 0; t < tokens; ++t) {
        const size_t visible = start + t + 1;
        for (size_t h = 0; h < heads; ++h) {
            const float *q = queries + t * q_dim + h * head_dim;
            for (size_t p = 0; p < visible; ++p)
                scores[p] = or_dot(q, keys + p * kv_dim + (h / group) * head_dim, head_dim) * scale;
            or_softmax(scores, visible);
            float *o = out + t * q_dim + h * head_dim;
            for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
            for (size_t p = 0; p < visible; ++p) {
                const float *v = values + p * kv_dim + (h / group) * head_dim;
                for (size_t d = 0; d < head_dim; ++d) o[d] += scores[p] * v[d];
            }
        }
    }
    free(scores);
}

/* cuda/tests/attention_reference/mod.rs:1-49 */
void or_attention_f64(const float *queries, const float *keys, const float *values, float *out, size_t heads,
                      size_t kv_heads, size_t head_dim, size_t start, size_t tokens) {
    const size_t group = heads / kv_heads, kv_dim = kv_heads * head_dim, q_dim = heads * head_dim;
    double *scores = (double *)malloc((start + tokens) * sizeof(double));
    for (size_t t = 0; t < tokens; ++t) {
        const size_t visible = start + t + 1;
        for (size_t h = 0; h < heads; ++h) {
            const float *q = queries + t * q_dim + h * head_dim;
            const size_t kvh = h / group;
            double max = -INFINITY;
            for (size_t p = 0; p < visible; ++p) {
                double dot = 0.0;
                for (size_t d = 0; d < head_dim; ++d) dot += (double)(q[d] * keys[p * kv_dim + kvh * head_dim + d]);
                scores[p] = dot / sqrt((double)head_dim);
                if (scores[p] > max) max = scores[p];
            }
            double total = 0.0;
            for (size_t p = 0; p < visible; ++p) {
                scores[p] = exp(scores[p] - max);
                total += scores[p];
            }
            for (size_t d = 0; d < head_dim; ++d) {
                double acc = 0.0;
                for (size_t p = 0; p < visible; ++p) acc += scores[p] * (double)values[p * kv_dim + kvh * head_dim + d];
                out[t * q_dim + h * head_dim + d] = (float)(acc / total);
            }
        }
    }
    free(scores);
}

/* sampler/src/lib.rs:40-48: f32::total_cmp, strictly greater replaces, so the lowest index wins ties. */
static inline int32_t total_key(float v) {
    int32_t b = (int32_t)f32_bits(v);
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}
uint32_t or_argmax(const float *values, size_t n) {
    uint32_t best = 0;
    int32_t top = total_key(values[0]);
    for (size_t i = 1; i < n; ++i) {
        int32_t k = total_key(values[i]);
        if (k > top) {
            top = k;
            best = (uint32_t)i;
        }
    }
    return best;
}

/* ---- synthetic weights ---- */
static inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

uint16_t or_synth_bf16(uint64_t seed, uint64_t stream, uint64_t index, double std_dev) {
    const uint64_t base = splitmix64(seed ^ splitmix64(stream + 0x632BE59BD9B4E019ull));
    int64_t sum = 0;
    for (int k = 0; k < 3; ++k) {
        uint64_t r = splitmix64(base + 3 * index + (uint64_t)k);
        sum += (int64_t)(r & 0xffff) + (int64_t)((r >> 16) & 0xffff) + (int64_t)((r >> 32) & 0xffff) +
               (int64_t)(r >> 48);
    }
    /* twelve uniforms (r + 1/2) / 2^16 summed, minus 6: (sum + 6 - 6 * 2^16) / 2^16 */
    const int64_t centred = sum + 6 - 6 * 65536;
    const double value = (double)centred * (std_dev / 65536.0);
    return or_f32_to_bf16((float)value);
}

void or_synth_fill(uint64_t seed, uint64_t stream, double std_dev, uint16_t *out, size_t count) {
    or_synth_fill_at(seed, stream, std_dev, 0, out, count);
}

void or_synth_fill_at(uint64_t seed, uint64_t stream, double std_dev, uint64_t start, uint16_t *out, size_t count) {
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (long i = 0; i < (long)count; ++i) out[i] = or_synth_bf16(seed, stream, start + (uint64_t)i, std_dev);
}

/* ---- Qwen3 forward: model/src/qwen3/model.rs:81-131, layer.rs:39-105, mlp.rs:22-37 ---- */
static void matmul(const or_matrix *m, const float *x, size_t tokens, float *out) {
    if (m->bits == 0) {
        dense_matmul(m->dense, x, out, m->rows, m->cols, tokens);
    } else if (tokens == 1 && m->bits == 8) {
        or_q8_gemv(m->codes, m->scales, x, out, m->rows, m->cols, m->group);
    } else {
        or_matmul_dot(m->codes, m->scales, x, out, m->rows, m->cols, m->bits, m->group, tokens);
    }
}

static void embed_row(const or_matrix *m, uint32_t id, float *out) {
    if (m->bits == 0) memcpy(out, m->dense + (size_t)id * m->cols, m->cols * sizeof(float));
    else or_dequantize_row(m->codes, m->scales, m->cols, m->bits, m->group, id, out);
}

int or_qwen3_forward(or_qwen3 *M, const uint32_t *tokens, size_t count, float *logits) {
    if (count == 0 || M->len + count > M->capacity) return 1;
    for (size_t t = 0; t < count; ++t)
        if (tokens[t] >= M->vocab) return 2;
    const size_t H = M->hidden, qd = M->heads * M->head_dim, kvd = M->kv_heads * M->head_dim, F = M->ffn;
    const size_t start = M->len;
    float *hidden = (float *)malloc(count * H * sizeof(float));
    float *normed = (float *)malloc(count * H * sizeof(float));
    float *q = (float *)malloc(count * qd * sizeof(float));
    float *k = (float *)malloc(count * kvd * sizeof(float));
    float *v = (float *)malloc(count * kvd * sizeof(float));
    float *ctx = (float *)malloc(count * qd * sizeof(float));
    float *att = (float *)malloc(count * H * sizeof(float));
    float *gate = (float *)malloc(count * F * sizeof(float));
    float *up = (float *)malloc(count * F * sizeof(float));
    for (size_t t = 0; t < count; ++t) embed_row(&M->embed, tokens[t], hidden + t * H);
    for (size_t l = 0; l < M->layers; ++l) {
        const or_layer *L = &M->layer[l];
        memcpy(normed, hidden, count * H * sizeof(float));
        or_rms_norm_rows(normed, count * H, L->input_norm, H, M->eps);
        matmul(&L->q, normed, count, q);
        matmul(&L->k, normed, count, k);
        matmul(&L->v, normed, count, v);
        or_rms_norm_rows(q, count * qd, L->q_norm, M->head_dim, M->eps);
        or_rms_norm_rows(k, count * kvd, L->k_norm, M->head_dim, M->eps);
        or_rope_tokens(q, count * qd, qd, M->head_dim, start, M->theta);
        or_rope_tokens(k, count * kvd, kvd, M->head_dim, start, M->theta);
        float *keys = M->keys + l * M->capacity * kvd, *vals = M->values + l * M->capacity * kvd;
        for (size_t i = 0; i < count * kvd; ++i) {
            float kk = k[i], vv = v[i];
            if (M->kv_f16) {
                kk = or_f16_to_f32(or_f32_to_f16_sat(kk));
                vv = or_f16_to_f32(or_f32_to_f16_sat(vv));
            }
            keys[start * kvd + i] = kk;
            vals[start * kvd + i] = vv;
        }
        or_attention(q, keys, vals, ctx, M->heads, M->kv_heads, M->head_dim, start, count);
        matmul(&L->o, ctx, count, att);
        for (size_t i = 0; i < count * H; ++i) hidden[i] += att[i];
        memcpy(normed, hidden, count * H * sizeof(float));
        or_rms_norm_rows(normed, count * H, L->post_norm, H, M->eps);
        matmul(&L->gate, normed, count, gate);
        matmul(&L->up, normed, count, up);
        or_silu_mul(gate, up, count * F);
        matmul(&L->down, gate, count, att);
        for (size_t i = 0; i < count * H; ++i) hidden[i] += att[i];
    }
    float *last = normed;
    memcpy(last, hidden + (count - 1) * H, H * sizeof(float));
    or_rms_norm_rows(last, H, M->final_norm, H, M->eps);
    const or_matrix *head = M->lm_head.rows ? &M->lm_head : &M->embed;
    matmul(head, last, 1, logits);
    M->len += count;
    free(hidden);
    free(normed);
    free(q);
    free(k);
    free(v);
    free(ctx);
    free(att);
    free(gate);
    free(up);
    return 0;
}
