// Quantized matrices on the device (crates/cuda/src/quant.rs + quant.cu of the reference, redesigned for gfx950):
// upload and device layout, the general VALU product for layouts the matrix-core product does not take, the int8
// embedding lookup, the on-device synthetic weights + quantizer, and the C ABI entry points. The matrix-core
// product itself is in gemv.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "gemm.hpp"
#include "gemv.hpp"

namespace marin {


// ---------------------------------------------------------------------------------------------------------------
// General product for any group (a multiple of 32) and int4: one wave per row, a lane takes 8 consecutive columns per
// 512-column step (always inside one group), up to 8 tokens per block row (grid.y tiles the tokens). The row's
// partial sums are f32 FMAs of the dequantized codes, scaled once per 8 columns as in quant.cu's matvec_row.
template <int BITS, typename ST>
__global__ __launch_bounds__(256) void gemv_valu(const uint8_t *__restrict__ codes, const ST *__restrict__ scales,
                                                 const float *__restrict__ x, float *__restrict__ y, int tokens,
                                                 int rows, int cols, int group) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int t0 = blockIdx.y * 8;
    const int nt = min(8, tokens - t0);
    const int groups = cols / group;
    const size_t row_bytes = BITS == 8 ? (size_t)cols : (size_t)(cols + 1) / 2;
    const uint8_t *crow = codes + (size_t)row * row_bytes;
    const ST *srow = scales + (size_t)(row / 16) * groups * 16 + (row % 16);
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int c = lane * 8; c < cols; c += 512) {
        float wv[8];
        if constexpr (BITS == 8) {
            const uint2 u = *reinterpret_cast<const uint2 *>(crow + c);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                wv[i] = (float)(int8_t)(u.x >> (8 * i));
                wv[i + 4] = (float)(int8_t)(u.y >> (8 * i));
            }
        } else {
            // device int4 layout: byte e of each 4-byte word holds column e (low nibble) and column 4 + e (high)
            const uint32_t u = *reinterpret_cast<const uint32_t *>(crow + c / 2);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                wv[i] = (float)((int)((u >> (8 * i)) & 15u) - 8);
                wv[i + 4] = (float)((int)((u >> (8 * i + 4)) & 15u) - 8);
            }
        }
        float s;
        if constexpr (sizeof(ST) == 4) s = srow[(c / group) * 16];
        else s = __uint_as_float((unsigned)srow[(c / group) * 16] << 16);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j >= nt) break;
            const float *xr = x + (size_t)(t0 + j) * cols + c;
            const float4 xa = *reinterpret_cast<const float4 *>(xr);
            const float4 xb = *reinterpret_cast<const float4 *>(xr + 4);
            const float d = wv[0] * xa.x + wv[1] * xa.y + wv[2] * xa.z + wv[3] * xa.w + wv[4] * xb.x + wv[5] * xb.y +
                            wv[6] * xb.z + wv[7] * xb.w;
            acc[j] += s * d;
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        float v = acc[j];
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0 && j < nt) y[(size_t)(t0 + j) * rows + row] = v;
    }
}

void launch_gemv_valu(marin_gpu *g, const marin_quant_matrix *w, const float *x, size_t tokens, float *y) {
    if (!tokens) return;
    dim3 grid((unsigned)((w->rows + 3) / 4), (unsigned)((tokens + 7) / 8));
#define MARIN_VALU(B, S)                                                                                   \
    gemv_valu<B, S><<<grid, dim3(256), 0, g->stream>>>(w->codes, (const S *)w->scales, x, y, (int)tokens, \
                                                       (int)w->rows, (int)w->cols, (int)w->group)
    if (w->bits == 8) {
        if (w->bf16_scales) MARIN_VALU(8, uint16_t);
        else MARIN_VALU(8, float);
    } else {
        if (w->bf16_scales) MARIN_VALU(4, uint16_t);
        else MARIN_VALU(4, float);
    }
#undef MARIN_VALU
    g->launched();
}

// ---------------------------------------------------------------------------------------------------------------
// out[t][i] = code * scale of row ids[t] (quant.cu:209-214): one block per token.
template <typename ST>
__global__ void embed_q8_kernel(const uint8_t *__restrict__ codes, const ST *__restrict__ scales,
                                const uint32_t *__restrict__ ids, float *__restrict__ out, int cols, int group,
                                bool windowed) {
    const size_t row = ids[blockIdx.x];
    const int groups = cols / group;
    const ST *srow = scales + (row / 16) * (size_t)groups * 16 + (row % 16);
    for (int i = threadIdx.x; i < cols; i += blockDim.x) {
        float s;
        if constexpr (sizeof(ST) == 4) s = srow[(i / group) * 16];
        else s = __uint_as_float((unsigned)srow[(i / group) * 16] << 16);
        out[(size_t)blockIdx.x * cols + i] = (float)(int8_t)codes[code_offset(row, i, cols, windowed, 16)] * s;
    }
}

void launch_embed_q8(marin_gpu *g, const marin_quant_matrix *w, const uint32_t *ids, size_t n, float *out) {
    if (!n) return;
    if (w->bf16_scales)
        embed_q8_kernel<uint16_t><<<dim3((unsigned)n), dim3(256), 0, g->stream>>>(
            w->codes, (const uint16_t *)w->scales, ids, out, (int)w->cols, (int)w->group, w->windowed);
    else
        embed_q8_kernel<float><<<dim3((unsigned)n), dim3(256), 0, g->stream>>>(
            w->codes, (const float *)w->scales, ids, out, (int)w->cols, (int)w->group, w->windowed);
    g->launched();
}

// ---------------------------------------------------------------------------------------------------------------
// Synthetic weights + the reference quantizer (tensor/src/quant.rs:181-234) on the device. The generator is the one
// oracle/marin_oracle.c restates: twelve 16-bit uniforms from three splitmix64 draws, summed in integers, one IEEE
// double multiply, rounded to f32 and then to bf16 (nearest even). One wave per (row, group).
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__device__ __forceinline__ float synth_value(uint64_t base, uint64_t index, double step) {
    int64_t sum = 0;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const uint64_t r = splitmix64(base + 3 * index + (uint64_t)k);
        sum += (int64_t)(r & 0xffff) + (int64_t)((r >> 16) & 0xffff) + (int64_t)((r >> 32) & 0xffff) +
               (int64_t)(r >> 48);
    }
    const double value = __dmul_rn((double)(sum + 6 - 6 * 65536), step);
    const float f = __double2float_rn(value);
    unsigned u = __float_as_uint(f);
    u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
    return __uint_as_float(u);
}

template <int PER_LANE>
__global__ __launch_bounds__(256) void synth_quantize_kernel(uint8_t *__restrict__ codes, float *__restrict__ scales,
                                                             uint64_t base, double step, int src_rows, int cols,
                                                             int group, int dst_row0, int dst_row_step) {
    const int lane = threadIdx.x & 63;
    const int groups = cols / group;
    const long unit = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (unit >= (long)src_rows * groups) return;
    const int r = (int)(unit / groups), gi = (int)(unit % groups);
    float v[PER_LANE];
    float largest = 0.0f;
#pragma unroll
    for (int k = 0; k < PER_LANE; ++k) {
        const int i = lane + 64 * k;
        v[k] = i < group ? synth_value(base, (uint64_t)r * cols + (uint64_t)gi * group + i, step) : 0.0f;
        largest = fmaxf(largest, fabsf(v[k]));
    }
    for (int o = 32; o > 0; o >>= 1) largest = fmaxf(largest, __shfl_xor(largest, o));
    const float scale = largest / 127.0f;
    const size_t dst = (size_t)dst_row0 + (size_t)r * dst_row_step;
#pragma unroll
    for (int k = 0; k < PER_LANE; ++k) {
        const int i = lane + 64 * k;
        if (i >= group) break;
        int code = 0;
        if (scale > 0.0f) {
            const float qf = roundf(v[k] / scale);
            code = (int)fminf(fmaxf(qf, -127.0f), 127.0f);
        }
        codes[code_offset(dst, (size_t)gi * group + i, cols, true, 16)] = (uint8_t)(int8_t)code;
    }
    if (lane == 0) scales[(dst / 16) * (size_t)groups * 16 + (size_t)gi * 16 + (dst % 16)] = scale;
}

void launch_synth_quantize(marin_gpu *g, marin_quant_matrix *w, uint64_t seed, uint64_t stream, double std_dev,
                           size_t src_rows, size_t dst_row0, size_t dst_row_step) {
    if (w->bits != 8 || w->bf16_scales) throw Error(MARIN_UNSUPPORTED, "synthetic matrices are int8 with f32 scales");
    if (w->group > 256) unsupported("synthetic group size", 256, w->group);
    if (!w->windowed) unsupported("synthetic matrix layout (group and columns multiples of 64)", 64, w->group);
    // Same mixing as or_synth_bf16: base = splitmix64(seed ^ splitmix64(stream + constant)).
    auto mix = [](uint64_t x) {
        x += 0x9E3779B97F4A7C15ull;
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        return x ^ (x >> 31);
    };
    const uint64_t base = mix(seed ^ mix(stream + 0x632BE59BD9B4E019ull));
    const double step = std_dev / 65536.0;
    const size_t units = src_rows * w->groups();
    dim3 grid((unsigned)((units + 3) / 4));
    if (w->group <= 64)
        synth_quantize_kernel<1><<<grid, dim3(256), 0, g->stream>>>(w->codes, (float *)w->scales, base, step,
                                                                    (int)src_rows, (int)w->cols, (int)w->group,
                                                                    (int)dst_row0, (int)dst_row_step);
    else if (w->group <= 128)
        synth_quantize_kernel<2><<<grid, dim3(256), 0, g->stream>>>(w->codes, (float *)w->scales, base, step,
                                                                    (int)src_rows, (int)w->cols, (int)w->group,
                                                                    (int)dst_row0, (int)dst_row_step);
    else
        synth_quantize_kernel<4><<<grid, dim3(256), 0, g->stream>>>(w->codes, (float *)w->scales, base, step,
                                                                    (int)src_rows, (int)w->cols, (int)w->group,
                                                                    (int)dst_row0, (int)dst_row_step);
    g->launched();
}

// ---------------------------------------------------------------------------------------------------------------
marin_quant_matrix *new_quant_matrix(marin_gpu *g, size_t rows, size_t cols, int bits, size_t group, bool bf16) {
    auto *m = new marin_quant_matrix();
    m->gpu = g;
    m->rows = rows;
    m->cols = cols;
    m->bits = bits;
    m->group = group;
    m->bf16_scales = bf16;
    m->rows_padded = (rows + ROW_PAD - 1) / ROW_PAD * ROW_PAD;
    m->windowed = group % 64 == 0 && cols % 64 == 0;
    try {
        m->codes = (uint8_t *)g->alloc(mul(m->rows_padded, m->row_bytes(), "quantized codes") + 16, true);
        m->scales = g->alloc(mul(mul(m->rows_padded, m->groups(), "quantization scales"), bf16 ? 2 : 4,
                                 "quantization scales"),
                             true);
    } catch (...) {
        free_quant_matrix(m);
        throw;
    }
    return m;
}

void free_quant_matrix(marin_quant_matrix *m) {
    if (!m) return;
    (void)hipStreamSynchronize(m->gpu->stream);
    m->gpu->release(m->codes);
    m->gpu->release(m->scales);
    delete m;
}

// tensor::Quantized keeps int4 as byte j = column 2j (low nibble) | column 2j + 1 (high). The device keeps each
// 8-column group as 4 bytes whose low nibbles are columns 0-3 and high nibbles columns 4-7, so two masks turn a
// word into four bytes of consecutive columns.
static void repack_int4(const uint8_t *src, uint8_t *dst, size_t bytes) {
    for (size_t w = 0; w + 4 <= bytes; w += 4) {
        uint8_t nib[8];
        for (int j = 0; j < 4; ++j) {
            nib[2 * j] = src[w + j] & 15u;
            nib[2 * j + 1] = src[w + j] >> 4;
        }
        for (int e = 0; e < 4; ++e) dst[w + e] = (uint8_t)(nib[e] | (nib[4 + e] << 4));
    }
}

void upload_rows(marin_quant_matrix *m, const uint8_t *codes_in, const void *scales, size_t src_rows, size_t dst_row0,
                 size_t dst_row_step) {
    marin_gpu *g = m->gpu;
    const size_t rb = m->row_bytes(), groups = m->groups(), es = m->bf16_scales ? 2 : 4;
    std::vector<uint8_t> repacked;
    const uint8_t *codes = codes_in;
    if (m->bits == 4) {
        repacked.resize(src_rows * rb);
        repack_int4(codes_in, repacked.data(), repacked.size());
        codes = repacked.data();
    }
    // Codes: rebuild the 16-row tiles the rows touch on the host (rows of a tile are contiguous in both layouts),
    // then one upload.
    const size_t last_row = dst_row0 + (src_rows - 1) * dst_row_step;
    const size_t ct0 = dst_row0 / 16, ct1 = last_row / 16 + 1;
    const size_t tile_bytes = 16 * rb, cb = code_chunk(m->bits);
    std::vector<uint8_t> code_tiles((ct1 - ct0) * tile_bytes);
    const bool whole = dst_row_step == 1 && dst_row0 % 16 == 0 && (src_rows % 16 == 0 || last_row + 1 >= m->rows);
    if (!whole) g->download(code_tiles.data(), m->codes + ct0 * tile_bytes, code_tiles.size());
    for (size_t r = 0; r < src_rows; ++r) {
        const size_t dst = dst_row0 + r * dst_row_step;
        const uint8_t *src = codes + r * rb;
        uint8_t *tile = code_tiles.data() + (dst / 16 - ct0) * tile_bytes;
        if (!m->windowed) {
            std::memcpy(tile + (dst % 16) * rb, src, rb);
        } else {
            for (size_t b0 = 0; b0 < rb; b0 += cb)
                std::memcpy(tile + code_offset(dst % 16, b0, rb, true, cb), src + b0, cb);
        }
    }
    g->upload(m->codes + ct0 * tile_bytes, code_tiles.data(), code_tiles.size());
    // Scales: rebuild the tiles the rows touch on the host, then upload them.
    const size_t last = dst_row0 + (src_rows - 1) * dst_row_step;
    const size_t t0 = dst_row0 / 16, t1 = last / 16 + 1;
    std::vector<uint8_t> tiles((t1 - t0) * groups * 16 * es);
    g->download(tiles.data(), (uint8_t *)m->scales + t0 * groups * 16 * es, tiles.size());
    for (size_t r = 0; r < src_rows; ++r) {
        const size_t dst = dst_row0 + r * dst_row_step;
        for (size_t gi = 0; gi < groups; ++gi)
            std::memcpy(&tiles[(((dst / 16) - t0) * groups * 16 + gi * 16 + dst % 16) * es],
                        (const uint8_t *)scales + (r * groups + gi) * es, es);
    }
    g->upload((uint8_t *)m->scales + t0 * groups * 16 * es, tiles.data(), tiles.size());
}

void matmul_f32(marin_gpu *g, const marin_quant_matrix *w, const float *x, size_t tokens, float *y, bool precise) {
    (void)precise;  // the matrix-core product keeps 30 bits of every activation: f32-grade at every token count
    if (!tokens) return;
    if (!gemv_supported(w)) {
        launch_gemv_valu(g, w, x, tokens, y);
        return;
    }
    GemvIn in;
    in.mode = IN_F32;
    in.x = x;
    in.x_stride = w->cols;
    GemvOut out;
    out.mode = OUT_F32;
    out.y = y;
    out.y_stride = w->rows;
    launch_product(g, w, in, out, tokens);
}

}  // namespace marin

using namespace marin;

static void check_quantized(size_t rows, size_t cols, int bits, size_t group, size_t codes_len, size_t scales_len) {
    if (bits != 8 && bits != 4) unsupported("quantized width in bits", 8, (size_t)bits);
    if (group == 0 || group % 32 != 0 || cols % group != 0) shape("quantization group", group, cols);
    const size_t rb = bits == 8 ? cols : (cols + 1) / 2;
    const size_t codes = mul(rows, rb, "quantized codes");
    const size_t scales = mul(rows, cols / group, "quantization scales");
    if (codes_len != codes) shape("quantized codes", codes, codes_len);
    if (scales_len != scales) shape("quantization scales", scales, scales_len);
}

extern "C" {

marin_status marin_quantized_synthetic(marin_gpu *g, size_t rows, size_t cols, size_t group, uint64_t seed,
                                       uint64_t stream, double std_dev, marin_quant_matrix **out) {
    return guard([&] {
        if (group == 0 || group % 32 != 0 || cols % group != 0) shape("quantization group", group, cols);
        if (!rows) shape("rows", 1, 0);
        marin_quant_matrix *m = new_quant_matrix(g, rows, cols, 8, group, false);
        try {
            launch_synth_quantize(g, m, seed, stream, std_dev, rows, 0, 1);
        } catch (...) {
            free_quant_matrix(m);
            throw;
        }
        *out = m;
    });
}

marin_status marin_upload_quantized(marin_gpu *g, size_t rows, size_t cols, int bits, size_t group,
                                    const uint8_t *codes, size_t codes_len, const float *scales, size_t scales_len,
                                    marin_quant_matrix **out) {
    return guard([&] {
        check_quantized(rows, cols, bits, group, codes_len, scales_len);
        marin_quant_matrix *m = new_quant_matrix(g, rows, cols, bits, group, false);
        try {
            if (rows) upload_rows(m, codes, scales, rows, 0, 1);
        } catch (...) {
            free_quant_matrix(m);
            throw;
        }
        *out = m;
    });
}

marin_status marin_upload_quantized_bf16_scales(marin_gpu *g, size_t rows, size_t cols, int bits, size_t group,
                                                const uint8_t *codes, size_t codes_len, const uint16_t *scales,
                                                size_t scales_len, marin_quant_matrix **out) {
    return guard([&] {
        check_quantized(rows, cols, bits, group, codes_len, scales_len);
        marin_quant_matrix *m = new_quant_matrix(g, rows, cols, bits, group, true);
        try {
            if (rows) upload_rows(m, codes, scales, rows, 0, 1);
        } catch (...) {
            free_quant_matrix(m);
            throw;
        }
        *out = m;
    });
}

void marin_quant_matrix_free(marin_quant_matrix *m) { free_quant_matrix(m); }

void marin_quant_matrix_shape(const marin_quant_matrix *m, size_t *rows, size_t *cols, int *bits, size_t *group) {
    if (rows) *rows = m->rows;
    if (cols) *cols = m->cols;
    if (bits) *bits = m->bits;
    if (group) *group = m->group;
}

size_t marin_quant_matrix_bytes(const marin_quant_matrix *m) {
    return m->rows * m->row_bytes() + m->rows * m->groups() * (m->bf16_scales ? 2 : 4);
}

marin_status marin_embed_quant(marin_gpu *g, const marin_quant_matrix *table, const uint32_t *ids, size_t n,
                               marin_tokens *scratch, marin_buffer *out) {
    return guard([&] {
        if (table->bits != 8) unsupported("quantized embedding width in bits", 8, 4);
        check_len("embed output", mul(n, table->cols, "embed output"), out->len);
        if (out->dtype != MARIN_F32) shape("embed output element size", 4, dtype_bytes(out->dtype));
        for (size_t i = 0; i < n; ++i)
            if (ids[i] >= table->rows) shape("token id", table->rows, ids[i]);
        if (n == 0) return;
        if (n > scratch->capacity) shape("embed token capacity", scratch->capacity, n);
        void *staged = g->stage(ids, n * 4);
        HIP_CHECK(hipMemcpyAsync(scratch->data, staged, n * 4, hipMemcpyHostToDevice, g->stream));
        g->traffic.uploads++;
        g->traffic.upload_bytes += n * 4;
        launch_embed_q8(g, table, scratch->data, n, (float *)out->data);
    });
}

static void check_matmul(const marin_quant_matrix *w, const marin_buffer *x, size_t tokens, const marin_buffer *out,
                         marin_dtype dt) {
    if (x->dtype != dt) shape("matmul input element size", dtype_bytes(dt), dtype_bytes(x->dtype));
    if (out->dtype != dt) shape("matmul output element size", dtype_bytes(dt), dtype_bytes(out->dtype));
    check_len("matmul input", mul(tokens, w->cols, "matmul input"), x->len);
    check_len("matmul output", mul(tokens, w->rows, "matmul output"), out->len);
}

marin_status marin_matmul_quant(marin_gpu *g, const marin_quant_matrix *w, const marin_buffer *x, size_t tokens,
                                marin_buffer *out) {
    return guard([&] {
        check_matmul(w, x, tokens, out, MARIN_F32);
        if (!tokens || !w->rows || !w->cols) return;
        matmul_f32(g, w, (const float *)x->data, tokens, (float *)out->data, false);
    });
}

marin_status marin_matmul_quant_precise(marin_gpu *g, const marin_quant_matrix *w, const marin_buffer *x,
                                        size_t tokens, marin_buffer *out) {
    return guard([&] {
        check_matmul(w, x, tokens, out, MARIN_F32);
        if (!tokens || !w->rows || !w->cols) return;
        matmul_f32(g, w, (const float *)x->data, tokens, (float *)out->data, true);
    });
}

marin_status marin_matmul_quant_bf16(marin_gpu *g, const marin_quant_matrix *w, const marin_buffer *x, size_t tokens,
                                     marin_buffer *out) {
    return guard([&] {
        check_matmul(w, x, tokens, out, MARIN_BF16);
        if (!tokens || !w->rows || !w->cols) return;
        if (!gemv_supported(w)) unsupported("bf16 product layout (group and cols multiples of 64)", 64, w->group);
        GemvIn in;
        in.mode = IN_BF16;
        in.x = x->data;
        in.x_stride = w->cols;
        GemvOut o;
        o.mode = OUT_BF16;
        o.y = out->data;
        o.y_stride = w->rows;
        launch_product(g, w, in, o, tokens);
    });
}

// Measurement (config 1): `reps` bf16-in, bf16-out products cycling through `n` same-shaped matrices (so the
// weights stream from HBM, not the last-level cache), captured into one HIP graph and replayed between two events on
// the stream: mean seconds per product.
marin_status marin_time_matmul_bf16(marin_gpu *g, const marin_quant_matrix *const *mats, size_t n,
                                    const marin_buffer *x, size_t tokens, marin_buffer *out, int reps,
                                    double *seconds) {
    return guard([&] {
        if (!n || reps < 1 || !tokens) shape("timed products", 1, 0);
        for (size_t i = 0; i < n; ++i) {
            check_matmul(mats[i], x, tokens, out, MARIN_BF16);
            if (mats[i]->rows != mats[0]->rows || mats[i]->cols != mats[0]->cols) shape("timed matrix rows", mats[0]->rows, mats[i]->rows);
            if (!gemv_supported(mats[i])) unsupported("bf16 product layout (group and cols multiples of 64)", 64, mats[i]->group);
        }
        auto one = [&](const marin_quant_matrix *w) {
            GemvIn in;
            in.mode = IN_BF16;
            in.x = x->data;
            in.x_stride = w->cols;
            GemvOut o;
            o.mode = OUT_BF16;
            o.y = out->data;
            o.y_stride = w->rows;
            launch_product(g, w, in, o, tokens);
        };
        one(mats[0]);  // grows the workspace outside the capture
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        HIP_CHECK(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal));
        try {
            for (int r = 0; r < reps; ++r) one(mats[r % n]);
        } catch (...) {
            hipGraph_t junk = nullptr;
            (void)hipStreamEndCapture(g->stream, &junk);
            if (junk) (void)hipGraphDestroy(junk);
            throw;
        }
        HIP_CHECK(hipStreamEndCapture(g->stream, &graph));
        hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        hip_check(e, "hipGraphInstantiate");
        hipEvent_t a = g->next_event(), b = g->next_event();
        float ms = 0.0f;
        e = hipGraphLaunch(exec, g->stream);  // warm-up
        if (e == hipSuccess) e = hipEventRecord(a, g->stream);
        if (e == hipSuccess) e = hipGraphLaunch(exec, g->stream);
        if (e == hipSuccess) e = hipEventRecord(b, g->stream);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        (void)hipGraphExecDestroy(exec);
        hip_check(e, "timed product graph");
        *seconds = ms * 1e-3 / reps;
    });
}

}  // extern "C"
