// Quantized linear layers on CDNA4 (crates/cuda/src/quant.rs + quant.cu of the reference, redesigned for gfx950).
//
// The hot product streams int8 codes with one 16-byte load per lane, turns them into f16 exactly in registers
// (0x6400 | (code ^ 0x80) is the f16 1024 + code + 128), and multiplies them on the matrix cores
// (v_mfma_f32_16x16x32_f16) against the activations split into f16 parts: x * 2^s = hi + lo (+ mid), each part one
// B column. f16 holds every code exactly and the parts carry 22 (33) bits of each activation, so the products are
// f32-grade while the conversion costs about one VALU op per weight instead of a convert and an FMA. Partial sums are
// f32 in the MFMA accumulators; each 64-column window is scaled by its group's scale once.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "quant.hpp"

namespace marin {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

size_t split_bytes(size_t tokens, size_t cols) {
    size_t data = tokens * 3 * cols * sizeof(_Float16);  // room for three parts
    data = (data + 255) & ~size_t(255);
    return data + tokens * sizeof(float) + 256;
}

SplitView split_view(void *base, size_t tokens, size_t cols) {
    SplitView v;
    v.data = (_Float16 *)base;
    size_t data = tokens * 3 * cols * sizeof(_Float16);
    data = (data + 255) & ~size_t(255);
    v.inv = (float *)((char *)base + data);
    v.cols = cols;
    v.tokens = tokens;
    return v;
}

// ---------------------------------------------------------------------------------------------------------------
// Activation split: one block per token. With scale_tokens the token is first scaled by the power of two that puts
// its largest magnitude in [2^14, 2^15), which keeps every part inside f16's normal range; inv undoes it exactly.
// Part p of token t lives at data[(t * parts + p) * cols].
template <int PARTS, typename In>
__global__ __launch_bounds__(256) void split_kernel(const In *__restrict__ x, size_t cols, _Float16 *__restrict__ data,
                                                     float *__restrict__ inv, int scale_tokens) {
    const size_t t = blockIdx.x;
    const In *row = x + t * cols;
    __shared__ float red[4];
    float scale = 1.0f, undo = 1.0f;
    if (scale_tokens) {
        float m = 0.0f;
        for (size_t i = threadIdx.x; i < cols; i += 256) {
            float v;
            if constexpr (sizeof(In) == 4) v = row[i];
            else v = __uint_as_float((unsigned)row[i] << 16);
            m = fmaxf(m, fabsf(v));
        }
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        if (m > 0.0f && m < INFINITY) {
            int e;
            (void)frexpf(m, &e);  // m = f * 2^e, f in [0.5, 1)
            int s = 15 - e;
            s = s > 100 ? 100 : (s < -100 ? -100 : s);
            scale = ldexpf(1.0f, s);
            undo = ldexpf(1.0f, -s);
        }
    }
    for (size_t i = threadIdx.x; i < cols; i += 256) {
        float v;
        if constexpr (sizeof(In) == 4) v = row[i];
        else v = __uint_as_float((unsigned)row[i] << 16);
        v *= scale;
        _Float16 hi = (_Float16)v;
        float rest = v - (float)hi;
        _Float16 mid = (_Float16)rest;
        data[(t * PARTS + 0) * cols + i] = hi;
        data[(t * PARTS + 1) * cols + i] = mid;
        if constexpr (PARTS == 3) data[(t * PARTS + 2) * cols + i] = (_Float16)(rest - (float)mid);
    }
    if (threadIdx.x == 0) inv[t] = undo;
}

void launch_split_f32(marin_gpu *g, const float *x, size_t tokens, size_t cols, SplitView out, bool scale_tokens) {
    if (!tokens) return;
    split_kernel<2, float><<<dim3((unsigned)tokens), dim3(256), 0, g->stream>>>(x, cols, out.data, out.inv,
                                                                                scale_tokens ? 1 : 0);
    g->launched();
}

static void launch_split3_f32(marin_gpu *g, const float *x, size_t tokens, size_t cols, SplitView out) {
    if (!tokens) return;
    split_kernel<3, float><<<dim3((unsigned)tokens), dim3(256), 0, g->stream>>>(x, cols, out.data, out.inv, 1);
    g->launched();
}

void launch_split_bf16(marin_gpu *g, const uint16_t *x, size_t tokens, size_t cols, SplitView out) {
    if (!tokens) return;
    split_kernel<2, uint16_t><<<dim3((unsigned)tokens), dim3(256), 0, g->stream>>>(x, cols, out.data, out.inv, 1);
    g->launched();
}

// ---------------------------------------------------------------------------------------------------------------
// int8 codes -> f16, exactly: byte b becomes the f16 with bits 0x6400 | (b ^ 0x80), i.e. 1024 + code + 128, and one
// packed subtraction of 1152 leaves the code.
__device__ __forceinline__ half2v pair_f16(uint32_t word, int shift) {
    const uint32_t lo = (word >> shift) & 0xffu, hi = (word >> (shift + 8)) & 0xffu;
    const uint32_t bits = lo | (hi << 16) | 0x64006400u;
    return __builtin_bit_cast(half2v, bits) - (half2v){(_Float16)1152.0f, (_Float16)1152.0f};
}

__device__ __forceinline__ half8 decode8(uint32_t w0, uint32_t w1) {
    w0 ^= 0x80808080u;
    w1 ^= 0x80808080u;
    const half2v a = pair_f16(w0, 0), b = pair_f16(w0, 16), c = pair_f16(w1, 0), d = pair_f16(w1, 16);
    return (half8){a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

template <typename ST>
__device__ __forceinline__ floatx4 load_scale4(const ST *p) {
    if constexpr (sizeof(ST) == 4) {
        return *reinterpret_cast<const floatx4 *>(p);
    } else {
        const uint2 u = *reinterpret_cast<const uint2 *>(p);
        return (floatx4){__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                         __uint_as_float(u.y & 0xffff0000u)};
    }
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

constexpr int WAVES = 4;
constexpr int MAX_COLS = 16;  // B columns of one MFMA

// One block: 16*RT rows (RT tiles of 16) of the matrix, the windows [w0, w1) of 64 columns split into contiguous
// runs across its four waves. Lane l of a wave loads 16 code bytes of row (l % 16) at column 64w + 16(l / 16) and the
// matching 8+8 f16 of every B column c = l % 16 < used; the MFMA's D gives lane l rows 4(l/16)..+3 of column l % 16.
// Grid: x = row blocks, y = column splits (kb). With more than one split, each block leaves its sums in `partials`
// and the last block to arrive at a row block's counter adds them in split order, so results do not depend on
// timing; that block also puts the counter back to zero.
template <int RT, typename ST, int EPI, int PARTS, bool ONE>
__global__ __launch_bounds__(256) void gemv_i8_mfma(const uint8_t *__restrict__ codes, const ST *__restrict__ scales,
                                                   const _Float16 *__restrict__ xs, const float *__restrict__ xinv,
                                                   int tokens_arg, int rows, int rows_padded, int cols, int group,
                                                   int windows_per_split, float *__restrict__ partials,
                                                   unsigned *__restrict__ counters, EpiArgs epi) {
    // ONE: a single token (decode), known at compile time; otherwise up to MAX_GEMV_TOKENS.
    const int tokens = ONE ? 1 : tokens_arg;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, q = lane >> 4;
    const int used = tokens * PARTS;
    const int total_windows = cols >> 6;
    const int splits = gridDim.y;
    const int kw0 = blockIdx.y * windows_per_split;
    const int kw1 = min(total_windows, kw0 + windows_per_split);
    const int span = kw1 > kw0 ? kw1 - kw0 : 0;
    const int per_wave = (span + WAVES - 1) / WAVES;
    const int w0 = kw0 + min(span, wave * per_wave);
    const int w1 = kw0 + min(span, (wave + 1) * per_wave);
    const int groups = cols / group;
    const int tile0 = blockIdx.x * RT;

    floatx4 total[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) total[r] = (floatx4){0.f, 0.f, 0.f, 0.f};

    const uint8_t *arow[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) arow[r] = codes + (size_t)((tile0 + r) * 16 + c) * cols + 16 * q;
    const _Float16 *brow = xs + (size_t)c * cols + 16 * q;
    const bool bcol = c < used;
    const ST *srow[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) srow[r] = scales + (size_t)(tile0 + r) * groups * 16 + 4 * q;

    constexpr int D = 4;  // windows in flight per wave
    int w = w0;
    for (; w + D <= w1; w += D) {
        u32x4 a[D][RT];
        half8 b[D][2];
        floatx4 s[D][RT];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int col = (w + d) * 64;
#pragma unroll
            for (int r = 0; r < RT; ++r) a[d][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(arow[r] + col));
            if (bcol) {
                b[d][0] = *reinterpret_cast<const half8 *>(brow + col);
                b[d][1] = *reinterpret_cast<const half8 *>(brow + col + 8);
            } else {
                b[d][0] = (half8){0, 0, 0, 0, 0, 0, 0, 0};
                b[d][1] = b[d][0];
            }
            const int gi = col / group;
#pragma unroll
            for (int r = 0; r < RT; ++r) s[d][r] = load_scale4(srow[r] + gi * 16);
        }
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                floatx4 acc = (floatx4){0.f, 0.f, 0.f, 0.f};
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(decode8(a[d][r].x, a[d][r].y), b[d][0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(decode8(a[d][r].z, a[d][r].w), b[d][1], acc, 0, 0, 0);
                total[r] += acc * s[d][r];
            }
    }
    for (; w < w1; ++w) {
        const int col = w * 64;
        half8 b0 = (half8){0, 0, 0, 0, 0, 0, 0, 0}, b1 = b0;
        if (bcol) {
            b0 = *reinterpret_cast<const half8 *>(brow + col);
            b1 = *reinterpret_cast<const half8 *>(brow + col + 8);
        }
        const int gi = col / group;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(arow[r] + col));
            const floatx4 s = load_scale4(srow[r] + gi * 16);
            floatx4 acc = (floatx4){0.f, 0.f, 0.f, 0.f};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(decode8(a.x, a.y), b0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(decode8(a.z, a.w), b1, acc, 0, 0, 0);
            total[r] += acc * s;
        }
    }

    // Sum the waves (and the parts of each token) through LDS: red[wave][tile][column][row].
    __shared__ float red[WAVES][RT][MAX_COLS][16];
    __shared__ float vals[RT][MAX_GEMV_TOKENS][16];
    __shared__ bool last;
    if (c < used) {
#pragma unroll
        for (int r = 0; r < RT; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[wave][r][c][4 * q + i] = total[r][i];
    }
    __syncthreads();
    const int outputs = RT * tokens * 16;
    for (int o = threadIdx.x; o < outputs; o += 256) {
        const int r = o / (tokens * 16), t = (o / 16) % tokens, row = o % 16;
        float v = 0.0f;
#pragma unroll
        for (int wv = 0; wv < WAVES; ++wv) {
            float part = 0.0f;
#pragma unroll
            for (int p = 0; p < PARTS; ++p) part += red[wv][r][t * PARTS + p][row];
            v += part;
        }
        vals[r][t][row] = v * xinv[t];
    }
    __syncthreads();
    if (splits > 1) {
        const size_t stride = (size_t)rows_padded;
        for (int o = threadIdx.x; o < outputs; o += 256) {
            const int r = o / (tokens * 16), t = (o / 16) % tokens, row = o % 16;
            partials[((size_t)blockIdx.y * tokens + t) * stride + (tile0 + r) * 16 + row] = vals[r][t][row];
        }
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned prev = atomicAdd(&counters[blockIdx.x], 1u);
            last = prev == (unsigned)(splits - 1);
            if (last) counters[blockIdx.x] = 0u;
        }
        __syncthreads();
        if (!last) return;
        __threadfence();
        for (int o = threadIdx.x; o < outputs; o += 256) {
            const int r = o / (tokens * 16), t = (o / 16) % tokens, row = o % 16;
            float v = 0.0f;
            for (int k = 0; k < splits; ++k)
                v += __builtin_nontemporal_load(&partials[((size_t)k * tokens + t) * stride + (tile0 + r) * 16 + row]);
            vals[r][t][row] = v;
        }
        __syncthreads();
    }
    // Epilogue.
    if constexpr (EPI == EPI_SILU_SPLIT) {
        const int pairs = RT * 8 * tokens;
        for (int o = threadIdx.x; o < pairs; o += 256) {
            const int r = o / (tokens * 8), t = (o / 8) % tokens, pr = o % 8;
            const int row = (tile0 + r) * 16 + 2 * pr;
            if (row >= rows) continue;
            const float a = silu_f(vals[r][t][2 * pr]) * vals[r][t][2 * pr + 1];
            const size_t k = row >> 1, kc = epi.split_out.cols;
            const _Float16 hi = (_Float16)a;
            epi.split_out.data[(t * 2 + 0) * kc + k] = hi;
            epi.split_out.data[(t * 2 + 1) * kc + k] = (_Float16)(a - (float)hi);
            if (epi.act_out) epi.act_out[t * kc + k] = a;
        }
        if (blockIdx.x == 0 && threadIdx.x < (unsigned)tokens) epi.split_out.inv[threadIdx.x] = 1.0f;
    } else {
        for (int o = threadIdx.x; o < outputs; o += 256) {
            const int r = o / (tokens * 16), t = (o / 16) % tokens, row16 = o % 16;
            const int row = (tile0 + r) * 16 + row16;
            if (row >= rows) continue;
            const float v = vals[r][t][row16];
            const size_t at = (size_t)t * epi.y_stride + row;
            if constexpr (EPI == EPI_F32) reinterpret_cast<float *>(epi.y)[at] = v;
            if constexpr (EPI == EPI_ADD) reinterpret_cast<float *>(epi.y)[at] += v;
            if constexpr (EPI == EPI_BF16) {
                const unsigned u = __float_as_uint(v);
                const unsigned rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
                reinterpret_cast<uint16_t *>(epi.y)[at] = (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40u : rounded);
            }
        }
    }
}

bool mfma_supported(const marin_quant_matrix *w) {
    return w->bits == 8 && w->group % 64 == 0 && w->cols % 64 == 0;
}

// Chooses rows per block and column splits so a launch has about 2048+ waves with at least two windows each.
template <typename ST, int EPI, int PARTS>
static void launch_mfma_t(marin_gpu *g, const marin_quant_matrix *w, SplitView x, size_t tokens,
                          const EpiArgs &args) {
    const int windows = (int)(w->cols / 64);
    const size_t tiles = w->rows_padded / 16;
    int rt = tiles >= 4096 ? 4 : (tiles >= 1024 ? 2 : 1);
    const size_t blocks_x = tiles / rt;
    const size_t cu = (size_t)(g->cu_count > 0 ? g->cu_count : 256);
    int splits = 1;
    while (blocks_x * splits < 8 * cu && windows / (splits * 2) >= 2 * WAVES) splits *= 2;
    const int per_split = (windows + splits - 1) / splits;
    splits = (windows + per_split - 1) / per_split;
    if (splits > 1) g->ensure_partials((size_t)splits * tokens * w->rows_padded, blocks_x);
    const ST *sc = (const ST *)w->scales;
    dim3 grid((unsigned)blocks_x, (unsigned)splits);
#define MARIN_LAUNCH1(RT, ONE)                                                                                   \
    gemv_i8_mfma<RT, ST, EPI, PARTS, ONE><<<grid, dim3(256), 0, g->stream>>>(                                   \
        w->codes, sc, x.data, x.inv, (int)tokens, (int)w->rows, (int)w->rows_padded, (int)w->cols, (int)w->group, \
        per_split, g->partials, g->counters, args)
#define MARIN_LAUNCH(RT)                    \
    do {                                    \
        if (tokens == 1) MARIN_LAUNCH1(RT, true); \
        else MARIN_LAUNCH1(RT, false);      \
    } while (0)
    if (rt == 4) MARIN_LAUNCH(4);
    else if (rt == 2) MARIN_LAUNCH(2);
    else MARIN_LAUNCH(1);
#undef MARIN_LAUNCH
#undef MARIN_LAUNCH1
    // algorithmic bytes: codes + scales once, activations (f32) and outputs once
    const double bytes = (double)w->rows * w->row_bytes() + (double)w->rows * w->groups() * (w->bf16_scales ? 2 : 4) +
                         (double)tokens * w->cols * 4 + (double)tokens * w->rows * 4;
    g->launched(marin_gpu::GEMV, bytes);
}

template <int EPI, int PARTS>
static void launch_mfma_e(marin_gpu *g, const marin_quant_matrix *w, SplitView x, size_t tokens,
                          const EpiArgs &args) {
    if (w->bf16_scales) launch_mfma_t<uint16_t, EPI, PARTS>(g, w, x, tokens, args);
    else launch_mfma_t<float, EPI, PARTS>(g, w, x, tokens, args);
}

void launch_gemv_mfma(marin_gpu *g, const marin_quant_matrix *w, SplitView x, size_t tokens, Epilogue epi,
                      const EpiArgs &args) {
    if (tokens == 0) return;
    if (tokens > MAX_GEMV_TOKENS) throw Error(MARIN_UNSUPPORTED, "gemv tokens", MAX_GEMV_TOKENS, tokens);
    switch (epi) {
        case EPI_F32: launch_mfma_e<EPI_F32, 2>(g, w, x, tokens, args); break;
        case EPI_ADD: launch_mfma_e<EPI_ADD, 2>(g, w, x, tokens, args); break;
        case EPI_BF16: launch_mfma_e<EPI_BF16, 2>(g, w, x, tokens, args); break;
        case EPI_SILU_SPLIT: launch_mfma_e<EPI_SILU_SPLIT, 2>(g, w, x, tokens, args); break;
    }
}

static void launch_gemv_mfma_precise(marin_gpu *g, const marin_quant_matrix *w, SplitView x, size_t tokens,
                                     float *y) {
    EpiArgs a;
    a.y = y;
    a.y_stride = w->rows;
    launch_mfma_e<EPI_F32, 3>(g, w, x, tokens, a);
}

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
            const uint32_t u = *reinterpret_cast<const uint32_t *>(crow + c / 2);
#pragma unroll
            for (int i = 0; i < 8; ++i) wv[i] = (float)((int)((u >> (4 * i)) & 15u) - 8);
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
                                const uint32_t *__restrict__ ids, float *__restrict__ out, int cols, int group) {
    const size_t row = ids[blockIdx.x];
    const int groups = cols / group;
    const ST *srow = scales + (row / 16) * (size_t)groups * 16 + (row % 16);
    for (int i = threadIdx.x; i < cols; i += blockDim.x) {
        float s;
        if constexpr (sizeof(ST) == 4) s = srow[(i / group) * 16];
        else s = __uint_as_float((unsigned)srow[(i / group) * 16] << 16);
        out[(size_t)blockIdx.x * cols + i] = (float)(int8_t)codes[row * cols + i] * s;
    }
}

void launch_embed_q8(marin_gpu *g, const marin_quant_matrix *w, const uint32_t *ids, size_t n, float *out) {
    if (!n) return;
    if (w->bf16_scales)
        embed_q8_kernel<uint16_t><<<dim3((unsigned)n), dim3(256), 0, g->stream>>>(
            w->codes, (const uint16_t *)w->scales, ids, out, (int)w->cols, (int)w->group);
    else
        embed_q8_kernel<float><<<dim3((unsigned)n), dim3(256), 0, g->stream>>>(
            w->codes, (const float *)w->scales, ids, out, (int)w->cols, (int)w->group);
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
        codes[dst * cols + (size_t)gi * group + i] = (uint8_t)(int8_t)code;
    }
    if (lane == 0) scales[(dst / 16) * (size_t)groups * 16 + (size_t)gi * 16 + (dst % 16)] = scale;
}

void launch_synth_quantize(marin_gpu *g, marin_quant_matrix *w, uint64_t seed, uint64_t stream, double std_dev,
                           size_t src_rows, size_t dst_row0, size_t dst_row_step) {
    if (w->bits != 8 || w->bf16_scales) throw Error(MARIN_UNSUPPORTED, "synthetic matrices are int8 with f32 scales");
    if (w->group > 256) unsupported("synthetic group size", 256, w->group);
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

void upload_rows(marin_quant_matrix *m, const uint8_t *codes, const void *scales, size_t src_rows, size_t dst_row0,
                 size_t dst_row_step) {
    marin_gpu *g = m->gpu;
    const size_t rb = m->row_bytes(), groups = m->groups(), es = m->bf16_scales ? 2 : 4;
    // Codes: contiguous when the rows land contiguously, else row by row on the host side.
    std::vector<uint8_t> code_rows;
    if (dst_row_step == 1) {
        g->upload(m->codes + dst_row0 * rb, codes, src_rows * rb);
    } else {
        // Interleave into a host copy of the destination range, then one upload.
        const size_t last = dst_row0 + (src_rows - 1) * dst_row_step;
        const size_t span = last - dst_row0 + 1;
        code_rows.resize(span * rb);
        g->download(code_rows.data(), m->codes + dst_row0 * rb, span * rb);
        for (size_t r = 0; r < src_rows; ++r)
            std::memcpy(&code_rows[r * dst_row_step * rb], codes + r * rb, rb);
        g->upload(m->codes + dst_row0 * rb, code_rows.data(), span * rb);
    }
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
    if (!tokens) return;
    if (!mfma_supported(w)) {
        launch_gemv_valu(g, w, x, tokens, y);
        return;
    }
    const size_t chunk = precise ? 5 : MAX_GEMV_TOKENS;
    g->ensure_split(split_bytes(chunk, w->cols));
    for (size_t t0 = 0; t0 < tokens; t0 += chunk) {
        const size_t nt = std::min(chunk, tokens - t0);
        SplitView v = split_view(g->split, nt, w->cols);
        if (precise) {
            launch_split3_f32(g, x + t0 * w->cols, nt, w->cols, v);
            launch_gemv_mfma_precise(g, w, v, nt, y + t0 * w->rows);
        } else {
            launch_split_f32(g, x + t0 * w->cols, nt, w->cols, v, true);
            EpiArgs a;
            a.y = y + t0 * w->rows;
            a.y_stride = w->rows;
            launch_gemv_mfma(g, w, v, nt, EPI_F32, a);
        }
    }
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
        if (!mfma_supported(w)) unsupported("bf16 product group/width (int8, group and cols multiples of 64)", 8,
                                            (size_t)w->bits);
        g->ensure_split(split_bytes(MAX_GEMV_TOKENS, w->cols));
        for (size_t t0 = 0; t0 < tokens; t0 += MAX_GEMV_TOKENS) {
            const size_t nt = std::min<size_t>(MAX_GEMV_TOKENS, tokens - t0);
            SplitView v = split_view(g->split, nt, w->cols);
            launch_split_bf16(g, (const uint16_t *)x->data + t0 * w->cols, nt, w->cols, v);
            EpiArgs a;
            a.y = (uint16_t *)out->data + t0 * w->rows;
            a.y_stride = w->rows;
            launch_gemv_mfma(g, w, v, nt, EPI_BF16, a);
        }
    });
}

}  // extern "C"
