// The quantized product of the decode path on CDNA4's integer matrix cores.
//
// Codes go to v_mfma_i32_16x16x64_i8 untouched: a lane's 16-byte load of one weight row is its A operand. The
// activations become exact integers: each token is scaled by the power of two 2^s that puts its largest magnitude
// in [2^29, 2^30) and rounded to an integer, which four signed 8-bit limbs hold exactly (x = l3 2^24 + l2 2^16 +
// l1 2^8 + l0). The limbs are the B columns (four per token, so four tokens per MFMA). Products accumulate exactly
// in int32 across a group of 128 columns (2^21 at most), are converted to f32 once per group and scaled by the
// group's weight scale; the limb weights 2^(8l - s) are applied once at the end. Activations keep 30 bits below
// each token's largest value, so the result is f32-grade, and the weights cost no VALU work at all. int4 codes are
// unpacked to bytes with two masks (stored nibble = code + 8) and the offset is removed exactly in integers:
// sum (code + 8) l = sum code l + 8 sum l, with sum l precomputed per group and column.
//
// The prologue computes the per-token statistics (and the RMSNorm of the input when asked), the limbs into LDS and
// the tile's scales into LDS, while the first windows of codes are already in flight. Each wave then streams its
// share of the 128-column units through a ring of registers. The waves' sums meet in LDS for the epilogue.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "gemv.hpp"

namespace marin {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int GW = 8;        // waves per block
constexpr int LIMBS = 4;     // limbs per token
constexpr int pfu(int rt) { return rt >= 4 ? 2 : 4; }  // units of codes in flight per wave
constexpr int LDS_LIMBS = 64 * 1024;

struct TokenStat {
    float rs;   // RMSNorm factor (1 without a norm)
    float up;   // 2^s
    float down; // 2^-s
    float pad;
};

// Eight consecutive inputs of token t from column k (k a multiple of 8), with the norm weight applied when asked.
__device__ __forceinline__ void load_in8(const GemvIn &in, int t, int k, float v[8]) {
    if (in.mode == IN_BF16) {
        const uint4 u = *reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(in.x) +
                                                         (size_t)t * in.x_stride + k);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    } else {
        const float *p = reinterpret_cast<const float *>(in.x) + (size_t)t * in.x_stride + k;
        const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

__device__ __forceinline__ void load_norm8(const GemvIn &in, int k, float w[8]) {
    const float4 a = *reinterpret_cast<const float4 *>(in.norm + k), b = *reinterpret_cast<const float4 *>(in.norm + k + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

template <typename ST>
__device__ __forceinline__ float scale_at(const ST *p) {
    if constexpr (sizeof(ST) == 4) return *p;
    else return __uint_as_float((unsigned)*p << 16);
}

__device__ __forceinline__ float block_sum(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < GW; ++w) s += red[w];
    return s;
}

__device__ __forceinline__ float block_max(float v, float *red) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < GW; ++w) s = fmaxf(s, red[w]);
    return s;
}

__device__ __forceinline__ int total_key(float v) {
    const int b = __float_as_int(v);
    return b ^ (int)(((unsigned)(b >> 31)) >> 1);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// BITS: 8 or 4. RT: 16-row tiles per tile block. UW: 64-column windows per unit (2 when a group spans 128 columns).
// The grid is persistent: block b takes tile blocks b, b + gridDim.x, ... and pays for its prologue once. A wave's
// work is one sequence of (segment, unit) steps, a segment being one tile block (times one column chunk when the
// limbs are staged in chunks); its ring of code loads runs across segment ends, so the next tile's codes are in
// flight while a tile's sums are reduced and written.
template <int BITS, int RT, int UW, typename ST, bool ONE>
__global__ __launch_bounds__(64 * GW) void gemv_q(const uint8_t *__restrict__ codes, const ST *__restrict__ scales,
                                                  GemvIn in, GemvOut out, int tokens_arg, int rows, int cols,
                                                  int group, int kc, int tile_blocks) {
    extern __shared__ __align__(16) unsigned char lds[];
    const int tokens = ONE ? 1 : tokens_arg;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    const int used = tokens * LIMBS;
    const int groups = cols / group;
    constexpr int UC = 64 * UW;  // columns per unit
    const int units = cols / UC;
    constexpr int CB = BITS == 8 ? 16 : 8;  // code bytes per lane per window
    constexpr int PFU = pfu(RT);
    const size_t row_bytes = BITS == 8 ? (size_t)cols : (size_t)cols / 2;

    // LDS: token stats | limbs [tokens*4][kc] | column sums [kc/UC][16] (int4) | red [GW][RT][16][16] | vals
    TokenStat *stat = reinterpret_cast<TokenStat *>(lds);
    float *red8 = reinterpret_cast<float *>(lds + 4 * sizeof(TokenStat));
    int8_t *limbs = reinterpret_cast<int8_t *>(lds + 256);
    int *colsum = reinterpret_cast<int *>(lds + 256 + (size_t)used * kc);
    const size_t cs_bytes = BITS == 4 ? (size_t)(kc / UC) * 16 * 4 : 0;
    float *red = reinterpret_cast<float *>(lds + 256 + (size_t)used * kc + cs_bytes);
    float *vals = red + GW * RT * 16 * 16;

    // ---- the wave's step sequence
    const int chunks = (cols + kc - 1) / kc;
    const int upc = kc / UC;                   // units per chunk
    const int n_uni = (upc + GW - 1) / GW;     // steps per segment (the same for every wave)
    const int my_tbs = tile_blocks > (int)blockIdx.x ? (tile_blocks - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
    const int total_s = my_tbs * chunks * n_uni;
    // step s -> tile block, chunk, chunk-local unit (clamped to a real unit for loads)
    auto step_unit = [&](int st, int &tile0, int &ch, int &i, int &unit) {
        const int seg = st / n_uni;
        i = st % n_uni;
        ch = seg % chunks;
        tile0 = ((int)blockIdx.x + (seg / chunks) * (int)gridDim.x) * RT;
        const int in_chunk = min(upc, units - ch * upc);
        const int lu = min(wave + i * GW, in_chunk - 1);
        unit = ch * upc + lu;
    };
    typedef typename std::conditional<BITS == 8, u32x4, uint2>::type Raw;
    typedef typename std::conditional<sizeof(ST) == 4, floatx4, uint2>::type SRaw;
    Raw ring[PFU][RT][UW];
    SRaw sring[PFU][RT];
    auto load_step = [&](int st, Raw (&dst)[RT][UW], SRaw (&sdst)[RT]) {
        int tile0, ch, i, u;
        step_unit(st, tile0, ch, i, u);
        const int gi = (u * UC) / group;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
            const uint8_t *rowp = codes + (size_t)(tile0 + r) * 16 * row_bytes + CB * lane;
#pragma unroll
            for (int w = 0; w < UW; ++w) {
                const size_t off = (size_t)(u * UW + w) * 64 * CB;
                if constexpr (BITS == 8)
                    dst[r][w] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(rowp + off));
                else
                    dst[r][w] = *reinterpret_cast<const uint2 *>(rowp + off);
            }
            sdst[r] = *reinterpret_cast<const SRaw *>(scales + ((size_t)(tile0 + r) * groups + gi) * 16 + 4 * q);
        }
    };
    const int last_s = total_s > 0 ? total_s - 1 : 0;
    if (total_s > 0) {
#pragma unroll
        for (int j = 0; j < PFU; ++j) load_step(min(j, last_s), ring[j], sring[j]);
    }

    // ---- per-token statistics: RMSNorm factor and the power of two for the limbs
    for (int t = 0; t < tokens; ++t) {
        float ss = 0.0f, mx = 0.0f;
        for (int k = threadIdx.x * 8; k < cols; k += 8 * 64 * GW) {
            float x[8], w[8];
            load_in8(in, t, k, x);
            if (in.mode == IN_NORM) load_norm8(in, k, w);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                ss += x[e] * x[e];
                mx = fmaxf(mx, fabsf(in.mode == IN_NORM ? x[e] * w[e] : x[e]));
            }
        }
        float rs = 1.0f;
        if (in.mode == IN_NORM) {
            const float total = block_sum(ss, red8);
            rs = 1.0f / sqrtf(total / (float)cols + in.eps);
        }
        float m = block_max(mx, red8) * rs;
        if (threadIdx.x == 0) {
            int sh = 0;
            if (m > 0.0f && m < INFINITY) {
                int e;
                (void)frexpf(m, &e);
                sh = 30 - e;
                sh = sh > 90 ? 90 : (sh < -60 ? -60 : sh);
            }
            stat[t].rs = rs;
            stat[t].up = ldexpf(1.0f, sh);
            stat[t].down = ldexpf(1.0f, -sh);
        }
    }
    __syncthreads();

    // ---- limbs of chunk ch into LDS: a thread takes 8 consecutive columns of one token
    auto stage = [&](int ch) {
        const int col0 = ch * kc;
        const int kcols = min(kc, cols - col0);
        for (int idx = threadIdx.x; idx < tokens * (kcols / 8); idx += 64 * GW) {
            const int t = idx / (kcols / 8), k8 = (idx % (kcols / 8)) * 8;
            const TokenStat st = stat[t];
            float xv[8], wv[8];
            load_in8(in, t, col0 + k8, xv);
            if (in.mode == IN_NORM) load_norm8(in, col0 + k8, wv);
            uint32_t packed[LIMBS][2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t b[LIMBS] = {0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float v = xv[4 * h + e];
                    if (in.mode == IN_NORM) v = v * st.rs * wv[4 * h + e];
                    int xi = __float2int_rn(v * st.up);
#pragma unroll
                    for (int l = 0; l < LIMBS; ++l) {
                        const int lb = l == LIMBS - 1 ? xi : (int)(int8_t)(xi & 0xff);
                        b[l] |= ((uint32_t)lb & 0xffu) << (8 * e);
                        xi = (xi - lb) >> 8;
                    }
                }
#pragma unroll
                for (int l = 0; l < LIMBS; ++l) packed[l][h] = b[l];
            }
#pragma unroll
            for (int l = 0; l < LIMBS; ++l)
                *reinterpret_cast<uint2 *>(limbs + (size_t)(t * LIMBS + l) * kc + k8) =
                    make_uint2(packed[l][0], packed[l][1]);
            if constexpr (BITS == 4) {
                // per-unit column sums: UC/8 consecutive threads share a unit
#pragma unroll
                for (int l = 0; l < LIMBS; ++l) {
                    int sum = 0;
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int e = 0; e < 4; ++e) sum += (int)(int8_t)((packed[l][h] >> (8 * e)) & 0xffu);
#pragma unroll
                    for (int o = 1; o < UC / 8; o <<= 1) sum += __shfl_xor(sum, o);
                    if ((idx % (UC / 8)) == 0) colsum[(k8 / UC) * 16 + t * LIMBS + l] = sum;
                }
            }
        }
    };
    if (chunks == 1) {
        stage(0);
        __syncthreads();
    }

    floatx4 total[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) total[r] = (floatx4){0.f, 0.f, 0.f, 0.f};
    unsigned long long best = 0;  // greedy choice over this block's rows (argmax mode)

    for (int base = 0; base < total_s; base += PFU) {
#pragma unroll
        for (int j = 0; j < PFU; ++j) {
            const int st = base + j;  // slot j holds step st (base is a multiple of PFU)
            if (st >= total_s) break;
            Raw cur[RT][UW];
            SRaw scur[RT];
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                scur[r] = sring[j][r];
#pragma unroll
                for (int w = 0; w < UW; ++w) cur[r][w] = ring[j][r][w];
            }
            load_step(min(st + PFU, last_s), ring[j], sring[j]);
            int tile0, ch, i, u;
            step_unit(st, tile0, ch, i, u);
            if (chunks > 1 && i == 0) {
                __syncthreads();
                stage(ch);
                __syncthreads();
            }
            const int in_chunk = min(upc, units - ch * upc);
            if (wave + i * GW < in_chunk) {
                const int lcol = u * UC - ch * kc;  // column of the unit inside the chunk
                int4v b[UW];
#pragma unroll
                for (int w = 0; w < UW; ++w) {
                    b[w] = (int4v){0, 0, 0, 0};
                    if (c < used)
                        b[w] = *reinterpret_cast<const int4v *>(limbs + (size_t)c * kc + lcol + 64 * w + 16 * q);
                }
                int csum = 0;
                if constexpr (BITS == 4) csum = c < used ? colsum[(lcol / UC) * 16 + c] : 0;
#pragma unroll
                for (int r = 0; r < RT; ++r) {
                    int4v acc = (int4v){0, 0, 0, 0};
#pragma unroll
                    for (int w = 0; w < UW; ++w) {
                        int4v a;
                        if constexpr (BITS == 8) {
                            a = __builtin_bit_cast(int4v, cur[r][w]);
                        } else {
                            const uint2 raw = cur[r][w];
                            a = (int4v){(int)(raw.x & 0x0f0f0f0fu), (int)((raw.x >> 4) & 0x0f0f0f0fu),
                                        (int)(raw.y & 0x0f0f0f0fu), (int)((raw.y >> 4) & 0x0f0f0f0fu)};
                        }
                        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[w], acc, 0, 0, 0);
                    }
                    if constexpr (BITS == 4) acc -= (int4v){8 * csum, 8 * csum, 8 * csum, 8 * csum};
                    floatx4 sv;
                    if constexpr (sizeof(ST) == 4) {
                        sv = scur[r];
                    } else {
                        const uint2 sr = scur[r];
                        sv = (floatx4){__uint_as_float(sr.x << 16), __uint_as_float(sr.x & 0xffff0000u),
                                       __uint_as_float(sr.y << 16), __uint_as_float(sr.y & 0xffff0000u)};
                    }
                    const floatx4 d = (floatx4){(float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]};
                    total[r] += d * sv;
                }
            }
            if (i == n_uni - 1 && ch == chunks - 1) {
                // ---- end of a tile block: sum the waves and limbs, then the epilogue
                if (c < used) {
#pragma unroll
                    for (int r = 0; r < RT; ++r)
#pragma unroll
                        for (int k = 0; k < 4; ++k) red[((wave * RT + r) * 16 + c) * 16 + 4 * q + k] = total[r][k];
                }
#pragma unroll
                for (int r = 0; r < RT; ++r) total[r] = (floatx4){0.f, 0.f, 0.f, 0.f};
                __syncthreads();
                const int outputs = RT * tokens * 16;
                for (int o = threadIdx.x; o < outputs; o += 64 * GW) {
                    const int r = o / (tokens * 16), t = (o / 16) % tokens, row = o % 16;
                    float v = 0.0f;
                    float lw = stat[t].down;
#pragma unroll
                    for (int l = 0; l < LIMBS; ++l) {
                        float part = 0.0f;
#pragma unroll
                        for (int wv = 0; wv < GW; ++wv) part += red[((wv * RT + r) * 16 + t * LIMBS + l) * 16 + row];
                        v += part * lw;
                        lw *= 256.0f;
                    }
                    vals[(r * GEMV_TOKENS + t) * 16 + row] = v;
                }
                __syncthreads();
                if (out.mode == OUT_SILU) {
                    const int pairs = RT * 8 * tokens;
                    for (int o = threadIdx.x; o < pairs; o += 64 * GW) {
                        const int r = o / (tokens * 8), t = (o / 8) % tokens, pr = o % 8;
                        const int row = (tile0 + r) * 16 + 2 * pr;
                        if (row >= rows) continue;
                        const float g = vals[(r * GEMV_TOKENS + t) * 16 + 2 * pr];
                        const float uu = vals[(r * GEMV_TOKENS + t) * 16 + 2 * pr + 1];
                        reinterpret_cast<float *>(out.y)[(size_t)t * out.y_stride + (row >> 1)] = silu_f(g) * uu;
                    }
                } else {
                    for (int o = threadIdx.x; o < outputs; o += 64 * GW) {
                        const int r = o / (tokens * 16), t = (o / 16) % tokens, row16 = o % 16;
                        const int row = (tile0 + r) * 16 + row16;
                        if (row >= rows) continue;
                        const float v = vals[(r * GEMV_TOKENS + t) * 16 + row16];
                        const size_t at = (size_t)t * out.y_stride + row;
                        if (out.mode == OUT_F32) reinterpret_cast<float *>(out.y)[at] = v;
                        else if (out.mode == OUT_ADD) reinterpret_cast<float *>(out.y)[at] += v;
                        else {
                            const unsigned uu = __float_as_uint(v);
                            reinterpret_cast<uint16_t *>(out.y)[at] = (uint16_t)(
                                (uu & 0x7fffffffu) > 0x7f800000u ? (uu >> 16) | 0x40u
                                                                 : (uu + 0x7fffu + ((uu >> 16) & 1u)) >> 16);
                        }
                        if (out.argmax && t == tokens - 1) {
                            // largest under f32's total order, lowest row on ties (sampler/src/lib.rs:40-48)
                            const unsigned long long key =
                                (unsigned long long)((unsigned)total_key(v) ^ 0x80000000u) << 32 |
                                (unsigned long long)(0xffffffffu - (unsigned)row);
                            best = key > best ? key : best;
                        }
                    }
                }
                // vals/red are rewritten by the next tile block only after every thread has read them
                __syncthreads();
            }
        }
    }
    if (out.argmax) {
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(best, o);
            best = other > best ? other : best;
        }
        if (lane == 0 && best) atomicMax(out.argmax, best);
    }
}

bool gemv_supported(const marin_quant_matrix *w) {
    return (w->bits == 8 || w->bits == 4) && w->windowed;
}

template <int BITS, int RT, int UW, typename ST>
static void launch_t(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    const size_t groups = w->groups();
    // the whole row of limbs when it fits, else chunks of 4096 columns (a multiple of GW * pfu(RT) units)
    const size_t kc = tokens * LIMBS * w->cols <= (size_t)LDS_LIMBS ? w->cols : 4096;
    (void)groups;
    const size_t lds = 256 + tokens * LIMBS * kc + (BITS == 4 ? (kc / (64 * UW)) * 16 * 4 : 0) +
                       (size_t)(GW * RT * 16 * 16 + RT * GEMV_TOKENS * 16) * 4;
    // Persistent when the limbs stay in LDS for the whole launch: two blocks per compute unit walk the tile blocks.
    const size_t tile_blocks = w->rows_padded / 16 / RT;
    const size_t cu = (size_t)std::max(g->cu_count, 1);
    auto kern1 = gemv_q<BITS, RT, UW, ST, true>;
    auto kernn = gemv_q<BITS, RT, UW, ST, false>;
    auto kern = tokens == 1 ? kern1 : kernn;
    if (lds > 64 * 1024) {
        if (lds > 160 * 1024) unsupported("gemv shared memory (KiB)", 160, lds / 1024);
        HIP_CHECK(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    }
    int resident = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, kern, 64 * GW, lds) != hipSuccess || resident < 1)
        resident = 1;
    const size_t blocks = kc == w->cols ? std::min(tile_blocks, (size_t)resident * cu) : tile_blocks;
    dim3 grid((unsigned)blocks);
    kern<<<grid, dim3(64 * GW), lds, g->stream>>>(w->codes, (const ST *)w->scales, in, out, (int)tokens,
                                                   (int)w->rows, (int)w->cols, (int)w->group, (int)kc,
                                                   (int)tile_blocks);
}

template <int BITS, int UW, typename ST>
static void launch_rt(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    const size_t tiles = w->rows_padded / 16;
    (void)tiles;
    launch_t<BITS, 1, UW, ST>(g, w, in, out, tokens);
}

template <typename ST>
static void launch_st(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out,
                      size_t tokens) {
    const bool uw2 = w->group % 128 == 0;
    if (w->bits == 8) {
        if (uw2) launch_rt<8, 2, ST>(g, w, in, out, tokens);
        else launch_rt<8, 1, ST>(g, w, in, out, tokens);
    } else {
        if (uw2) launch_rt<4, 2, ST>(g, w, in, out, tokens);
        else launch_rt<4, 1, ST>(g, w, in, out, tokens);
    }
}

void launch_gemv(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    if (!tokens) return;
    if (tokens > GEMV_TOKENS) unsupported("tokens per product", GEMV_TOKENS, tokens);
    if (!gemv_supported(w)) unsupported("matrix-core product layout (group and columns multiples of 64)", 64, w->group);
    const char *name = "gemv_q";
    if (tokens == 1 && gemv_decode_supported(w)) {
        name = launch_gemv_decode(g, w, in, out);
    } else {
        if (g->only && strcmp(g->only, name)) return;
        if (w->bf16_scales) launch_st<uint16_t>(g, w, in, out, tokens);
        else launch_st<float>(g, w, in, out, tokens);
    }
    if (g->skipped) {
        g->skipped = false;
        return;
    }
    // algorithmic bytes: codes + scales once, activations and outputs once
    const double act = in.mode == IN_BF16 ? 2.0 : 4.0, res = out.mode == OUT_BF16 ? 2.0 : 4.0;
    const double rows = in.tile_map ? 16.0 * in.map_tiles * in.map_count : (double)w->rows;  // rows read
    const double outs = out.mode == OUT_SILU ? rows / 2 : rows;
    const double bytes = rows * w->row_bytes() + rows * w->groups() * (w->bf16_scales ? 2 : 4) +
                         (double)tokens * w->cols * act + (double)tokens * outs * res;
    g->launched(marin_gpu::GEMV, bytes, name);
}

}  // namespace marin
