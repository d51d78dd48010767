// The multi-token quantized product (prompt passes, mma.cu:52-268 of the reference redesigned): a GEMM on CDNA4's
// int8 matrix cores with the same exact arithmetic as the decode product.
//
// quantize_act turns a block of activation rows into signed 8-bit limbs: per (token, quantization group) the power
// of two 2^s that puts the group's largest magnitude in [2^29, 2^30), x 2^s rounded to an integer held exactly by
// four limbs (x = l3 2^24 + l2 2^16 + l1 2^8 + l0), limbs stored [token][limb][column]. With an RMSNorm input the
// limbs hold x * weight and the token's factor 1 / sqrt(mean(x^2) + eps) multiplies the token's outputs at the end.
//
// gemm_q8: a workgroup of 4 waves computes 128 weight rows x 32 tokens. Each wave owns two 16-row tiles and streams
// their code windows (the A operands of v_mfma_i32_16x16x64_i8, one contiguous KiB each); the token block's limbs
// for one group (B operands: 4 tokens x 4 limbs per 16 columns) are staged in LDS, double-buffered, and shared by
// the 4 waves. Per group: int32 sums, converted once, scaled by weight scale x 2^-s of the token, accumulated in f32.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "gemm.hpp"

namespace marin {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int QA_THREADS = 256;
// quantize_act's grid: a workgroup per (token, 1024 columns)
inline dim3 qa_grid(size_t tokens, size_t cols) { return dim3((unsigned)tokens, (unsigned)((cols + 1023) / 1024)); }
constexpr int GM_WAVES = 4;       // waves along the rows (128 rows per workgroup)
constexpr int GM_ROW_TILES = 2;   // 16-row tiles per wave
// Token halves of a workgroup: blocks of 64+ tokens take two sets of row waves, one per 32 tokens, so each code
// window a workgroup reads from memory serves 64 tokens (the second wave's load of it hits the caches).
__host__ __device__ constexpr int gm_halves(int tok) { return tok >= 64 ? tok / 32 : 1; }
constexpr int GM_TOKENS = 32;     // tokens per workgroup of the prompt GEMM

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

// (f32 total order, lowest row on ties) as one word: the larger word is the greedy choice (sampler/src/lib.rs:40-48)
__device__ __forceinline__ unsigned long long choice_key(float v, int row) {
    const int b = __float_as_int(v);
    const unsigned k = (unsigned)(b ^ (int)(((unsigned)(b >> 31)) >> 1)) ^ 0x80000000u;
    return (unsigned long long)k << 32 | (unsigned long long)(0xffffffffu - (unsigned)row);
}

}  // namespace

// grid (tokens, column slices of 1024): workgroup (t, y) quantizes columns [1024 y, 1024 (y + 1)) of token row t
// (GPI groups of GCOLS columns, GPI * GCOLS = 1024), one load per thread, so no workgroup walks a long row alone;
// workgroup (t, 0) also computes the row's RMSNorm factor. GCOLS = quantization group width (a multiple of 4, at most
// 4 * 64).
// FRAG false: limbs [token][limb][column]. FRAG true (the batch product): the limbs already in B-operand order,
// [window][token tile][64 lanes][16 bytes] with lane 16 q + 4 (token % 4) + limb holding columns 64 w + 16 q .. + 16,
// so each B fragment is one contiguous KiB; `ttiles` = token tiles of 4.
// L: limbs per value, 4 (30 bits below the group's largest magnitude) or 3 (22 bits, limbs [token][3][column],
// FRAG false only).
template <int GCOLS, bool FRAG, int L = 4>
__global__ __launch_bounds__(QA_THREADS) void quantize_act(GemvIn in, int cols, int8_t *__restrict__ limbs,
                                                           float *__restrict__ exps, float *__restrict__ rs_out,
                                                           int ttiles) {
    constexpr int TPG = GCOLS / 4;  // threads per group, 4 consecutive columns each
    static_assert(TPG <= 64 && (TPG & (TPG - 1)) == 0, "group width");
    static_assert(L == 4 || (L == 3 && !FRAG), "limbs");
    __shared__ float red[QA_THREADS / 64];
    const int t = blockIdx.x;
    const int groups = cols / GCOLS;
    auto load4 = [&](int k, float v[4]) {
        if (in.mode == IN_BF16) {
            const uint2 u = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(in.x) + (size_t)t * in.x_stride + k);
            v[0] = __uint_as_float(u.x << 16);
            v[1] = __uint_as_float(u.x & 0xffff0000u);
            v[2] = __uint_as_float(u.y << 16);
            v[3] = __uint_as_float(u.y & 0xffff0000u);
        } else {
            const float4 f = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(in.x) + (size_t)t * in.x_stride + k);
            v[0] = f.x;
            v[1] = f.y;
            v[2] = f.z;
            v[3] = f.w;
        }
    };
    const bool norm = in.mode == IN_NORM;
    float rs = 1.0f;
    if (norm && blockIdx.y == 0) {
        float ss = 0.0f;
#pragma unroll 4
        for (int k = threadIdx.x * 4; k < cols; k += QA_THREADS * 4) {
            float v[4];
            load4(k, v);
            ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
        }
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < QA_THREADS / 64; ++w) total += red[w];
        rs = 1.0f / sqrtf(total / (float)cols + in.eps);
    }
    if (threadIdx.x == 0 && blockIdx.y == 0) rs_out[t] = rs;
    constexpr int GPI = QA_THREADS / TPG;  // groups per iteration
    static_assert(GPI * GCOLS == 1024, "column slices of 1024");
    for (int g0 = (int)blockIdx.y * GPI; g0 < groups; g0 += GPI * (int)gridDim.y) {
        const int g = g0 + (int)threadIdx.x / TPG;
        const int k = g * GCOLS + ((int)threadIdx.x % TPG) * 4;
        const bool on = g < groups;
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (on) {
            load4(k, v);
            if (norm) {
                const float4 w = *reinterpret_cast<const float4 *>(in.norm + k);
                v[0] *= w.x;
                v[1] *= w.y;
                v[2] *= w.z;
                v[3] *= w.w;
            }
        }
        float mx = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        for (int o = 1; o < TPG; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        int sh = 0;
        if (mx > 0.0f && mx < INFINITY) {
            int e;
            (void)frexpf(mx, &e);
            sh = (8 * L - 2) - e;  // largest magnitude in [2^(8L-3), 2^(8L-2)): the top limb stays a signed byte
            sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
        }
        if (!on) continue;
        const float up = ldexpf(1.0f, sh);
        uint32_t word[L] = {};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int xi = __float2int_rn(v[e] * up);
#pragma unroll
            for (int l = 0; l < L; ++l) {
                const int lb = l == L - 1 ? xi : (int)(int8_t)(xi & 0xff);
                word[l] |= ((uint32_t)lb & 0xffu) << (8 * e);
                xi = (xi - lb) >> 8;
            }
        }
#pragma unroll
        for (int l = 0; l < L; ++l) {
            size_t at;
            if constexpr (FRAG) {
                const int lane = ((k & 63) >> 4) * 16 + (t & 3) * 4 + l;
                at = (((size_t)(k >> 6) * ttiles + (t >> 2)) * 64 + lane) * 16 + (k & 15);
            } else {
                at = ((size_t)t * L + l) * cols + k;
            }
            *reinterpret_cast<uint32_t *>(limbs + at) = word[l];
        }
        if ((threadIdx.x % TPG) == 0) exps[(size_t)t * groups + g] = ldexpf(1.0f, -sh);
    }
}

// The same limbs in one pass, for short rows of a decode batch (the batch product's B fragments): one token per
// workgroup of 1024 threads, thread T holding columns 4 T + 4096 i (i < IT) in registers from a single load burst
// (the row and its norm weights), one block reduction for the RMSNorm statistic, then the limbs in fragment order.
constexpr int QR_THREADS = 1024;
template <int GCOLS, int IT>
__global__ __launch_bounds__(QR_THREADS) void quantize_rows(GemvIn in, int cols, int8_t *__restrict__ limbs,
                                                            float *__restrict__ exps, float *__restrict__ rs_out,
                                                            int32_t *__restrict__ lsum, int ttiles) {
    constexpr int TPG = GCOLS / 4;
    __shared__ float red[QR_THREADS / 64];
    const int t = blockIdx.x;
    const int groups = cols / GCOLS;
    const bool norm = in.mode == IN_NORM;
    // without a norm the columns may be split over gridDim.y workgroups of 4 QR_THREADS IT columns each
    const int col0 = (int)blockIdx.y * 4 * QR_THREADS * IT;
    float v[IT][4], w[IT][4];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int k = min(col0 + 4 * ((int)threadIdx.x + QR_THREADS * it), cols - 4);  // clamped: loads stay unconditional
        if (in.mode == IN_BF16) {
            const uint2 u = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(in.x) + (size_t)t * in.x_stride + k);
            v[it][0] = __uint_as_float(u.x << 16);
            v[it][1] = __uint_as_float(u.x & 0xffff0000u);
            v[it][2] = __uint_as_float(u.y << 16);
            v[it][3] = __uint_as_float(u.y & 0xffff0000u);
        } else {
            const float4 f = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(in.x) + (size_t)t * in.x_stride + k);
            v[it][0] = f.x;
            v[it][1] = f.y;
            v[it][2] = f.z;
            v[it][3] = f.w;
        }
        const float4 nw = *reinterpret_cast<const float4 *>(norm ? in.norm + k : reinterpret_cast<const float *>(in.x) + k);
        w[it][0] = nw.x;
        w[it][1] = nw.y;
        w[it][2] = nw.z;
        w[it][3] = nw.w;
    }
    float rs = 1.0f;
    if (norm) {
        float ss = 0.0f;
#pragma unroll
        for (int it = 0; it < IT; ++it)
            if (4 * ((int)threadIdx.x + QR_THREADS * it) < cols)
#pragma unroll
                for (int e = 0; e < 4; ++e) ss += v[it][e] * v[it][e];
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < QR_THREADS / 64; ++i) total += red[i];
        rs = 1.0f / sqrtf(total / (float)cols + in.eps);
    }
    if (threadIdx.x == 0 && blockIdx.y == 0) rs_out[t] = rs;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
        const int k = col0 + 4 * ((int)threadIdx.x + QR_THREADS * it);
        const bool on = k < cols;
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = on ? (norm ? v[it][e] * w[it][e] : v[it][e]) : 0.0f;
        float mx = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
        for (int o = 1; o < TPG; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        int sh = 0;
        if (mx > 0.0f && mx < INFINITY) {
            int e;
            (void)frexpf(mx, &e);
            sh = 30 - e;
            sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
        }
        const float up = ldexpf(1.0f, sh);
        uint32_t word[4] = {0u, 0u, 0u, 0u};
        int ls[4] = {0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int xi = __float2int_rn(x[e] * up);
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const int lb = l == 3 ? xi : (int)(int8_t)(xi & 0xff);
                word[l] |= ((uint32_t)lb & 0xffu) << (8 * e);
                ls[l] += lb;
                xi = (xi - lb) >> 8;
            }
        }
        // the group's sum of each limb (int4 codes are stored + 8: the product removes 8 x this sum exactly)
#pragma unroll
        for (int l = 0; l < 4; ++l)
            for (int o = 1; o < TPG; o <<= 1) ls[l] += __shfl_xor(ls[l], o);
        if (!on) continue;
        if ((threadIdx.x % TPG) == 0)
            *reinterpret_cast<int4 *>(lsum + ((size_t)t * groups + k / GCOLS) * 4) = make_int4(ls[0], ls[1], ls[2], ls[3]);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const int lane = ((k & 63) >> 4) * 16 + (t & 3) * 4 + l;
            *reinterpret_cast<uint32_t *>(limbs + (((size_t)(k >> 6) * ttiles + (t >> 2)) * 64 + lane) * 16 + (k & 15)) = word[l];
        }
        if ((threadIdx.x % TPG) == 0) exps[(size_t)t * groups + k / GCOLS] = ldexpf(1.0f, -sh);
    }
}

// WG: 64-column windows per group; TOK: tokens per workgroup (a multiple of 4).
// Prompt GEMM (MOE false): grid (row blocks of 128, token blocks of TOK).
// Grouped expert product (MOE true, gate_up of a decode batch of at most TOK tokens): grid (row blocks of 128 of
// one expert, distinct selected experts); workgroup (x, u) computes rows 128 x .. of expert plan.experts[u] for every
// token and writes SiLU(gate) * up of the tokens that selected it into their (token, slot) activation rows. `tiles`
// is then the tiles of one expert.
template <int WG, typename ST, int TOK, bool MOE>
__global__ __launch_bounds__(64 * GM_WAVES * gm_halves(TOK)) void gemm_q8(const uint8_t *__restrict__ codes,
                                                         const ST *__restrict__ scales,
                                                         const int8_t *__restrict__ limbs,
                                                         const float *__restrict__ exps,
                                                         const float *__restrict__ rsv, GemvOut out, int tokens,
                                                         int rows, int cols, int tiles, MoePlanView plan) {
    constexpr int TT = TOK / 4;  // token tiles of 4 (one MFMA's 16 B columns)
    constexpr int TH = gm_halves(TOK), NWV = GM_WAVES * TH;  // token halves, waves
    constexpr int TTW = TT / TH;                               // token tiles per wave
    // B fragments of one group: [buffer][window][token tile][64 lanes] x 16 bytes, and the tokens' group factors
    __shared__ u32x4 bl[2][WG][TT][64];
    __shared__ float ex[2][TOK];
    __shared__ unsigned long long best_s[TOK];  // per-token greedy choice of the block (argmax_each)
    if (threadIdx.x < TOK) best_s[threadIdx.x] = 0ull;  // read after the pipeline's barriers
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    const int windows = cols >> 6;
    const int groups = windows / WG;
    int t0 = blockIdx.y * TOK, tbase = 0;
    if constexpr (MOE) {
        // the whole workgroup leaves together, before any barrier
        if ((int)blockIdx.y >= plan.plan[0]) return;
        t0 = 0;
        tbase = plan.plan[MOE_PLAN_EXPERTS + blockIdx.y] * tiles;  // the expert's first tile
    }
    const int wrow = wave % GM_WAVES, jbase = (wave / GM_WAVES) * TTW;  // the wave's rows and first token tile
    const int tile0 = (blockIdx.x * GM_WAVES + wrow) * GM_ROW_TILES;
    const size_t tile_bytes = (size_t)16 * cols;

    // staging of a group's B fragments: piece p = (window, token tile, lane) of the group, 16 bytes each
    constexpr int PIECES = WG * TT * 64;
    constexpr int PPT = (PIECES + 64 * NWV - 1) / (64 * NWV);  // pieces per thread (the last clamped)
    struct BStage {
        u32x4 v[PPT];
        float e;
    };
    struct AStage {
        u32x4 a[GM_ROW_TILES][WG];
        floatx4 sc[GM_ROW_TILES];
    };
    auto b_load = [&](int g, BStage &st) {
        g = min(g, groups - 1);
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int p = min((int)threadIdx.x + i * 64 * NWV, PIECES - 1);
            const int w = p / (TT * 64), j = (p / 64) % TT, ln = p % 64;
            const int tok = min(t0 + 4 * j + (ln & 15) / 4, tokens - 1);
            const int limb = (ln & 15) % 4;
            const int col = 64 * (g * WG + w) + 16 * (ln >> 4);
            st.v[i] = *reinterpret_cast<const u32x4 *>(limbs + ((size_t)tok * 4 + limb) * cols + col);
        }
        st.e = exps[(size_t)min(t0 + (int)(threadIdx.x % TOK), tokens - 1) * groups + g];
    };
    auto b_store = [&](int buf, const BStage &st) {
#pragma unroll
        for (int i = 0; i < PPT; ++i) {
            const int p = (int)threadIdx.x + i * 64 * NWV;
            const int w = p / (TT * 64), j = (p / 64) % TT, ln = p % 64;
            if (p < PIECES) bl[buf][w][j][ln] = st.v[i];
        }
        if (threadIdx.x < TOK) ex[buf][threadIdx.x] = st.e;
    };
    // A operands (codes) and weight scales of a group for the wave's tiles (clamped to a real tile and group)
    auto a_load = [&](int g, AStage &st) {
        g = min(g, groups - 1);
#pragma unroll
        for (int rt = 0; rt < GM_ROW_TILES; ++rt) {
            const int tl = tbase + min(tile0 + rt, tiles - 1);
            const uint8_t *base = codes + (size_t)tl * tile_bytes + 16 * lane;
#pragma unroll
            for (int w = 0; w < WG; ++w)
                st.a[rt][w] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + (size_t)(g * WG + w) * 1024));
            const ST *sp = scales + ((size_t)tl * groups + g) * 16 + 4 * q;
            if constexpr (sizeof(ST) == 4) {
                st.sc[rt] = *reinterpret_cast<const floatx4 *>(sp);
            } else {
                const uint2 sv = *reinterpret_cast<const uint2 *>(sp);
                st.sc[rt] = (floatx4){__uint_as_float(sv.x << 16), __uint_as_float(sv.x & 0xffff0000u),
                                      __uint_as_float(sv.y << 16), __uint_as_float(sv.y & 0xffff0000u)};
            }
        }
    };

    floatx4 total[GM_ROW_TILES][TTW];
#pragma unroll
    for (int rt = 0; rt < GM_ROW_TILES; ++rt)
#pragma unroll
        for (int j = 0; j < TTW; ++j) total[rt][j] = (floatx4){0.f, 0.f, 0.f, 0.f};

    // One group: MFMAs with A from registers and B from LDS buffer `buf`, then the group's scaling.
    auto compute = [&](int buf, const AStage &as) {
        int4v acc[GM_ROW_TILES][TTW];
#pragma unroll
        for (int rt = 0; rt < GM_ROW_TILES; ++rt)
#pragma unroll
            for (int j = 0; j < TTW; ++j) acc[rt][j] = (int4v){0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < WG; ++w) {
#pragma unroll
            for (int j = 0; j < TTW; ++j) {
                const int4v bfrag = __builtin_bit_cast(int4v, bl[buf][w][jbase + j][lane]);
#pragma unroll
                for (int rt = 0; rt < GM_ROW_TILES; ++rt)
                    acc[rt][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(int4v, as.a[rt][w]), bfrag,
                                                                       acc[rt][j], 0, 0, 0);
            }
        }
        // lane (q, c): rows 4q..4q+3 of each tile, token 4 (jbase + j) + c/4, limb c%4
#pragma unroll
        for (int j = 0; j < TTW; ++j) {
            const float tf = ex[buf][4 * (jbase + j) + c / 4];
#pragma unroll
            for (int rt = 0; rt < GM_ROW_TILES; ++rt) {
                const floatx4 f = (floatx4){(float)acc[rt][j][0], (float)acc[rt][j][1], (float)acc[rt][j][2],
                                            (float)acc[rt][j][3]};
                total[rt][j] += f * (as.sc[rt] * tf);
            }
        }
    };

    // Pipeline, two groups ahead: at iteration g, LDS buffer g%2 holds B(g), A(g) is in registers; B(g+1) and
    // A(g+1) are in flight; the iteration issues B(g+2), computes g, issues A(g+2) into the registers A(g) held,
    // stores B(g+1) into the other buffer and meets the other waves. Unrolled by two so every register ring index
    // is static.
    AStage ra[2];
    BStage rb[2];
    a_load(0, ra[0]);
    b_load(0, rb[0]);
    a_load(1, ra[1]);
    b_load(1, rb[1]);
    b_store(0, rb[0]);
    __syncthreads();
    auto iteration = [&](int g, AStage &a_now, BStage &b_free, BStage &b_next) {
        b_load(g + 2, b_free);
        compute(g & 1, a_now);
        a_load(g + 2, a_now);
        b_store((g + 1) & 1, b_next);
        __syncthreads();
    };
    for (int g = 0; g < groups; g += 2) {
        iteration(g, ra[0], rb[0], rb[1]);
        if (g + 1 < groups) iteration(g + 1, ra[1], rb[1], rb[0]);
    }

    // limbs weighted 2^(8 l) and summed over the four lanes of a token, then the outputs
    const float lw = (c & 3) == 0 ? 1.0f : (c & 3) == 1 ? 256.0f : (c & 3) == 2 ? 65536.0f : 16777216.0f;
#pragma unroll
    for (int rt = 0; rt < GM_ROW_TILES; ++rt) {
        const int tile = tile0 + rt;
#pragma unroll
        for (int j = 0; j < TTW; ++j) {
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float x = total[rt][j][k] * lw;
                x += __shfl_xor(x, 1);
                x += __shfl_xor(x, 2);
                v[k] = x;
            }
            const int tok = t0 + 4 * (jbase + j) + c / 4;
            const int row0 = tile * 16 + 4 * q;
            const bool mine = (c & 3) == 0 && tok < tokens && tile < tiles;
            const float r = rsv[min(tok, tokens - 1)];
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] *= r;
            if constexpr (!MOE) {
                if (out.argmax_each) {
                    // the rows of lanes q = 0..3 (same token) reduced by shuffles, then one LDS max per token
                    unsigned long long key = 0ull;
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (mine && row0 + k < rows) {
                            const unsigned long long kk = choice_key(v[k], row0 + k);
                            key = kk > key ? kk : key;
                        }
#pragma unroll
                    for (int o = 16; o < 64; o <<= 1) {
                        const unsigned long long other = __shfl_xor(key, o);
                        key = other > key ? other : key;
                    }
                    if (mine && q == 0 && key) atomicMax(&best_s[tok - t0], key);
                }
            }
            if (!mine) continue;
            if constexpr (MOE) {
                // the token's slot for this expert (-1: it did not select it); rows are the expert's interleaved
                // gate/up pairs
                const int slot = plan.plan[MOE_PLAN_SLOTS + blockIdx.y * MOE_BATCH + tok];
                if (slot < 0) continue;
                float *dst = reinterpret_cast<float *>(out.y) + ((size_t)tok * plan.k + slot) * plan.ffn;
#pragma unroll
                for (int k = 0; k < 4; k += 2) dst[(row0 + k) >> 1] = silu_f(v[k]) * v[k + 1];
                continue;
            }
            if (out.mode == OUT_SILU) {
#pragma unroll
                for (int k = 0; k < 4; k += 2) {
                    const int row = row0 + k;
                    if (row < rows)
                        reinterpret_cast<float *>(out.y)[(size_t)tok * out.y_stride + (row >> 1)] = silu_f(v[k]) * v[k + 1];
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int row = row0 + k;
                    if (row >= rows) continue;
                    const size_t at = (size_t)tok * out.y_stride + row;
                    if (out.mode == OUT_F32) reinterpret_cast<float *>(out.y)[at] = v[k];
                    else if (out.mode == OUT_ADD) reinterpret_cast<float *>(out.y)[at] += v[k];
                    else {
                        const unsigned uu = __float_as_uint(v[k]);
                        reinterpret_cast<uint16_t *>(out.y)[at] = (uint16_t)(
                            (uu & 0x7fffffffu) > 0x7f800000u ? (uu >> 16) | 0x40u
                                                             : (uu + 0x7fffu + ((uu >> 16) & 1u)) >> 16);
                    }
                }
            }
        }
    }
    if constexpr (!MOE) {
        if (out.argmax_each) {
            __syncthreads();
            if ((int)threadIdx.x < TOK && t0 + (int)threadIdx.x < tokens && best_s[threadIdx.x])
                atomicMax(out.argmax + t0 + threadIdx.x, best_s[threadIdx.x]);
        }
    }
}

// The prompt GEMM (gemm_prompt): prompt passes of GP_MIN_TOKENS+ tokens, a redesign of gemm_q8 around the
// matrix cores' feed. Activations are 22-bit fixed point below each (token, group)'s largest magnitude in three
// signed 8-bit limbs (the arithmetic of the reference's integer path, mma.cu:160-268), stored [token][3][column].
// A B operand holds 16 tokens of one limb (limb-major), so a 16x16x64 MFMA does a third more useful work than four
// limbs of 4 tokens. A workgroup of GP_WM x GP_WN waves computes GP_ROWS rows x GP_TOK tokens; a wave owns GP_RT
// 16-row tiles x GP_TN 16-token tiles, so every A fragment it reads from LDS feeds 6 MFMAs and every B fragment 4.
//
// Each 64-column window's operands (the rows' code windows, the tokens' limb fragments, the group's weight scales
// and token factors) go from memory straight into LDS (global_load_lds, 16 bytes a lane, no registers), into one of
// GP_STAGES stages, GP_STAGES - 1 windows ahead of the window being computed. Every wave issues the same number of
// these loads per window, so one counted wait (vmcnt) plus one barrier per window proves the window's stage complete
// for all waves and the previous stage free. The main loop issues no other vector-memory instruction, so the counts
// are exact.
//
// Workgroups are numbered so that all token blocks of a row block fall on one XCD (workgroup i runs on XCD i % 8):
// the row block's codes come from HBM once into that XCD's L2 and serve all of them.
constexpr int GP_WN = 2, GP_RT = 4, GP_TN = 2, GP_L = 3;
constexpr int GP_TOK = GP_WN * GP_TN * 16;  // tokens per workgroup
constexpr size_t GP_MIN_TOKENS = 32;
static_assert(GP_TOK <= 64, "one token factor per lane");
// The workgroup's shape for GP_WM row waves (4: 256 rows; 2: 128 rows, for matrices whose 256-row blocks would leave
// compute units idle) and its stage layout: A [tile][64 lanes][16 B] | B [token tile][limb][64 lanes][16 B] |
// scales [rows] f32 (bf16: the first half) | token factors [tokens] f32 | pad (the spare loads' target)
template <int WM, int GS>
struct GpShape {
    static constexpr int ROWS = WM * GP_RT * 16, TILES = ROWS / 16;
    static constexpr int WAVES = WM * GP_WN, THREADS = 64 * WAVES;
    // stages of GS windows: one-window stages 4 deep (3 for 128-row workgroups, so two fit a compute unit),
    // group stages 2 deep
    static constexpr int STAGES = GS > 1 ? 2 : (WM == 4 ? 4 : 3);
    static constexpr int A_BYTES = TILES * 1024, B_BYTES = GP_WN * GP_TN * GP_L * 1024;
    static constexpr int WIN_BYTES = A_BYTES + B_BYTES;  // one window's operands inside a stage
    static constexpr int SC_OFF = GS * WIN_BYTES, EX_OFF = SC_OFF + 1024, PAD_OFF = EX_OFF + GP_TOK * 4;
    static constexpr int STAGE_BYTES = (PAD_OFF + 1024 + 255) / 256 * 256;
    // loads per stage: A tiles and B fragments of each window, scales, token factors; padded to a whole number per
    // wave
    static constexpr int PER_WIN = TILES + GP_WN * GP_TN * GP_L;
    static constexpr int LOADS = GS * PER_WIN + 2;
    static constexpr int LPW = (LOADS + WAVES - 1) / WAVES;
    static_assert(ROWS * 4 <= 1024, "scales of one stage");
};

typedef __attribute__((address_space(3))) void gp_lds_t;
typedef __attribute__((address_space(1))) const void gp_glb_t;

template <int WG, typename ST, int WM, int GS>
__global__ __launch_bounds__((GpShape<WM, GS>::THREADS), WM == 4 ? 1 : 2) void gemm_prompt(const uint8_t *__restrict__ codes,
                                                              const ST *__restrict__ scales,
                                                              const int8_t *__restrict__ limbs,
                                                              const float *__restrict__ exps,
                                                              const float *__restrict__ rsv, GemvOut out, int tokens,
                                                              int rows, int cols, int tiles, int row_blocks,
                                                              int token_blocks) {
    extern __shared__ __align__(256) unsigned char gp_lds[];
    using S = GpShape<WM, GS>;
    static_assert(GS == 1 || GS == WG, "stages of one window or of one group");
    constexpr int GP_WM = WM, GP_TILES = S::TILES, GP_LPW = S::LPW;
    constexpr int GP_A_BYTES = S::A_BYTES, GP_SC_OFF = S::SC_OFF, GP_EX_OFF = S::EX_OFF, GP_PAD_OFF = S::PAD_OFF;
    constexpr int GP_STAGE_BYTES = S::STAGE_BYTES, GP_STAGES = S::STAGES;
    // XCD-aware numbering: ids in runs of 8 x token_blocks; within a run, id % 8 picks the row block, id / 8 the
    // token block
    const int run = 8 * token_blocks, id = (int)blockIdx.x;
    const int rb = (id / run) * 8 + id % 8, tb = (id % run) / 8;
    if (rb >= row_blocks) return;  // the whole workgroup, before any barrier
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave % GP_WM, wn = wave / GP_WM;
    const int c = lane & 15, q = lane >> 4;
    const int windows = cols >> 6;
    const int groups = windows / WG;
    const int t0 = tb * GP_TOK;
    const int tbase = rb * GP_TILES;
    const size_t tile_bytes = (size_t)16 * cols;

    // The wave's GP_LPW loads per window: each slot's per-lane source address without the window's offset, worked
    // out once (the loop adds a wave-uniform offset), its kind and its LDS offset inside a stage.
    const unsigned char *src[GP_LPW];
    int kind[GP_LPW], dst[GP_LPW];
    int sub_w[GP_LPW];  // the slot's window inside the stage
#pragma unroll
    for (int i = 0; i < GP_LPW; ++i) {
        const int k0 = wave * GP_LPW + i;  // wave-uniform
        const int u = k0 < GS * S::PER_WIN ? k0 / S::PER_WIN : 0;
        const int k = k0 < GS * S::PER_WIN ? k0 % S::PER_WIN : k0 - GS * S::PER_WIN + S::PER_WIN;
        sub_w[i] = u;
        if (k < GP_TILES) {
            const int tl = min(tbase + k, tiles - 1);
            src[i] = codes + (size_t)tl * tile_bytes + 16 * lane;
            kind[i] = 0;
            dst[i] = u * S::WIN_BYTES + k * 1024;
        } else if (k < GP_TILES + GP_WN * GP_TN * GP_L) {
            const int f = k - GP_TILES, j = f / GP_L, l = f % GP_L;
            const int tok = min(t0 + 16 * j + c, tokens - 1);
            src[i] = reinterpret_cast<const unsigned char *>(limbs + ((size_t)tok * GP_L + l) * cols + 16 * q);
            kind[i] = 1;
            dst[i] = u * S::WIN_BYTES + GP_A_BYTES + f * 1024;
        } else if (k == GP_TILES + GP_WN * GP_TN * GP_L) {
            // 16 bytes a lane: f32 scales of 4 rows (lane l: tile l / 4), bf16 of 8 rows (lanes 32+ repeat)
            const int r0 = sizeof(ST) == 4 ? 4 * lane : 8 * (lane & 31);
            const int tl = min(tbase + r0 / 16, tiles - 1);
            src[i] = reinterpret_cast<const unsigned char *>(scales + (size_t)tl * groups * 16 + r0 % 16);
            kind[i] = 2;
            dst[i] = GP_SC_OFF;
        } else {
            // the token factors (4 bytes a lane); past them, spare loads that keep every wave's count equal
            src[i] = reinterpret_cast<const unsigned char *>(exps + (size_t)min(t0 + lane, tokens - 1) * groups);
            kind[i] = 3;
            dst[i] = k == GP_TILES + GP_WN * GP_TN * GP_L + 1 ? GP_EX_OFF : GP_PAD_OFF;
        }
    }
    // the wave's loads of window `win` into stage `st` (a window past the last loads the last one again)
    auto issue = [&](int unit, int st) {  // stage unit `unit`: windows unit GS .. + GS - 1
        const int w0 = min(unit * GS, windows - GS);
        const int g = w0 / WG;
        unsigned char *base = gp_lds + st * GP_STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < GP_LPW; ++i) {
            const int win = w0 + sub_w[i];
            if (kind[i] == 0)
                __builtin_amdgcn_global_load_lds((gp_glb_t *)(src[i] + (size_t)win * 1024), (gp_lds_t *)(base + dst[i]), 16, 0, 0);
            else if (kind[i] == 1)
                __builtin_amdgcn_global_load_lds((gp_glb_t *)(src[i] + 64 * win), (gp_lds_t *)(base + dst[i]), 16, 0, 0);
            else if (kind[i] == 2)
                __builtin_amdgcn_global_load_lds((gp_glb_t *)(src[i] + (size_t)g * 16 * sizeof(ST)), (gp_lds_t *)(base + dst[i]), 16, 0, 0);
            else
                __builtin_amdgcn_global_load_lds((gp_glb_t *)(src[i] + (size_t)g * 4), (gp_lds_t *)(base + dst[i]), 4, 0, 0);
        }
    };

    floatx4 total[GP_RT][GP_TN];
#pragma unroll
    for (int rt = 0; rt < GP_RT; ++rt)
#pragma unroll
        for (int j = 0; j < GP_TN; ++j) total[rt][j] = (floatx4){0.f, 0.f, 0.f, 0.f};

    // One group: per window (from its stage) the MFMAs into int32 sums over the group (each below 2^21 in
    // magnitude), then the limbs recombined once: l0 + 256 l1 in an integer (below 2^30), + 65536 l2 in f32, scaled
    // by weight scale x the token's 2^-s.
    int4v acc[GP_RT][GP_TN][GP_L];
    auto mfmas = [&](int st, int u) {
        const unsigned char *base = gp_lds + st * GP_STAGE_BYTES + u * S::WIN_BYTES;
        int4v af[GP_RT];
#pragma unroll
        for (int rt = 0; rt < GP_RT; ++rt)
            af[rt] = *reinterpret_cast<const int4v *>(base + (wm * GP_RT + rt) * 1024 + 16 * lane);
#pragma unroll
        for (int j = 0; j < GP_TN; ++j) {
#pragma unroll
            for (int l = 0; l < GP_L; ++l) {
                const int4v bfrag = *reinterpret_cast<const int4v *>(base + GP_A_BYTES + ((wn * GP_TN + j) * GP_L + l) * 1024 + 16 * lane);
#pragma unroll
                for (int rt = 0; rt < GP_RT; ++rt)
                    acc[rt][j][l] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[rt], bfrag, acc[rt][j][l], 0, 0, 0);
            }
        }
    };
    auto finish = [&](int st) {
        const unsigned char *base = gp_lds + st * GP_STAGE_BYTES;
        // lane (q, c): rows 4q..4q+3 of each tile, token 16 (wn GP_TN + j) + c
        floatx4 sc[GP_RT];
#pragma unroll
        for (int rt = 0; rt < GP_RT; ++rt) {
            const int r = (wm * GP_RT + rt) * 16 + 4 * q;
            if constexpr (sizeof(ST) == 4) {
                sc[rt] = *reinterpret_cast<const floatx4 *>(base + GP_SC_OFF + 4 * r);
            } else {
                const uint2 sv = *reinterpret_cast<const uint2 *>(base + GP_SC_OFF + 2 * r);
                sc[rt] = (floatx4){__uint_as_float(sv.x << 16), __uint_as_float(sv.x & 0xffff0000u),
                                   __uint_as_float(sv.y << 16), __uint_as_float(sv.y & 0xffff0000u)};
            }
        }
#pragma unroll
        for (int j = 0; j < GP_TN; ++j) {
            const float tf = *reinterpret_cast<const float *>(base + GP_EX_OFF + 4 * (16 * (wn * GP_TN + j) + c));
#pragma unroll
            for (int rt = 0; rt < GP_RT; ++rt) {
                const floatx4 m = sc[rt] * tf;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int lo = acc[rt][j][0][k] + (acc[rt][j][1][k] << 8);
                    total[rt][j][k] += ((float)lo + 65536.0f * (float)acc[rt][j][2][k]) * m[k];
                }
            }
        }
    };

    // windows 0 .. GP_STAGES - 2 in flight, then per window: wait for this window's loads (the later windows' may
    // stay in flight), meet the other waves (the window is complete for all, and the stage computed last is free),
    // issue the window GP_STAGES - 1 ahead into that stage, compute.
#pragma unroll
    for (int i = 0; i < GP_STAGES - 1; ++i) issue(i, i);
    for (int g = 0; g < groups; ++g) {
#pragma unroll
        for (int rt = 0; rt < GP_RT; ++rt)
#pragma unroll
            for (int j = 0; j < GP_TN; ++j)
#pragma unroll
                for (int l = 0; l < GP_L; ++l) acc[rt][j][l] = (int4v){0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < WG; ++w) {
            const int i = g * WG + w;
            if (GS == 1 || w == 0) {
                const int unit = i / GS;
                // at most the loads of units unit + 1 .. unit + GP_STAGES - 2 outstanding
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"((GP_STAGES - 2) * GP_LPW) : "memory");
                __builtin_amdgcn_s_barrier();
                issue(unit + GP_STAGES - 1, (unit + GP_STAGES - 1) % GP_STAGES);
            }
            mfmas((i / GS) % GP_STAGES, i % GS);
            if (w == WG - 1) finish((i / GS) % GP_STAGES);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the spare loads past the last window land before exit
    __builtin_amdgcn_s_barrier();

    const int tile0 = tbase + wm * GP_RT;
#pragma unroll
    for (int rt = 0; rt < GP_RT; ++rt) {
        const int tile = tile0 + rt;
        const int row0 = tile * 16 + 4 * q;
#pragma unroll
        for (int j = 0; j < GP_TN; ++j) {
            const int tok = t0 + 16 * (wn * GP_TN + j) + c;
            if (tok >= tokens || tile >= tiles) continue;
            const float r = rsv[tok];
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = total[rt][j][k] * r;
            if (out.mode == OUT_SILU) {
#pragma unroll
                for (int k = 0; k < 4; k += 2) {
                    const int row = row0 + k;
                    if (row < rows)
                        reinterpret_cast<float *>(out.y)[(size_t)tok * out.y_stride + (row >> 1)] = silu_f(v[k]) * v[k + 1];
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int row = row0 + k;
                    if (row >= rows) continue;
                    const size_t at = (size_t)tok * out.y_stride + row;
                    if (out.mode == OUT_F32) reinterpret_cast<float *>(out.y)[at] = v[k];
                    else if (out.mode == OUT_ADD) reinterpret_cast<float *>(out.y)[at] += v[k];
                    else {
                        const unsigned uu = __float_as_uint(v[k]);
                        reinterpret_cast<uint16_t *>(out.y)[at] = (uint16_t)(
                            (uu & 0x7fffffffu) > 0x7f800000u ? (uu >> 16) | 0x40u
                                                             : (uu + 0x7fffu + ((uu >> 16) & 1u)) >> 16);
                    }
                }
            }
        }
    }
}

template <int WG, typename ST, int WM, int GS>
static void launch_prompt_wm(marin_gpu *g, const marin_quant_matrix *w, const int8_t *limbs, const float *exps,
                             const float *rs, const GemvOut &out, size_t tokens) {
    using S = GpShape<WM, GS>;
    const int tiles = (int)(w->rows_padded / 16);
    const int row_blocks = (int)((w->rows_padded + S::ROWS - 1) / S::ROWS);
    const int token_blocks = (int)((tokens + GP_TOK - 1) / GP_TOK);
    const unsigned grid = (unsigned)((row_blocks + 7) / 8 * 8 * token_blocks);
    const size_t lds = (size_t)S::STAGES * S::STAGE_BYTES;
    // dynamic LDS above 64 KiB must be allowed for the kernel (a host-side attribute, set on every launch so no
    // process-wide state is kept; a prompt product takes tens of microseconds at least)
    HIP_CHECK(hipFuncSetAttribute((const void *)gemm_prompt<WG, ST, WM, GS>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    gemm_prompt<WG, ST, WM, GS><<<grid, S::THREADS, lds, g->stream>>>(w->codes, (const ST *)w->scales, limbs, exps, rs, out,
                                                                   (int)tokens, (int)w->rows, (int)w->cols, tiles,
                                                                   row_blocks, token_blocks);
}

// 256-row workgroups unless they would cover at most half the compute units, then 128-row ones (two fit a unit)
template <int WG, typename ST>
static void launch_prompt_t(marin_gpu *g, const marin_quant_matrix *w, const int8_t *limbs, const float *exps,
                            const float *rs, const GemvOut &out, size_t tokens) {
    const size_t token_blocks = (tokens + GP_TOK - 1) / GP_TOK;
    const size_t big = (w->rows_padded + GpShape<4, 1>::ROWS - 1) / GpShape<4, 1>::ROWS * token_blocks;
    // 128-row workgroups stage whole groups, two deep (measured faster there: o 74.5 -> 71.2 us, down 194 -> 183 us
    // at 512 tokens); 256-row ones stage single windows, four deep (group stages were slower for them)
    if (2 * big > (size_t)std::max(g->cu_count, 1)) launch_prompt_wm<WG, ST, 4, 1>(g, w, limbs, exps, rs, out, tokens);
    else launch_prompt_wm<WG, ST, 2, WG>(g, w, limbs, exps, rs, out, tokens);
}

bool gemm_layout_ok(const marin_quant_matrix *w) {
    return w->bits == 8 && w->windowed && (w->group == 64 || w->group == 128) && w->cols % w->group == 0;
}

bool gemm_supported(const marin_quant_matrix *w, size_t tokens) {
    return tokens >= GEMM_MIN_TOKENS && gemm_layout_ok(w);
}

template <int WG, typename ST, int TOK>
static void launch_tok(marin_gpu *g, const marin_quant_matrix *w, const int8_t *limbs, const float *exps,
                       const float *rs, const GemvOut &out, size_t tokens) {
    const int tiles = (int)(w->rows_padded / 16);
    const int rows_per_block = GM_WAVES * GM_ROW_TILES * 16;
    dim3 grid((unsigned)((w->rows_padded + rows_per_block - 1) / rows_per_block), (unsigned)((tokens + TOK - 1) / TOK));
    gemm_q8<WG, ST, TOK, false><<<grid, dim3(64 * GM_WAVES * gm_halves(TOK)), 0, g->stream>>>(
        w->codes, (const ST *)w->scales, limbs, exps, rs, out, (int)tokens, (int)w->rows, (int)w->cols, tiles,
        MoePlanView{});
}

template <int WG, typename ST>
static void launch_t(marin_gpu *g, const marin_quant_matrix *w, const int8_t *limbs, const float *exps,
                     const float *rs, const GemvOut &out, size_t tokens) {
    // a decode batch in one token block of 8; prompts in blocks of 32
    if (tokens <= (size_t)MOE_BATCH) launch_tok<WG, ST, MOE_BATCH>(g, w, limbs, exps, rs, out, tokens);
    else if (tokens <= (size_t)GM_TOKENS) launch_tok<WG, ST, GM_TOKENS>(g, w, limbs, exps, rs, out, tokens);
    else launch_tok<WG, ST, 2 * GM_TOKENS>(g, w, limbs, exps, rs, out, tokens);
}

void launch_gemm(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    if (!tokens) return;
    if (!gemm_layout_ok(w)) unsupported("matrix-core GEMM layout (int8, group 64 or 128)", 128, w->group);
    if (out.argmax && !out.argmax_each) unsupported("GEMM greedy choice (one per token only)", 1, 0);
    const size_t cols = w->cols, groups = w->groups();
    const bool prompt = tokens >= GP_MIN_TOKENS && !out.argmax;
    const int nl = prompt ? GP_L : 4;
    // workspace: limbs [tokens][nl][cols] | exps [tokens][groups] | rs [tokens]
    const size_t limb_bytes = (tokens * nl * cols + 15) / 16 * 16;
    const size_t exp_bytes = (tokens * groups * 4 + 15) / 16 * 16;
    uint8_t *ws = (uint8_t *)g->workspace(limb_bytes + exp_bytes + tokens * 4);
    int8_t *limbs = (int8_t *)ws;
    float *exps = (float *)(ws + limb_bytes);
    float *rs = (float *)(ws + limb_bytes + exp_bytes);
    const bool wg2 = w->group == 128;
    if (prompt) {
        if (wg2) quantize_act<128, false, GP_L><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, 0);
        else quantize_act<64, false, GP_L><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, 0);
        g->launched();
        if (w->bf16_scales) {
            if (wg2) launch_prompt_t<2, uint16_t>(g, w, limbs, exps, rs, out, tokens);
            else launch_prompt_t<1, uint16_t>(g, w, limbs, exps, rs, out, tokens);
        } else {
            if (wg2) launch_prompt_t<2, float>(g, w, limbs, exps, rs, out, tokens);
            else launch_prompt_t<1, float>(g, w, limbs, exps, rs, out, tokens);
        }
    } else {
    if (w->group == 128) quantize_act<128, false><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, 0);
    else quantize_act<64, false><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, 0);
    g->launched();
    if (w->bf16_scales) {
        if (wg2) launch_t<2, uint16_t>(g, w, limbs, exps, rs, out, tokens);
        else launch_t<1, uint16_t>(g, w, limbs, exps, rs, out, tokens);
    } else {
        if (wg2) launch_t<2, float>(g, w, limbs, exps, rs, out, tokens);
        else launch_t<1, float>(g, w, limbs, exps, rs, out, tokens);
    }
    }
    const double act = in.mode == IN_BF16 ? 2.0 : 4.0, res = out.mode == OUT_BF16 ? 2.0 : 4.0;
    const double outs = out.mode == OUT_SILU ? (double)w->rows / 2 : (double)w->rows;
    const double bytes = (double)w->rows * w->row_bytes() + (double)w->rows * groups * (w->bf16_scales ? 2 : 4) +
                         (double)tokens * cols * act + (double)tokens * outs * res;
    g->launched(marin_gpu::GEMV, bytes, prompt ? "gemm_prompt" : "gemm_q8");
}

static size_t align16(size_t n) { return (n + 15) / 16 * 16; }

size_t moe_gate_up_workspace(size_t tokens, size_t cols, size_t group) {
    return align16(tokens * 4 * cols) + align16(tokens * (cols / group) * 4) + align16(tokens * (cols / group) * 16) +
           tokens * 4;
}

ActLimbs launch_quantize_act(marin_gpu *g, const GemvIn &in, size_t tokens, size_t cols, size_t group, bool frag) {
    // fragment order pads the tokens to whole tiles of 4 (the padding is never read: lanes of missing tokens read a
    // real token's fragment)
    const size_t ttiles = (tokens + 3) / 4;
    const size_t limb_bytes = align16((frag ? ttiles * 4 : tokens) * 4 * cols), exp_bytes = align16(tokens * (cols / group) * 4);
    uint8_t *ws = (uint8_t *)g->workspace(moe_gate_up_workspace(frag ? ttiles * 4 : tokens, cols, group));
    int8_t *limbs = (int8_t *)ws;
    float *exps = (float *)(ws + limb_bytes);
    int32_t *lsum = (int32_t *)(ws + limb_bytes + exp_bytes);
    float *rs = (float *)(ws + limb_bytes + exp_bytes + align16(tokens * (cols / group) * 16));
    const unsigned tt = (unsigned)ttiles;
    if (frag && in.mode != IN_NORM) {
        // no norm statistic: one workgroup per (token, 4096 columns)
        const dim3 grid((unsigned)tokens, (unsigned)((cols + 4095) / 4096));
        if (group == 128) quantize_rows<128, 1><<<grid, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt);
        else quantize_rows<64, 1><<<grid, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt);
        g->launched();
        return ActLimbs{limbs, exps, rs, lsum};
    }
    if (frag && cols <= 4 * 4096) {
        const unsigned nt = (unsigned)tokens;
        const int it = (int)((cols + 4095) / 4096);
        if (group == 128) {
            switch (it) {
                case 1: quantize_rows<128, 1><<<nt, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt); break;
                case 2: quantize_rows<128, 2><<<nt, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt); break;
                case 3: quantize_rows<128, 3><<<nt, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt); break;
                default: quantize_rows<128, 4><<<nt, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt); break;
            }
        } else {
            switch (it) {
                case 1: quantize_rows<64, 1><<<nt, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt); break;
                case 2: quantize_rows<64, 2><<<nt, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt); break;
                case 3: quantize_rows<64, 3><<<nt, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt); break;
                default: quantize_rows<64, 4><<<nt, QR_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, lsum, tt); break;
            }
        }
        g->launched();
        return ActLimbs{limbs, exps, rs, lsum};
    }
    if (group == 128) {
        if (frag) quantize_act<128, true><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, tt);
        else quantize_act<128, false><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, tt);
    } else {
        if (frag) quantize_act<64, true><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, tt);
        else quantize_act<64, false><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, tt);
    }
    g->launched();
    return ActLimbs{limbs, exps, rs, nullptr};
}

template <int WG, typename ST>
static void launch_moe_t(marin_gpu *g, const marin_quant_matrix *w, const int8_t *limbs, const float *exps,
                         const float *rs, size_t tokens, const MoePlanView &plan, size_t max_experts, float *act) {
    const int tiles = 2 * plan.ffn / 16;  // one expert's tiles
    const int rows_per_block = GM_WAVES * GM_ROW_TILES * 16;
    dim3 grid((unsigned)((2 * plan.ffn + rows_per_block - 1) / rows_per_block), (unsigned)max_experts);
    GemvOut out;
    out.mode = OUT_SILU;
    out.y = act;
    gemm_q8<WG, ST, MOE_BATCH, true><<<grid, dim3(64 * GM_WAVES), 0, g->stream>>>(
        w->codes, (const ST *)w->scales, limbs, exps, rs, out, (int)tokens, 2 * plan.ffn, (int)w->cols, tiles, plan);
}

void launch_moe_gate_up(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, size_t tokens,
                        const int32_t *plan, size_t max_experts, size_t k, size_t ffn, float *act) {
    if (tokens < 1 || tokens > (size_t)MOE_BATCH) unsupported("tokens of a grouped expert batch", MOE_BATCH, tokens);
    if (max_experts > (size_t)MOE_PLAN_MAX) unsupported("distinct experts of a batch", MOE_PLAN_MAX, max_experts);
    if (w->bits != 8 || !w->windowed || !(w->group == 64 || w->group == 128) || w->cols % w->group)
        unsupported("grouped expert layout (int8, group 64 or 128)", 128, w->group);
    const size_t cols = w->cols, groups = w->groups();
    const size_t limb_bytes = align16(tokens * 4 * cols), exp_bytes = align16(tokens * groups * 4);
    uint8_t *ws = (uint8_t *)g->workspace(moe_gate_up_workspace(tokens, cols, w->group));
    int8_t *limbs = (int8_t *)ws;
    float *exps = (float *)(ws + limb_bytes);
    float *rs = (float *)(ws + limb_bytes + exp_bytes);
    if (w->group == 128) quantize_act<128, false><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, 0);
    else quantize_act<64, false><<<qa_grid(tokens, cols), QA_THREADS, 0, g->stream>>>(in, (int)cols, limbs, exps, rs, 0);
    g->launched();
    MoePlanView pv;
    pv.plan = plan;
    pv.k = (int)k;
    pv.ffn = (int)ffn;
    const bool wg2 = w->group == 128;
    if (w->bf16_scales) {
        if (wg2) launch_moe_t<2, uint16_t>(g, w, limbs, exps, rs, tokens, pv, max_experts, act);
        else launch_moe_t<1, uint16_t>(g, w, limbs, exps, rs, tokens, pv, max_experts, act);
    } else {
        if (wg2) launch_moe_t<2, float>(g, w, limbs, exps, rs, tokens, pv, max_experts, act);
        else launch_moe_t<1, float>(g, w, limbs, exps, rs, tokens, pv, max_experts, act);
    }
}

void launch_product(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    if (!tokens) return;
    if (gemv_batch_supported(w, tokens) && (!out.argmax || out.argmax_each)) {
        launch_gemv_batch(g, w, in, out, tokens);
        return;
    }
    if ((gemm_supported(w, tokens) && !out.argmax) || (out.argmax_each && gemm_layout_ok(w))) {
        launch_gemm(g, w, in, out, tokens);
        return;
    }
    const size_t in_es = in.mode == IN_BF16 ? 2 : 4, out_es = out.mode == OUT_BF16 ? 2 : 4;
    for (size_t t0 = 0; t0 < tokens; t0 += GEMV_TOKENS) {
        const size_t nt = std::min<size_t>(GEMV_TOKENS, tokens - t0);
        GemvIn i2 = in;
        i2.x = (const uint8_t *)in.x + t0 * in.x_stride * in_es;
        GemvOut o2 = out;
        o2.y = (uint8_t *)out.y + t0 * out.y_stride * out_es;
        launch_gemv(g, w, i2, o2, nt);
    }
}

}  // namespace marin
