// Prompt attention on the matrix cores (the FA-style prefill path; the reference's attention_mma.cu covers the same
// step on NVIDIA tensor cores): one sequence, 16 or more new tokens, f16 keys and values.
//
// fa_prep: per (token, kv head), the group's q heads get RMSNorm(q_norm) + RoPE (or are taken as given), are scaled by
// a power of two 2^s per row (largest magnitude in [2^14, 2^15)) and split into two f16 parts, q 2^s = hi + lo (about
// 22 significant bits); with the fused inputs the token's key gets RMSNorm(k_norm) + RoPE and is stored with its
// value into the cache, rounded as every cache store.
//
// fa_prefill: a workgroup per (16 query tokens, kv head, span of 1024 positions when the context is longer), a wave
// per q head of the group. Key and value tiles of 64
// positions are staged in LDS once for the whole group (keys position-major, values transposed), the next tile's
// loads in flight while the current one is used. Per tile and wave: S = Q K^T on v_mfma_f32_16x16x32_f16 (hi and lo
// parts: keys are exact in f16, so the scores are f32-grade), causal mask, online softmax in the log2 domain with the
// row's 2^-s folded into the scale, P through LDS into the A layout split into hi + lo, O += P V on the same MFMA with
// the transposed values. Rows divide by their running sum at the end, or, split over spans, leave the running maximum,
// sum and values for fa_merge (so no workgroup walks a whole long context alone).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "attention.hpp"

namespace marin {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int FA_ROWS = 16;  // query tokens per workgroup (one MFMA's rows)

// Reductions over a row of 16 lanes with DPP (quad swaps, then the half-row and row mirrors): every step pairs lanes
// symmetrically, so all 16 lanes end with the same value (a + b and b + a round alike).
template <int CTRL>
__device__ __forceinline__ float fa_dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, fa_dpp<0xB1>(v));   // lanes xor 1
    v = fmaxf(v, fa_dpp<0x4E>(v));   // lanes xor 2
    v = fmaxf(v, fa_dpp<0x141>(v));  // half-row mirror (the other quad of 8 lanes)
    return fmaxf(v, fa_dpp<0x140>(v));  // row mirror (the other 8 lanes)
}
__device__ __forceinline__ float row16_sum(float v) {
    v += fa_dpp<0xB1>(v);
    v += fa_dpp<0x4E>(v);
    v += fa_dpp<0x141>(v);
    return v + fa_dpp<0x140>(v);
}
constexpr int FA_TILE = 64;  // positions per tile: FA_TILE / 16 score blocks, FA_TILE / 32 MFMA k-steps of P V
static_assert(FA_TILE % 32 == 0, "whole k-steps of P V");

// RMSNorm(weight) + RoPE of one head by one wave, as in the decode kernels: lane i holds the pairs (i, i + hd/2).
__device__ __forceinline__ void fa_norm_rope(const float *__restrict__ src, const float *__restrict__ w,
                                             const float *__restrict__ freq, uint32_t pos, int hd, float eps, int lane,
                                             float a[2], float b[2]) {
    const int half = hd / 2;
    float x[2], y[2], s = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = lane + 64 * k;
        x[k] = i < half ? src[i] : 0.0f;
        y[k] = i < half ? src[i + half] : 0.0f;
        s += x[k] * x[k] + y[k] * y[k];
    }
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    const float scale = 1.0f / sqrtf(s / (float)hd + eps);
    const float position = (float)pos;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = lane + 64 * k;
        a[k] = b[k] = 0.0f;
        if (i >= half) continue;
        const float xa = x[k] * scale * w[i], yb = y[k] * scale * w[i + half];
        float sn, cs;
        sincosf(position * freq[i], &sn, &cs);
        a[k] = xa * cs - yb * sn;
        b[k] = yb * cs + xa * sn;
    }
}

__device__ __forceinline__ void store_f16(uint8_t *row, int e, float x) {
    const float c = fminf(fmaxf(x, -65504.0f), 65504.0f);
    reinterpret_cast<_Float16 *>(row)[e] = (_Float16)(x != x ? x : c);
}

}  // namespace

// grid (tokens, kv_heads); waves 0..group-1 take the group's q heads, wave `group` the token's key and value.
// qh/ql: [tokens][heads][hd] f16 parts; qe: [tokens][heads] the rows' 2^-s.
template <bool BF16IN>
__global__ __launch_bounds__(576) void fa_prep(const void *__restrict__ qv, AttnFuse fuse,
                                               const uint64_t *__restrict__ table, const uint32_t *__restrict__ ctx_lens,
                                               KvGeom geom, int tokens, int heads, int kv_heads,
                                               _Float16 *__restrict__ qh, _Float16 *__restrict__ ql,
                                               float *__restrict__ qe) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x, kvh = blockIdx.y;
    const int hd = (int)geom.head_dim, half = hd / 2, group = heads / kv_heads;
    const int pos = (int)ctx_lens[0] - tokens + t;
    const size_t qkv_stride = (size_t)(heads + 2 * kv_heads) * hd;
    if (wave < group) {
        const int h = kvh * group + wave;
        float a[2], b[2];
        if (fuse.qkv) {
            fa_norm_rope(fuse.qkv + (size_t)t * qkv_stride + (size_t)h * hd, fuse.q_norm, fuse.freq, (uint32_t)pos, hd,
                         fuse.eps, lane, a, b);
        } else {
            const size_t base = ((size_t)t * heads + h) * hd;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int i = lane + 64 * k;
                a[k] = b[k] = 0.0f;
                if (i >= half) continue;
                if constexpr (BF16IN) {
                    const uint16_t *q16 = reinterpret_cast<const uint16_t *>(qv);
                    a[k] = __uint_as_float((unsigned)q16[base + i] << 16);
                    b[k] = __uint_as_float((unsigned)q16[base + i + half] << 16);
                } else {
                    a[k] = reinterpret_cast<const float *>(qv)[base + i];
                    b[k] = reinterpret_cast<const float *>(qv)[base + i + half];
                }
            }
        }
        float mx = fmaxf(fmaxf(fabsf(a[0]), fabsf(a[1])), fmaxf(fabsf(b[0]), fabsf(b[1])));
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        int sh = 0;
        if (mx > 0.0f && mx < INFINITY) {
            int e;
            (void)frexpf(mx, &e);
            sh = 15 - e;  // largest magnitude lands in [2^14, 2^15)
            sh = sh > 100 ? 100 : (sh < -100 ? -100 : sh);
        }
        const float up = ldexpf(1.0f, sh);
        const size_t row = ((size_t)t * heads + h) * hd;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = lane + 64 * k;
            if (i >= half) continue;
            const float va = a[k] * up, vb = b[k] * up;
            const _Float16 ha = (_Float16)va, hb = (_Float16)vb;
            qh[row + i] = ha;
            qh[row + i + half] = hb;
            ql[row + i] = (_Float16)(va - (float)ha);
            ql[row + i + half] = (_Float16)(vb - (float)hb);
        }
        if (lane == 0) qe[(size_t)t * heads + h] = ldexpf(1.0f, -sh);
    } else if (wave == group && fuse.qkv) {
        const uint64_t page = table[pos >> geom.page_shift] + geom.layer_offset + (uint64_t)kvh * geom.head_bytes +
                              (uint64_t)(pos & ((1 << geom.page_shift) - 1)) * hd * 2;
        uint8_t *krow = reinterpret_cast<uint8_t *>(page);
        uint8_t *vrow = reinterpret_cast<uint8_t *>(page + geom.value_offset);
        float a[2], b[2];
        fa_norm_rope(fuse.qkv + (size_t)t * qkv_stride + (size_t)(heads + kvh) * hd, fuse.k_norm, fuse.freq,
                     (uint32_t)pos, hd, fuse.eps, lane, a, b);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = lane + 64 * k;
            if (i < half) {
                store_f16(krow, i, a[k]);
                store_f16(krow, i + half, b[k]);
            }
        }
        const float *vsrc = fuse.qkv + (size_t)t * qkv_stride + (size_t)(heads + kv_heads + kvh) * hd;
        for (int i = lane; i < hd; i += 64) store_f16(vrow, i, vsrc[i]);
    }
}

// HD: head size (64 or 128); G: waves = q heads per kv head (1, 2, 4 or 8); RQ: 16-token row tiles per wave (every
// key and value fragment read from LDS feeds RQ MFMAs, and a tile staged once serves 16 RQ tokens).
// span 0: the workgroup walks every visible position and writes the output. span > 0 (a multiple of FA_TILE): split
// blockIdx.z takes positions [z span, (z + 1) span) and leaves its rows' running maximum, sum and weighted values in
// `part` ([splits][tokens][heads][HD] values, then [splits][tokens][heads] (max, sum)); fa_merge combines them.
template <int HD, int G, bool BF16IO, int RQ>
__global__ __launch_bounds__(64 * G) void fa_prefill(const _Float16 *__restrict__ qh, const _Float16 *__restrict__ ql,
                                                  const float *__restrict__ qe, const uint64_t *__restrict__ table,
                                                  const uint32_t *__restrict__ ctx_lens, KvGeom geom, int tokens,
                                                  int heads, int kv_heads, float scale, int span,
                                                  float *__restrict__ part, void *__restrict__ out) {
    constexpr int KP = HD + 8;        // key row pitch (halves): rows 16 bytes apart in banks
    constexpr int VP = FA_TILE + 8;   // transposed value row pitch (halves)
    constexpr int CH = HD / 8;        // 16-byte chunks per row
    constexpr int KK = HD / 32;       // MFMAs along the head for one score block
    constexpr int DT = HD / 16;       // output tiles of 16 head values
    constexpr int ROWS = FA_ROWS * RQ;
    constexpr int TB = FA_TILE / 16;  // 16-position score blocks per tile
    constexpr int KS = FA_TILE / 32;  // k-steps of 32 positions for P V
    __shared__ __align__(16) _Float16 kt[FA_TILE][KP];
    __shared__ __align__(16) _Float16 vt[HD][VP];
    __shared__ __align__(16) float pl[G][ROWS][FA_TILE + 4];
    constexpr int NT = 64 * G;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, q = lane >> 4;
    const int kvh = blockIdx.y, h = kvh * G + wave;
    const int t0 = blockIdx.x * ROWS;
    const int ctx = (int)ctx_lens[0];
    const int base_pos = ctx - tokens;  // position of token 0
    const int last_row = min(t0 + ROWS - 1, tokens - 1);
    const int max_pos = base_pos + last_row;  // the workgroup's last visible position
    const uint64_t head_off = geom.layer_offset + (uint64_t)kvh * geom.head_bytes;
    const uint32_t pmask = (1u << geom.page_shift) - 1u;

    // A operands of Q (rows = 16 tokens of row tile r, this wave's head): lane row c, head values 32 kk + 8 q .. + 8
    halfx8 aq_h[RQ][KK], aq_l[RQ][KK];
#pragma unroll
    for (int r = 0; r < RQ; ++r) {
        const int t = min(t0 + 16 * r + c, tokens - 1);
        const size_t row = ((size_t)t * heads + h) * HD;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            aq_h[r][kk] = *reinterpret_cast<const halfx8 *>(qh + row + 32 * kk + 8 * q);
            aq_l[r][kk] = *reinterpret_cast<const halfx8 *>(ql + row + 32 * kk + 8 * q);
        }
    }
    // the C layout's rows 4 q + i of each row tile: their tokens' positions and scale factors (scale x 2^-s, log2
    // domain)
    int rpos[RQ][4];
    float rsc[RQ][4];
#pragma unroll
    for (int r = 0; r < RQ; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = t0 + 16 * r + 4 * q + i;
            rpos[r][i] = t < tokens ? base_pos + t : -1;  // rows past the prompt see nothing
            rsc[r][i] = scale * qe[(size_t)min(t, tokens - 1) * heads + h];
        }

    // staging of one tile: chunk j of the tile (key or value row chunk), positions clamped to the visible ones.
    // TRV (when the threads divide them evenly): the value chunks go in units of VPU (4, else 2) consecutive
    // positions x 8 head values per thread, transposed in registers and stored as 8 rows of VPU halves (8- or 4-byte
    // stores) instead of 8 single halves per chunk.
    constexpr int CHUNKS = 2 * FA_TILE * CH;
    constexpr int SLOTS = (CHUNKS + NT - 1) / NT;
    constexpr int KCH = FA_TILE * CH;  // key chunks
    constexpr int VPU = (KCH / 4) % NT == 0 ? 4 : 2, VU = KCH / VPU;  // positions per value unit, value units
    constexpr bool TRV = KCH % NT == 0 && VU % NT == 0;
    constexpr int KPT = KCH / NT, VPT = VU / NT;  // (TRV) key chunks and value units per thread
    u32x4 stage[SLOTS];
    auto load_chunk = [&](int which, int r, int ch, int p0) {
        const uint32_t pos = (uint32_t)min(p0 + r, max_pos);
        const uint64_t page = table[pos >> geom.page_shift] + head_off + (which ? geom.value_offset : 0) +
                              (uint64_t)(pos & pmask) * HD * 2;
        return *reinterpret_cast<const u32x4 *>(reinterpret_cast<const uint8_t *>(page) + 16 * ch);
    };
    auto load_tile = [&](int p0) {
        if constexpr (TRV) {
#pragma unroll
            for (int s = 0; s < KPT; ++s) {
                const int j = (int)threadIdx.x + s * NT;
                stage[s] = load_chunk(0, j / CH, j % CH, p0);
            }
#pragma unroll
            for (int v = 0; v < VPT; ++v) {
                const int u = (int)threadIdx.x + v * NT, ch = u / (FA_TILE / VPU), pg = u % (FA_TILE / VPU);
#pragma unroll
                for (int k = 0; k < VPU; ++k) stage[KPT + VPU * v + k] = load_chunk(1, VPU * pg + k, ch, p0);
            }
        } else {
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const int j = min((int)threadIdx.x + s * NT, CHUNKS - 1);  // clamped: the loads stay unconditional
                stage[s] = load_chunk(j / (FA_TILE * CH), (j / CH) % FA_TILE, j % CH, p0);
            }
        }
    };
    auto store_tile = [&]() {
        if constexpr (TRV) {
#pragma unroll
            for (int s = 0; s < KPT; ++s) {
                const int j = (int)threadIdx.x + s * NT;
                *reinterpret_cast<u32x4 *>(&kt[j / CH][8 * (j % CH)]) = stage[s];
            }
#pragma unroll
            for (int v = 0; v < VPT; ++v) {
                const int u = (int)threadIdx.x + v * NT, ch = u / (FA_TILE / VPU), pg = u % (FA_TILE / VPU);
                const u32x4 *c4 = &stage[KPT + VPU * v];  // positions VPU pg .. + VPU - 1, head values 8 ch .. + 7
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int w = e / 2;
                    auto pair = [&](const u32x4 &a, const u32x4 &b) {  // half e of a (low), of b (high)
                        return (e & 1) ? (a[w] >> 16) | (b[w] & 0xffff0000u) : (a[w] & 0xffffu) | (b[w] << 16);
                    };
                    if constexpr (VPU == 4)
                        *reinterpret_cast<uint2 *>(&vt[8 * ch + e][4 * pg]) =
                            make_uint2(pair(c4[0], c4[1]), pair(c4[2], c4[3]));
                    else
                        *reinterpret_cast<uint32_t *>(&vt[8 * ch + e][2 * pg]) = pair(c4[0], c4[1]);
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const int j = (int)threadIdx.x + s * NT;
                if (j >= CHUNKS) continue;
                const int which = j / (FA_TILE * CH), r = (j / CH) % FA_TILE, ch = j % CH;
                if (which == 0) {
                    *reinterpret_cast<u32x4 *>(&kt[r][8 * ch]) = stage[s];
                } else {
                    const halfx8 v = __builtin_bit_cast(halfx8, stage[s]);
#pragma unroll
                    for (int e = 0; e < 8; ++e) vt[8 * ch + e][r] = v[e];
                }
            }
        }
    };

    floatx4 o[RQ][DT];
    float m[RQ][4], l[RQ][4];
#pragma unroll
    for (int r = 0; r < RQ; ++r) {
#pragma unroll
        for (int d = 0; d < DT; ++d) o[r][d] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            m[r][i] = -INFINITY;
            l[r][i] = 0.0f;
        }
    }

    const int p_begin = span ? (int)blockIdx.z * span : 0;
    const int p_end = span ? min(p_begin + span, max_pos + 1) : max_pos + 1;  // exclusive
    load_tile(min(p_begin, max_pos));
    for (int p0 = p_begin; p0 < p_end; p0 += FA_TILE) {
        __syncthreads();  // every wave is done with the previous tile
        store_tile();
        __syncthreads();
        load_tile(min(p0 + FA_TILE, max_pos));  // past the last tile: a harmless reload of the last positions

        // ---- scores: two 16-position blocks per row tile, hi and lo parts of q; each key fragment feeds RQ tiles
        floatx4 s[RQ][TB];
#pragma unroll
        for (int j = 0; j < TB; ++j) {
#pragma unroll
            for (int r = 0; r < RQ; ++r) s[r][j] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                const halfx8 bk = *reinterpret_cast<const halfx8 *>(&kt[16 * j + c][32 * kk + 8 * q]);
#pragma unroll
                for (int r = 0; r < RQ; ++r) {
                    s[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq_h[r][kk], bk, s[r][j], 0, 0, 0);
                    s[r][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq_l[r][kk], bk, s[r][j], 0, 0, 0);
                }
            }
        }
        // ---- online softmax of rows 4 q + i over this tile's positions (column c of block j: position p0 + 16 j + c)
#pragma unroll
        for (int r = 0; r < RQ; ++r) {
            float alpha[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float mx = -INFINITY;
#pragma unroll
                for (int j = 0; j < TB; ++j) {
                    const int pos = p0 + 16 * j + c;
                    const float v = pos <= rpos[r][i] ? s[r][j][i] * rsc[r][i] : -INFINITY;
                    s[r][j][i] = v;
                    mx = fmaxf(mx, v);
                }
                mx = row16_max(mx);
                const float mn = fmaxf(m[r][i], mx);
                alpha[i] = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[r][i] - mn);
                float sum = 0.0f;
#pragma unroll
                for (int j = 0; j < TB; ++j) {
                    const float p = s[r][j][i] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s[r][j][i] - mn);
                    s[r][j][i] = p;
                    sum += p;
                }
                sum = row16_sum(sum);
                l[r][i] = l[r][i] * alpha[i] + sum;
                m[r][i] = mn;
            }
#pragma unroll
            for (int d = 0; d < DT; ++d)
#pragma unroll
                for (int i = 0; i < 4; ++i) o[r][d][i] *= alpha[i];
            // P into the A layout (lane row c, positions 8 q .. + 8) through this wave's LDS tile
#pragma unroll
            for (int j = 0; j < TB; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) pl[wave][16 * r + 4 * q + i][16 * j + c] = s[r][j][i];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // the wave's own LDS stores complete (lgkmcnt 0) before they are read
        __builtin_amdgcn_wave_barrier();
        halfx8 ph[RQ][KS], plo[RQ][KS];
#pragma unroll
        for (int r = 0; r < RQ; ++r)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float p = pl[wave][16 * r + c][32 * ks + 8 * q + e];
                    const _Float16 hi = (_Float16)p;
                    ph[r][ks][e] = hi;
                    plo[r][ks][e] = (_Float16)(p - (float)hi);
                }
        // ---- O += P V: B operand lane column = head value 16 d + c, positions 8 q .. + 8 (transposed values)
#pragma unroll
        for (int d = 0; d < DT; ++d) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const halfx8 bv = *reinterpret_cast<const halfx8 *>(&vt[16 * d + c][32 * ks + 8 * q]);
#pragma unroll
                for (int r = 0; r < RQ; ++r) {
                    o[r][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ph[r][ks], bv, o[r][d], 0, 0, 0);
                    o[r][d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(plo[r][ks], bv, o[r][d], 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();  // reads of pl done before the next tile overwrites it
    }
    if (span) {
        // ---- this split's rows: running maximum and sum, unnormalized values (a split past a row's last position
        // leaves -inf, 0 and zeros)
        const size_t plane = (size_t)tokens * heads;
        float *ml = part + (size_t)gridDim.z * plane * HD;
#pragma unroll
        for (int r = 0; r < RQ; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + 16 * r + 4 * q + i;
                if (t >= tokens) continue;
                const size_t unit = (size_t)blockIdx.z * plane + (size_t)t * heads + h;
#pragma unroll
                for (int d = 0; d < DT; ++d) part[unit * HD + 16 * d + c] = o[r][d][i];
                if (c == 0) *reinterpret_cast<float2 *>(ml + unit * 2) = make_float2(m[r][i], l[r][i]);
            }
        return;
    }
    // ---- out: lane holds rows 4 q + i of each row tile, head value 16 d + c
#pragma unroll
    for (int r = 0; r < RQ; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = t0 + 16 * r + 4 * q + i;
            if (t >= tokens) continue;
            const float inv = 1.0f / l[r][i];
            const size_t row = ((size_t)t * heads + h) * HD;
#pragma unroll
            for (int d = 0; d < DT; ++d) {
                const float v = o[r][d][i] * inv;
                if constexpr (BF16IO) {
                    const unsigned u = __float_as_uint(v);
                    reinterpret_cast<uint16_t *>(out)[row + 16 * d + c] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
                } else {
                    reinterpret_cast<float *>(out)[row + 16 * d + c] = v;
                }
            }
        }
}

// The splits of every (token, head) row combined in split order: weights 2^(m_s - M) of the rows' maxima (log2
// domain), values summed and divided by the weighted sums. One thread per head value, a workgroup per row.
template <int HD, bool BF16IO>
__global__ __launch_bounds__(HD) void fa_merge(const float *__restrict__ part, int splits, int tokens, int heads,
                                               void *__restrict__ out) {
    const size_t unit = blockIdx.x, plane = (size_t)tokens * heads;
    const float *ml = part + (size_t)splits * plane * HD;
    float mx = -INFINITY;
    for (int z = 0; z < splits; ++z) mx = fmaxf(mx, ml[((size_t)z * plane + unit) * 2]);
    float sum = 0.0f, v = 0.0f;
    for (int z = 0; z < splits; ++z) {
        const float2 s = *reinterpret_cast<const float2 *>(ml + ((size_t)z * plane + unit) * 2);
        const float w = s.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(s.x - mx);
        sum += s.y * w;
        v += part[((size_t)z * plane + unit) * HD + threadIdx.x] * w;
    }
    v /= sum;
    const size_t at = unit * HD + threadIdx.x;
    if constexpr (BF16IO) {
        const unsigned u = __float_as_uint(v);
        reinterpret_cast<uint16_t *>(out)[at] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    } else {
        reinterpret_cast<float *>(out)[at] = v;
    }
}

size_t prefill_fa_scratch(size_t tokens, size_t heads, size_t hd) { return tokens * heads * (hd * 4 + 4); }

constexpr int FA_SPAN = 1024;   // positions per split of a long row
constexpr int FA_MAX_SPLITS = 8;

// Splits of the rows' positions: one when the context fits a span or the scratch cannot hold the partials.
static int fa_splits(const AttentionArgs &a) {
    const size_t hd = a.geom.head_dim;
    const size_t s = std::min<size_t>((a.max_ctx + FA_SPAN - 1) / FA_SPAN, FA_MAX_SPLITS);
    if (s <= 1) return 1;
    const size_t need = (prefill_fa_scratch(a.tokens, a.heads, hd) + 15) / 16 * 16 + s * a.tokens * a.heads * (hd + 2) * 4;
    return need <= a.partial_floats * 4 ? (int)s : 1;
}

bool prefill_fa_fits(const AttentionArgs &a) {
    const size_t hd = a.geom.head_dim, group = a.heads / a.kv_heads;
    return a.batch == 1 && a.tokens >= FA_ROWS && a.geom.format == MARIN_KV_F16 && (hd == 64 || hd == 128) &&
           (group == 1 || group == 2 || group == 4 || group == 8) &&
           a.partial_floats * 4 >= prefill_fa_scratch(a.tokens, a.heads, hd);
}

constexpr int FA_RQ = 1;  // 16-token row tiles per wave (2 measured slower: one wave per SIMD from its registers)

template <int HD, int G>
static void launch_fa_t(marin_gpu *g, const AttentionArgs &a, const _Float16 *qh, const _Float16 *ql, const float *qe,
                        float scale, int splits, float *part) {
    dim3 grid((unsigned)((a.tokens + FA_ROWS * FA_RQ - 1) / (FA_ROWS * FA_RQ)), (unsigned)a.kv_heads, (unsigned)splits);
    const int span = splits > 1 ? FA_SPAN : 0;
    if (a.bf16_io)
        fa_prefill<HD, G, true, FA_RQ><<<grid, 64 * G, 0, g->stream>>>(qh, ql, qe, a.tables, a.ctx, a.geom, (int)a.tokens,
                                                                       (int)a.heads, (int)a.kv_heads, scale, span, part, a.out);
    else
        fa_prefill<HD, G, false, FA_RQ><<<grid, 64 * G, 0, g->stream>>>(qh, ql, qe, a.tables, a.ctx, a.geom, (int)a.tokens,
                                                                        (int)a.heads, (int)a.kv_heads, scale, span, part, a.out);
    if (splits > 1) {
        g->launched(marin_gpu::ATTENTION, a.bytes_hint, "fa_prefill");
        const unsigned rows = (unsigned)(a.tokens * a.heads);
        if (a.bf16_io) fa_merge<HD, true><<<rows, HD, 0, g->stream>>>(part, splits, (int)a.tokens, (int)a.heads, a.out);
        else fa_merge<HD, false><<<rows, HD, 0, g->stream>>>(part, splits, (int)a.tokens, (int)a.heads, a.out);
    }
}

template <int HD>
static void launch_fa_hd(marin_gpu *g, const AttentionArgs &a, const _Float16 *qh, const _Float16 *ql,
                         const float *qe, float scale, int splits, float *part) {
    switch (a.heads / a.kv_heads) {
        case 1: launch_fa_t<HD, 1>(g, a, qh, ql, qe, scale, splits, part); break;
        case 2: launch_fa_t<HD, 2>(g, a, qh, ql, qe, scale, splits, part); break;
        case 4: launch_fa_t<HD, 4>(g, a, qh, ql, qe, scale, splits, part); break;
        default: launch_fa_t<HD, 8>(g, a, qh, ql, qe, scale, splits, part); break;
    }
}

void launch_prefill_fa(marin_gpu *g, const AttentionArgs &a) {
    const int hd = (int)a.geom.head_dim, group = (int)(a.heads / a.kv_heads);
    // q parts in the partial-record scratch: hi [tokens][heads][hd] f16, lo likewise, then the rows' 2^-s
    _Float16 *qh = reinterpret_cast<_Float16 *>(a.partials);
    _Float16 *ql = qh + a.tokens * a.heads * hd;
    float *qe = reinterpret_cast<float *>(ql + a.tokens * a.heads * hd);
    dim3 pgrid((unsigned)a.tokens, (unsigned)a.kv_heads);
    const int pthreads = 64 * (group + 1);
    if (a.bf16_io && !a.fuse.qkv)
        fa_prep<true><<<pgrid, pthreads, 0, g->stream>>>(a.q, a.fuse, a.tables, a.ctx, a.geom, (int)a.tokens,
                                                          (int)a.heads, (int)a.kv_heads, qh, ql, qe);
    else
        fa_prep<false><<<pgrid, pthreads, 0, g->stream>>>(a.q, a.fuse, a.tables, a.ctx, a.geom, (int)a.tokens,
                                                           (int)a.heads, (int)a.kv_heads, qh, ql, qe);
    g->launched();
    const float scale = (float)(1.4426950408889634 / std::sqrt((double)hd));
    // split partials after the q parts
    const int splits = fa_splits(a);
    float *part = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(a.partials) +
                                            (prefill_fa_scratch(a.tokens, a.heads, hd) + 15) / 16 * 16);
    if (hd == 128) launch_fa_hd<128>(g, a, qh, ql, qe, scale, splits, part);
    else launch_fa_hd<64>(g, a, qh, ql, qe, scale, splits, part);
    if (splits > 1) g->launched(marin_gpu::OTHER, 0.0, "fa_merge");
    else g->launched(marin_gpu::ATTENTION, a.bytes_hint, "fa_prefill");
}

}  // namespace marin
