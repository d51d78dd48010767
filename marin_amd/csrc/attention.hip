// Paged KV cache and grouped-query decode attention on CDNA4 (crates/cuda/src/kv.rs, pages.rs, attention.rs and
// attention.cu of the reference, redesigned).
//
// Attention splits the visible context into chunks; a workgroup takes one chunk of one kv head for up to 8 query rows
// (the heads sharing that kv head, times the new tokens). Lanes are grouped per position: a group of LPP lanes covers
// one position's head with 8 contiguous values per lane (16-byte loads for bf16/f16), so a wave reads 64/LPP rows of
// a page per step and each key or value row is read once for all the rows of the group. Keys and values are read in
// the same pass with an online softmax; the chunks of a row group are merged (log-sum-exp) by the last of them to
// finish, in the same launch.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "attention.hpp"

namespace marin {

size_t kv_elem_bytes(marin_kv_format f) { return f == MARIN_KV_F32 ? 4 : 2; }

constexpr int ROWS = 8;         // query rows per workgroup
constexpr int MAX_CHUNK = 256;  // positions per workgroup
constexpr int MIN_CHUNK = 32;
constexpr int MAX_SPLITS = 256;  // chunks of one context: two merge levels of at most 16

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((unsigned)b << 16); }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
typedef __attribute__((address_space(1))) const uint32_t g_u32;
typedef __attribute__((address_space(1))) const uint16_t g_u16;

// Eight values of a key or value row as stored (f32: two 16-byte words, f16/bf16: one). Page addresses are plain
// integers; the loads go through global-address-space pointers so they are counted as vector-memory loads only.
template <int F>
struct Raw8 {
    u32x4 w[F == MARIN_KV_F32 ? 2 : 1];
};

// Values d .. d + 7 of a row (VEC: d + 8 <= head_dim and 16-byte aligned; else element by element, zero past hd).
// NT: nontemporal (streaming) loads, for rows read once per launch.
template <int F, bool VEC, bool NT = false>
__device__ __forceinline__ void load_raw(const uint8_t *row, int d, int hd, Raw8<F> &r) {
    constexpr int ES = F == MARIN_KV_F32 ? 4 : 2;
    const uintptr_t base = (uintptr_t)row + (uintptr_t)d * ES;
    if constexpr (VEC && NT) {
        r.w[0] = __builtin_nontemporal_load((g_u32x4 *)base);
        if constexpr (F == MARIN_KV_F32) r.w[1] = __builtin_nontemporal_load((g_u32x4 *)(base + 16));
    } else if constexpr (VEC) {
        r.w[0] = *(g_u32x4 *)base;
        if constexpr (F == MARIN_KV_F32) r.w[1] = *(g_u32x4 *)(base + 16);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t x = 0;
            if (d + i < hd) x = F == MARIN_KV_F32 ? *(g_u32 *)(base + 4 * i) : (uint32_t) * (g_u16 *)(base + 2 * i);
            if constexpr (F == MARIN_KV_F32) {
                r.w[i / 4][i % 4] = x;
            } else {
                if (i % 2 == 0) r.w[0][i / 2] = x;
                else r.w[0][i / 2] |= x << 16;
            }
        }
    }
}

// Sum over aligned groups of N lanes (N = 1, 2, 4, 8, 16 or 32), every lane of a group getting the group's sum:
// DPP quad permutes (xor 1, xor 2), half-row and row mirrors (8 and 16 lanes), then one cross-row swap for 32.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    auto dpp = [](float x, int ctrl_tag) {
        int r = 0;
        const int xi = __float_as_int(x);
        switch (ctrl_tag) {
            case 0: r = __builtin_amdgcn_update_dpp(0, xi, 0xB1, 0xF, 0xF, false); break;   // quad_perm [1,0,3,2]
            case 1: r = __builtin_amdgcn_update_dpp(0, xi, 0x4E, 0xF, 0xF, false); break;   // quad_perm [2,3,0,1]
            case 2: r = __builtin_amdgcn_update_dpp(0, xi, 0x141, 0xF, 0xF, false); break;  // row_half_mirror
            default: r = __builtin_amdgcn_update_dpp(0, xi, 0x140, 0xF, 0xF, false); break; // row_mirror
        }
        return __int_as_float(r);
    };
    if constexpr (N >= 2) v += dpp(v, 0);
    if constexpr (N >= 4) v += dpp(v, 1);
    if constexpr (N >= 8) v += dpp(v, 2);
    if constexpr (N >= 16) v += dpp(v, 3);
    if constexpr (N >= 32) v += __shfl_xor(v, 16);
    return v;
}

template <int F>
__device__ __forceinline__ float elem(const Raw8<F> &r, int i) {
    if constexpr (F == MARIN_KV_F32) return __uint_as_float(r.w[i / 4][i % 4]);
    const uint32_t w = r.w[0][i / 2];
    if constexpr (F == MARIN_KV_F16) return f16_bits_to_f32((uint16_t)(i % 2 ? w >> 16 : w & 0xffffu));
    return __uint_as_float(i % 2 ? w & 0xffff0000u : w << 16);
}

__device__ __forceinline__ const uint8_t *kv_row(const uint64_t *table, const KvGeom &g, int which, int kvh,
                                                 uint32_t pos) {
    const uint64_t page = table[pos >> g.page_shift];
    const uint32_t in_page = pos & ((1u << g.page_shift) - 1u);
    const size_t es = g.format == MARIN_KV_F32 ? 4 : 2;
    return reinterpret_cast<const uint8_t *>(page + g.layer_offset + (which ? g.value_offset : 0) +
                                             (uint64_t)kvh * g.head_bytes + (uint64_t)in_page * g.head_dim * es);
}

// Stores one value of a key/value row in the cache's format (kv_format.cu:48-72): f16 rounds to nearest and saturates
// at the largest finite value (NaN stays NaN), bf16 rounds to nearest even (NaN stays NaN).
template <int F>
__device__ __forceinline__ void store_kv(uint8_t *row, int e, float x) {
    if constexpr (F == MARIN_KV_F32) reinterpret_cast<float *>(row)[e] = x;
    if constexpr (F == MARIN_KV_F16) {
        const float c = fminf(fmaxf(x, -65504.0f), 65504.0f);
        reinterpret_cast<_Float16 *>(row)[e] = (_Float16)(x != x ? x : c);
    }
    if constexpr (F == MARIN_KV_BF16) {
        const unsigned u = __float_as_uint(x);
        reinterpret_cast<uint16_t *>(row)[e] =
            (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40u : (u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
}

// One head's RMSNorm(weight) + RoPE inputs held by one wave: lane i takes the pairs (i, i + hd/2), i < hd/2 (hd
// even, at most 256), with their norm weights and RoPE frequencies.
struct HeadIn {
    float a[2], b[2], wa[2], wb[2], f[2], s[2];  // f: the frequency, or with a cos/sin table the cosine (s the sine)
};

__device__ __forceinline__ HeadIn load_head(const float *__restrict__ src, const float *__restrict__ w,
                                            const float *__restrict__ freq, int hd, int lane) {
    const int half = hd / 2;
    HeadIn h;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = lane + 64 * k;
        const bool in = i < half;
        h.a[k] = in ? src[i] : 0.0f;
        h.b[k] = in ? src[i + half] : 0.0f;
        h.wa[k] = in ? w[i] : 0.0f;
        h.wb[k] = in ? w[i + half] : 0.0f;
        h.f[k] = in ? freq[i] : 0.0f;
    }
    return h;
}

// Norm: x * (1 / sqrtf(mean(x^2) + eps)) * w (kernels.cu:51-60); RoPE: angle = pos * freq[i] with the host's powf
// table, sincosf on the device, (a, b) -> (a cos - b sin, b cos + a sin) (ops.rs:56-95).
__device__ __forceinline__ void finish_head(const HeadIn &h, uint32_t pos, int hd, float eps, int lane, float a[2],
                                            float b[2]) {
    const int half = hd / 2;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) s += h.a[k] * h.a[k] + h.b[k] * h.b[k];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    const float scale = 1.0f / sqrtf(s / (float)hd + eps);
    const float position = (float)pos;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = lane + 64 * k;
        a[k] = b[k] = 0.0f;
        if (i >= half) continue;
        const float x = h.a[k] * scale * h.wa[k], y = h.b[k] * scale * h.wb[k];
        float sn, cs;
        sincosf(position * h.f[k], &sn, &cs);
        a[k] = x * cs - y * sn;
        b[k] = y * cs + x * sn;
    }
}

// RMSNorm(weight) then RoPE at `pos` of one head, by one wave.
__device__ __forceinline__ void norm_rope_head(const float *__restrict__ src, const float *__restrict__ w,
                                               const float *__restrict__ freq, uint32_t pos, int hd, float eps,
                                               int lane, float a[2], float b[2]) {
    finish_head(load_head(src, w, freq, hd, lane), pos, hd, eps, lane, a, b);
}

// Diagnostic build flag ATTN_TIMING (off in every shipped build; ATT_T then compiles to nothing): thread 0 of each
// workgroup records the 100 MHz wall clock at numbered points of the attention kernels into attn_dbg, eight slots per
// workgroup, read back by marin_attn_dbg. In attention_decode: 6 entry, 0 context length known, 1 row loads issued,
// 2 query ready, 3 softmax done, 4 partials combined, 5 records written.
#ifdef ATTN_TIMING
__device__ unsigned long long attn_dbg[65536 * 8];
#define ATT_T(k)                                                                                                 \
    if (threadIdx.x == 0)                                                                                        \
        attn_dbg[((size_t)(blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * 8 + (k)] = wall_clock64();
extern "C" void marin_attn_dbg(void *out) { (void)hipMemcpyFromSymbol(out, HIP_SYMBOL(attn_dbg), sizeof(attn_dbg)); }
extern "C" void marin_attn_dbg_clear() {
    static unsigned long long zeros[65536 * 8];
    (void)hipMemcpyToSymbol(HIP_SYMBOL(attn_dbg), zeros, sizeof(zeros));
}
#else
#define ATT_T(k)
#endif

// One launch of split-context attention. grid: x = chunk of the context (split), y = kv_head * row_groups + row_group,
// z = sequence. A workgroup of NW waves takes `chunk` positions of one kv head for up to R query rows (row r of the kv
// head: token r / group, head kvh * group + r % group). Lanes work in groups of LPP per position, 8 head values a
// lane; each lane group loads the key and value rows of U positions together, so a chunk is one pass over HBM with an
// online softmax per row. The chunk's page addresses are read into LDS first. Scores are kept in the log2 domain (the
// host folds log2(e) into `scale`), so every weight is one hardware exp2.
//
// The chunks of a (sequence, kv head, row group) meet in the same launch, in two levels: each chunk writes a record
// (max, sum of weights, weighted values) per row; the last chunk of every GROUP consecutive chunks to finish (an
// atomic count, reset by that workgroup) merges the group's records with log-sum-exp weights, and the last group to
// finish merges the group records into the output. Every sum runs in a fixed order, so results do not depend on
// which workgroup finishes last. A context of one chunk writes the output directly.
//
// FUSE: q and the new tokens' keys and values are the raw projections [tokens][heads + 2 kv_heads][hd]; the kernel
// applies q/k RMSNorm and RoPE itself and stores the new keys and values of its chunk into the cache before reading
// it (every row group of the chunk stores the same bytes).
constexpr int POS_IN_FLIGHT = 2;  // positions per lane group loaded together
constexpr int GROUP = 16;         // chunks merged together at the first level

// Records: [max, sum, 0, 0, values, pad] of rec_floats(hd) floats (a multiple of 4), written and read with 16-byte
// agent-coherent buffer accesses (sc1): no dirty lines stay in one die's L2, so a merging workgroup on another die
// reads them without a cache write-back. Level-1 records [unit][splits], then level-2 records [unit][groups].
__host__ __device__ inline int rec_floats(int hd) { return (hd + 4 + 3) / 4 * 4; }
__host__ __device__ inline int groups_of(int splits) { return (splits + GROUP - 1) / GROUP; }

template <int R, int NW>
struct MergeLds {
    float mw[R][GROUP];  // record maxima, then weights
    float lw[R][GROUP];
};

template <int F, int LPP, bool VEC, bool BF16IO, int R, bool FUSE, int NW>
__global__ __launch_bounds__(64 * NW) void attention_split(
    const void *__restrict__ qv, AttnFuse fuse, const uint64_t *__restrict__ tables, size_t table_stride,
    const uint32_t *__restrict__ ctx_lens, KvGeom geom, int tokens, int heads, int kv_heads, int chunk, int splits,
    float scale, float *__restrict__ part, int part_bytes, uint32_t *__restrict__ counters, void *__restrict__ out) {
    constexpr int NT = 64 * NW;
    constexpr int HMAX = 256;
    constexpr int U = POS_IN_FLIGHT;
    constexpr int PPW = 64 / LPP;  // positions per wave step
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / LPP, sub = lane % LPP;
    const int hd = (int)geom.head_dim;
    const int group = heads / kv_heads;
    const int total_rows = tokens * group;
    const int row_groups = (total_rows + R - 1) / R;
    const int kvh = blockIdx.y / row_groups, rg = blockIdx.y % row_groups;
    const int b = blockIdx.z, split = blockIdx.x;
    const int ctx = (int)ctx_lens[b];
    const int first = split * chunk;
    if (first >= ctx) return;
    ATT_T(0);
    const int count = min(chunk, ctx - first);
    const int used = (ctx + chunk - 1) / chunk;
    const int r0 = rg * R;
    const int nrows = min(R, total_rows - r0);
    const uint64_t *table = tables + (size_t)b * table_stride;
    const int d = sub * 8;
    const size_t es = F == MARIN_KV_F32 ? 4 : 2;
    const uint64_t head_off = (uint64_t)kvh * geom.head_bytes + geom.layer_offset;
    const uint32_t pmask = (1u << geom.page_shift) - 1u;

    __shared__ uint64_t pages_s[MAX_CHUNK + 1];
    __shared__ float q_s[R][HMAX];          // q rows; then the workgroup's (or a merge's) weighted values
    __shared__ float red_acc[NW][R][HMAX];  // every wave's weighted values
    __shared__ float red_ml[NW][R][2];      // every wave's maximum and sum
    __shared__ float ml_s[R][2];            // the workgroup's (or a merge's) maximum and sum
    __shared__ MergeLds<R, NW> mg;
    __shared__ int last_s;

    const int page0 = first >> geom.page_shift;
    const int npages = ((first + count - 1) >> geom.page_shift) - page0 + 1;
    for (int i = threadIdx.x; i < npages; i += NT) pages_s[i] = table[page0 + i] + head_off;

    const size_t qkv_stride = (size_t)(heads + 2 * kv_heads) * hd;
    if constexpr (FUSE) {
        for (int r = wave; r < nrows; r += NW) {
            const int rr = r0 + r, t = rr / group, h = kvh * group + rr % group;
            float a2[2], b2[2];
            norm_rope_head(fuse.qkv + (size_t)t * qkv_stride + (size_t)h * hd, fuse.q_norm, fuse.freq,
                           (uint32_t)(ctx - tokens + t), hd, fuse.eps, lane, a2, b2);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int i = lane + 64 * k;
                if (i < hd / 2) {
                    q_s[r][i] = a2[k];
                    q_s[r][i + hd / 2] = b2[k];
                }
            }
        }
        // the new positions that fall in this chunk: keys normalized and rotated, values as they are
        for (int t = wave; t < tokens; t += NW) {
            const int np = ctx - tokens + t;
            if (np < first || np >= first + count) continue;
            const uint64_t page = table[np >> geom.page_shift] + head_off + (uint64_t)(np & pmask) * hd * es;
            uint8_t *krow = reinterpret_cast<uint8_t *>(page);
            uint8_t *vrow = reinterpret_cast<uint8_t *>(page + geom.value_offset);
            float a2[2], b2[2];
            norm_rope_head(fuse.qkv + (size_t)t * qkv_stride + (size_t)(heads + kvh) * hd, fuse.k_norm, fuse.freq,
                           (uint32_t)np, hd, fuse.eps, lane, a2, b2);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int i = lane + 64 * k;
                if (i < hd / 2) {
                    store_kv<F>(krow, i, a2[k]);
                    store_kv<F>(krow, i + hd / 2, b2[k]);
                }
            }
            const float *vsrc = fuse.qkv + (size_t)t * qkv_stride + (size_t)(heads + kv_heads + kvh) * hd;
            for (int i = lane; i < hd; i += 64) store_kv<F>(vrow, i, vsrc[i]);
        }
    } else {
        for (int i = threadIdx.x; i < nrows * hd; i += NT) {
            const int r = i / hd, e = i % hd;
            const int rr = r0 + r, t = rr / group, h = kvh * group + rr % group;
            const size_t at = (((size_t)b * tokens + t) * heads + h) * hd + e;
            if constexpr (BF16IO) q_s[r][e] = bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(qv)[at]);
            else q_s[r][e] = reinterpret_cast<const float *>(qv)[at];
        }
    }
    __syncthreads();
    ATT_T(1);

    float q[R][8];
    int visible[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int rr = r0 + r, t = rr / group;
        visible[r] = r < nrows ? ctx - tokens + t + 1 : 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) q[r][i] = (d + i < hd) ? q_s[r][d + i] : 0.0f;
    }
    auto row_ptr = [&](int which, int p) {
        const uint32_t pos = (uint32_t)(first + p);
        return reinterpret_cast<const uint8_t *>(pages_s[(pos >> geom.page_shift) - page0] +
                                                 (which ? geom.value_offset : 0) + (uint64_t)(pos & pmask) * hd * es);
    };

    float mrow[R], lrow[R], acc[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        mrow[r] = -INFINITY;
        lrow[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r][i] = 0.0f;
    }
    constexpr int STEP = NW * PPW;
    for (int p0 = wave * PPW; p0 < count; p0 += STEP * U) {
        Raw8<F> kr[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int p = p0 + u * STEP + slot;
#pragma unroll
            for (int j = 0; j < (F == MARIN_KV_F32 ? 2 : 1); ++j) kr[u].w[j] = vr[u].w[j] = (u32x4){0, 0, 0, 0};
            if (p < count && d < hd) {
                load_raw<F, VEC>(row_ptr(0, p), d, hd, kr[u]);
                load_raw<F, VEC>(row_ptr(1, p), d, hd, vr[u]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sc[U];
            float mx = -INFINITY;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float dot = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) dot += q[r][i] * elem<F>(kr[u], i);
                dot = group_sum<LPP>(dot);
                const int p = p0 + u * STEP + slot;
                sc[u] = (p < count && first + p < visible[r]) ? dot * scale : -INFINITY;
                mx = fmaxf(mx, sc[u]);
            }
            const float mn = fmaxf(mrow[r], mx);
            if (mn != -INFINITY) {
                const float corr = __builtin_amdgcn_exp2f(mrow[r] - mn);
                lrow[r] *= corr;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[r][i] *= corr;
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const float e = __builtin_amdgcn_exp2f(sc[u] - mn);
                    lrow[r] += e;
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[r][i] += e * elem<F>(vr[u], i);
                }
                mrow[r] = mn;
            }
        }
    }
    // Combine the position slots of the wave (lanes with the same sub), then the waves in a fixed order.
#pragma unroll
    for (int o = LPP; o < 64; o <<= 1) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float mo = __shfl_xor(mrow[r], o), lo = __shfl_xor(lrow[r], o);
            float ao[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) ao[i] = __shfl_xor(acc[r][i], o);
            const float mn = fmaxf(mrow[r], mo);
            const float wa = mrow[r] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mrow[r] - mn);
            const float wb = mo == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mo - mn);
            lrow[r] = lrow[r] * wa + lo * wb;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[r][i] = acc[r][i] * wa + ao[i] * wb;
            mrow[r] = mn;
        }
    }
    if (slot == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (d + i < hd) red_acc[wave][r][d + i] = acc[r][i];
            if (sub == 0) {
                red_ml[wave][r][0] = mrow[r];
                red_ml[wave][r][1] = lrow[r];
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < nrows) {
        const int r = threadIdx.x;
        float mn = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) mn = fmaxf(mn, red_ml[w][r][0]);
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = red_ml[w][r][0];
            l += mw == -INFINITY ? 0.0f : red_ml[w][r][1] * __builtin_amdgcn_exp2f(mw - mn);
        }
        ml_s[r][0] = mn;
        ml_s[r][1] = l;
    }
    for (int o = threadIdx.x; o < nrows * hd; o += NT) {
        const int r = o / hd, e = o % hd;
        float mn = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) mn = fmaxf(mn, red_ml[w][r][0]);
        float a = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = red_ml[w][r][0];
            a += mw == -INFINITY ? 0.0f : red_acc[w][r][e] * __builtin_amdgcn_exp2f(mw - mn);
        }
        q_s[r][e] = a;
    }
    __syncthreads();
    ATT_T(2);

    auto write_out = [&](int r, int e, float v) {
        const int rr = r0 + r, t = rr / group, h = kvh * group + rr % group;
        const size_t at = (((size_t)b * tokens + t) * heads + h) * hd + e;
        if constexpr (BF16IO) {
            const unsigned u = __float_as_uint(v);
            reinterpret_cast<uint16_t *>(out)[at] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        } else {
            reinterpret_cast<float *>(out)[at] = v;
        }
    };
    if (used == 1) {
        for (int o = threadIdx.x; o < nrows * hd; o += NT) write_out(o / hd, o % hd, q_s[o / hd][o % hd] / ml_s[o / hd][1]);
        return;
    }

    const int RS = rec_floats(hd);
    const int ngroups = groups_of(used);
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(part, (short)0, part_bytes, 0x00020000);
    constexpr int SC1 = 16;
    const size_t l2_base = (size_t)gridDim.z * tokens * heads * splits;  // first level-2 record
    auto unit_of = [&](int r) {
        const int rr = r0 + r, t = rr / group, h = kvh * group + rr % group;
        return ((size_t)b * tokens + t) * heads + h;
    };
    auto l1_off = [&](int r, int sp) { return (int)((unit_of(r) * splits + sp) * (size_t)RS * 4); };
    auto l2_off = [&](int r, int gi) {
        return (int)((l2_base + unit_of(r) * (size_t)groups_of(splits) + gi) * (size_t)RS * 4);
    };
    // Writes the workgroup's current (ml_s, q_s) as a record.
    auto write_record = [&](auto off_of) {
        for (int o = threadIdx.x; o < nrows * (RS / 4); o += NT) {
            const int r = o / (RS / 4), c4 = o % (RS / 4);
            u32x4 v;
            if (c4 == 0) {
                v = (u32x4){__float_as_uint(ml_s[r][0]), __float_as_uint(ml_s[r][1]), 0u, 0u};
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int e = 4 * (c4 - 1) + j;
                    v[j] = e < hd ? __float_as_uint(q_s[r][e]) : 0u;
                }
            }
            __builtin_amdgcn_raw_buffer_store_b128(v, prs, off_of(r) + 16 * c4, 0, SC1);
        }
        // every wave's stores acknowledged before the workgroup counts itself in
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    };
    // Counts the workgroup in; true for the last of `n`. The count is an acquire-release at agent scope: the
    // workgroup's record stores (acknowledged above) are released with it, and the last arriver's merge loads are
    // ordered after it, whatever the cache bits of those loads and stores.
    auto arrive = [&](uint32_t *counter, int n) {
        if (threadIdx.x == 0)
            last_s = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(n - 1);
        __syncthreads();
        return last_s != 0;
    };
    // Merges n (<= GROUP) records at off_of(r, k) into (ml_s, q_s), sums in record order.
    auto merge = [&](auto off_of, int n) {
        for (int i = threadIdx.x; i < nrows * n; i += NT) {
            const int r = i / n, k = i - r * n;
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(prs, off_of(r, k), 0, SC1);
            mg.mw[r][k] = __uint_as_float(v[0]);
            mg.lw[r][k] = __uint_as_float(v[1]);
        }
        __syncthreads();
        if (threadIdx.x < nrows) {
            const int r = threadIdx.x;
            float mn = -INFINITY;
            for (int k = 0; k < n; ++k) mn = fmaxf(mn, mg.mw[r][k]);
            float l = 0.0f;
            for (int k = 0; k < n; ++k) {
                const float mk = mg.mw[r][k];
                const float wt = mk == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mk - mn);
                mg.mw[r][k] = wt;
                l += mg.lw[r][k] * wt;
            }
            ml_s[r][0] = mn;
            ml_s[r][1] = l;
        }
        __syncthreads();
        const int c4 = (hd + 3) / 4;
        for (int col = threadIdx.x; col < nrows * c4; col += NT) {
            const int r = col / c4, e4 = col - r * c4;
            u32x4 v[GROUP];
#pragma unroll
            for (int k = 0; k < GROUP; ++k)
                v[k] = __builtin_amdgcn_raw_buffer_load_b128(prs, off_of(r, min(k, n - 1)) + 16 * (1 + e4), 0, SC1);
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < GROUP; ++k) {
                const float wt = k < n ? mg.mw[r][k] : 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) a[j] += __uint_as_float(v[k][j]) * wt;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (4 * e4 + j < hd) q_s[r][4 * e4 + j] = a[j];
        }
        __syncthreads();
    };

    // level 1: this chunk's record; the last of its group merges the group
    write_record([&](int r) { return l1_off(r, split); });
    ATT_T(3);
    const int gi = split / GROUP;
    const int gsize = min(GROUP, used - gi * GROUP);
    const size_t cbase = (((size_t)b * kv_heads + kvh) * row_groups + rg) * (size_t)(1 + groups_of(splits));
    uint32_t *c1 = counters + cbase + 1 + gi;
    if (!arrive(c1, gsize)) return;
    ATT_T(4);
    merge([&](int r, int k) { return l1_off(r, gi * GROUP + k); }, gsize);
    if (threadIdx.x == 0) __hip_atomic_store(c1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ATT_T(5);
    if (ngroups > 1) {
        // level 2: the group's record; the last group merges the groups
        write_record([&](int r) { return l2_off(r, gi); });
        uint32_t *c2 = counters + cbase;
        if (!arrive(c2, ngroups)) return;
        ATT_T(6);
        merge([&](int r, int k) { return l2_off(r, k); }, ngroups);
        if (threadIdx.x == 0) __hip_atomic_store(c2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    ATT_T(7);
    for (int o = threadIdx.x; o < nrows * hd; o += NT) write_out(o / hd, o % hd, q_s[o / hd][o % hd] / ml_s[o / hd][1]);
}

// ---------------------------------------------------------------------------------------------------------------
// One-token decode attention (every sequence adds one position): one launch, merge included.
//
// grid: x = chunk of the context, y = kv head, z = sequence; 4 waves. A workgroup takes `chunk` = U steps of
// positions of one kv head for all `group` query heads of it (R >= group rows). Lanes work in groups of LPP per
// position with 8 head values a lane (a wave covers 64 / LPP positions per step). Every lane reads the page address of
// each of its positions itself and then issues all of its key and value rows at once, so a chunk costs two dependent
// memory round trips and nothing waits on a barrier before the rows are in flight.
//  - With FUSE the query heads (and, in the workgroup whose chunk holds the new position, the new key and value) are
//    loaded before anything else and get RMSNorm + RoPE while the rows are in flight; that workgroup takes the new key
//    and value from LDS (rounded to the cache format exactly as stored) and stores them into the cache last.
//  - Scores and weights are in the log2 domain (the host folds log2(e) into `scale`). A lane group keeps its
//    positions' (max, sum, weighted values); the groups of a wave combine through lane shuffles, the waves through
//    LDS, all in a fixed order.
//  - More than one chunk: each writes a record (max, sum, weighted values) per row with agent-coherent stores, waits
//    for them, and counts itself in on the (sequence, kv head)'s counter; the last to arrive reads every record of its
//    rows and merges them in chunk order, so the result does not depend on arrival order. Its loads are
//    agent-coherent too: on gfx950 a store or load with the device scope bit (sc1) goes through to the device's
//    coherence point rather than one die's L2, so the records need no cache write-back or invalidation, and the
//    counter's atomic is issued only after the record stores have been acknowledged (s_waitcnt vmcnt(0)).
// Values of lane `lane` and its partner `o` lanes away (o a power of two), as (lower lane's, upper lane's), the same in
// both lanes. Partners 16 and 32 lanes away use the gfx950 row swaps (VALU, no LDS round trip).
__device__ __forceinline__ void pair_lanes(float v, int o, int lane, float &lo, float &hi) {
    if (o == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else if (o == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        lo = __uint_as_float(r[0]);
        hi = __uint_as_float(r[1]);
    } else {
        const float other = __shfl_xor(v, o);
        const bool upper = (lane & o) != 0;
        lo = upper ? other : v;
        hi = upper ? v : other;
    }
}

// load_head with the RoPE angle's cosine and sine read from a table row (pairs for i = 0 .. hd/2 - 1) instead of
// the frequency; finish_head_cs applies them.
__device__ __forceinline__ HeadIn load_head_cs(const float *__restrict__ src, const float *__restrict__ w,
                                               const float2 *__restrict__ cs, int hd, int lane) {
    const int half = hd / 2;
    HeadIn h;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = lane + 64 * k;
        const bool in = i < half;
        h.a[k] = in ? src[i] : 0.0f;
        h.b[k] = in ? src[i + half] : 0.0f;
        h.wa[k] = in ? w[i] : 0.0f;
        h.wb[k] = in ? w[i + half] : 0.0f;
        const float2 c = in ? cs[i] : make_float2(1.0f, 0.0f);
        h.f[k] = c.x;
        h.s[k] = c.y;
    }
    return h;
}

__device__ __forceinline__ void finish_head_cs(const HeadIn &h, int hd, float eps, int lane, float a[2], float b[2]) {
    const int half = hd / 2;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) s += h.a[k] * h.a[k] + h.b[k] * h.b[k];
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    const float scale = 1.0f / sqrtf(s / (float)hd + eps);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = lane + 64 * k;
        a[k] = b[k] = 0.0f;
        if (i >= half) continue;
        const float x = h.a[k] * scale * h.wa[k], y = h.b[k] * scale * h.wb[k];
        const float cs = h.f[k], sn = h.s[k];
        a[k] = x * cs - y * sn;
        b[k] = y * cs + x * sn;
    }
}

constexpr int DEC_NW = 4;           // waves per workgroup
constexpr int DEC_MAX_SPLITS = 64;  // chunks the last workgroup merges (a lane of one wave each)

// Steps of key/value loads per lane a workgroup may take (the burst held in registers).
template <int F, int R>
__host__ __device__ constexpr int dec_umax() { return F == MARIN_KV_F32 ? (R <= 4 ? 8 : 4) : (R <= 4 ? 16 : 8); }

// Eight values of a new key or value row in the cache's storage format (store_kv's rounding).
template <int F>
__device__ __forceinline__ Raw8<F> to_raw(const float *v) {
    Raw8<F> r;
    if constexpr (F == MARIN_KV_F32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) r.w[i / 4][i % 4] = __float_as_uint(v[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            uint32_t lo, hi;
            if constexpr (F == MARIN_KV_F16) {
                const float a = v[i] != v[i] ? v[i] : fminf(fmaxf(v[i], -65504.0f), 65504.0f);
                const float b = v[i + 1] != v[i + 1] ? v[i + 1] : fminf(fmaxf(v[i + 1], -65504.0f), 65504.0f);
                lo = __builtin_bit_cast(uint16_t, (_Float16)a);
                hi = __builtin_bit_cast(uint16_t, (_Float16)b);
            } else {
                auto rne = [](float x) {
                    const unsigned u = __float_as_uint(x);
                    return (u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40u : (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
                };
                lo = rne(v[i]);
                hi = rne(v[i + 1]);
            }
            r.w[0][i / 2] = (lo & 0xffffu) | (hi << 16);
        }
    }
    return r;
}

// Merges the records of `used` chunks for the `group` rows of one (sequence, kv head) and writes the rows' outputs.
// One memory round trip: the value threads (a thread per (row, 4 values, share of the records), up to VR records
// each) issue their loads, then a wave per row loads the records' (max, sum), a lane per record; the row's maximum,
// weights and weighted sum are lane reductions in a fixed pattern, so the result does not depend on which chunk
// finished last. LDS: wt_s [R][DEC_MAX_SPLITS] weights, lsum_s [R], sh_s 3 * group * hd floats.
template <bool BF16IO, int R, int NW>
__device__ __forceinline__ void merge_records(__amdgpu_buffer_rsrc_t prs, int rec0, int rec_row, int rec_bytes,
                                              int hd, int group, int used, float (*wt_s)[DEC_MAX_SPLITS],
                                              float *lsum_s, float *sh_s, void *out, size_t out_row0) {
    constexpr int NT = 64 * NW, QPW = (R + NW - 1) / NW;
    constexpr int SC1 = 16;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    auto rec_off = [&](int r, int k) { return rec0 + r * rec_row + k * rec_bytes; };
    auto write_out = [&](int r, int e, float v) {
        const size_t at = (out_row0 + r) * hd + e;
        if constexpr (BF16IO) {
            const unsigned u = __float_as_uint(v);
            reinterpret_cast<uint16_t *>(out)[at] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        } else {
            reinterpret_cast<float *>(out)[at] = v;
        }
    };
    constexpr int VR = 16;                 // records' values a thread holds
    const int c4n = hd / 4;
    const int items = group * c4n;         // (row, 4 values)
    const int shares = max(1, min(NT / items, 4));
    const int per = (used + shares - 1) / shares;  // records of one share
    const int item = (int)threadIdx.x % items, share = (int)threadIdx.x / items;
    const bool valuer = share < shares;
    const int r = item / c4n, e4 = item - r * c4n;
    const int k_lo = share * per, k_hi = min(used, k_lo + per);
    u32x4 vv[VR];
    auto value_burst = [&](int k0) {
#pragma unroll
        for (int j = 0; j < VR; ++j) {
            const int k = min(k0 + j, max(k_hi - 1, 0));
            vv[j] = __builtin_amdgcn_raw_buffer_load_b128(prs, rec_off(r, k) + 16 * (1 + e4), 0, SC1);
        }
    };
    if (valuer) value_burst(k_lo);
    {
        u32x4 hdr[QPW];
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const int rr = min(wave + j * NW, group - 1);
            hdr[j] = __builtin_amdgcn_raw_buffer_load_b128(prs, rec_off(rr, min(lane, used - 1)), 0, SC1);
        }
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const int rr = wave + j * NW;
            const float mk = lane < used ? __uint_as_float(hdr[j][0]) : -INFINITY;
            const float lk = lane < used ? __uint_as_float(hdr[j][1]) : 0.0f;
            float mx = mk;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
            const float wt = mk == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mk - mx);
            float lsum = lk * wt;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o);
            if (rr < group) {
                wt_s[rr][lane] = wt;
                if (lane == 0) lsum_s[rr] = lsum;
            }
        }
    }
    __syncthreads();
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (valuer) {
        for (int k0 = k_lo; k0 < k_hi; k0 += VR) {
            if (k0 != k_lo) value_burst(k0);
#pragma unroll
            for (int j = 0; j < VR; ++j) {
                const int k = k0 + j;
                const float wt = k < k_hi ? wt_s[r][k] : 0.0f;
#pragma unroll
                for (int t = 0; t < 4; ++t) a[t] += __uint_as_float(vv[j][t]) * wt;
            }
        }
    }
    // the shares' sums meet in share order
    if (valuer && share > 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) sh_s[((share - 1) * items + item) * 4 + t] = a[t];
    }
    __syncthreads();
    if (valuer && share == 0) {
        for (int sh = 1; sh < shares; ++sh)
#pragma unroll
            for (int t = 0; t < 4; ++t) a[t] += sh_s[((sh - 1) * items + item) * 4 + t];
        const float lsum = lsum_s[r];
#pragma unroll
        for (int t = 0; t < 4; ++t) write_out(r, 4 * e4 + t, a[t] / lsum);
    }
}

template <int F, int LPP, bool BF16IO, int R, bool FUSE, int U>
__global__ __launch_bounds__(64 * DEC_NW) void attention_decode(
    const void *__restrict__ qv, AttnFuse fuse, const uint64_t *__restrict__ tables, size_t table_stride,
    int table_len, const uint8_t *__restrict__ zero_row, const uint32_t *__restrict__ ctx_lens, KvGeom geom,
    int heads, int kv_heads, int chunk, int splits, float scale, float *__restrict__ part, int part_bytes,
    void *__restrict__ out) {
    constexpr int NW = DEC_NW, NT = 64 * NW;
    constexpr int HMAX = 8 * LPP;  // head values covered by the lanes of one position
    constexpr int PPW = 64 / LPP;  // positions per wave step
    constexpr int STEP = NW * PPW; // positions per workgroup step
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / LPP, sub = lane % LPP;
    const int hd = (int)geom.head_dim;
    const int group = heads / kv_heads;
    const int kvh = blockIdx.y, b = blockIdx.z, split = blockIdx.x;
    const int first = split * chunk;
    const uint64_t *table = tables + (size_t)b * table_stride;
    ATT_T(6);
    // ---- 1. page addresses of this lane's positions, first of all loads and before the context length is known
    // (an index past the table is clamped; entries past the context are never dereferenced)
    uint64_t pg[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int p = first + wave * PPW + slot + u * STEP;
        pg[u] = table[min(p >> (int)geom.page_shift, table_len - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);
    const int ctx = (int)ctx_lens[b];
    if (first >= ctx) return;
    const int count = min(chunk, ctx - first);
    const int used = (ctx + chunk - 1) / chunk;
    const int d = sub * 8;
    const int dl = min(d, hd - 8);  // load offset: lanes past the head's end read its last 8 values, weighted by 0
    const size_t es = F == MARIN_KV_F32 ? 4 : 2;
    const uint64_t head_off = (uint64_t)kvh * geom.head_bytes + geom.layer_offset;
    const uint32_t pmask = (1u << geom.page_shift) - 1u;
    const int newpos = ctx - 1;
    const bool owns_new = FUSE && newpos >= first && newpos < first + count;

    ATT_T(0);
    // partials: every lane group's (R > 4: every pair of lane groups 32 lanes apart) max, sum and weighted values
    constexpr int PRE = R > 4 ? 1 : 0;
    constexpr int NP = NW * (PPW >> PRE);
    __shared__ float q_s[R][HMAX];
    __shared__ float new_s[2][HMAX];  // the new key (normalized and rotated) and value
    __shared__ float pacc_s[NP][R][HMAX];
    __shared__ float pm_s[R][NP], pl_s[R][NP], pw_s[R][NP];
    __shared__ float rm_s[R], rl_s[R];

    // ---- 2. the query inputs (FUSE: raw q heads with the cos/sin of the new position, and the raw new key and value
    // where this chunk holds them), issued behind the page addresses so waiting for those does not wait for these
    constexpr int QPW = (R + NW - 1) / NW;  // q heads per wave
    const float *fq = FUSE ? fuse.qkv + (size_t)b * (heads + 2 * kv_heads) * hd : nullptr;
    HeadIn qin[QPW], kin;
    float vin[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float q[R][8];
    if constexpr (FUSE) {
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const int r = wave + j * NW;
            if (r < group) qin[j] = load_head_cs(fq + (size_t)(kvh * group + r) * hd, fuse.q_norm, fuse.rope + (size_t)newpos * (hd / 2), hd, lane);
        }
        if (owns_new && wave == NW - 1) {
            kin = load_head_cs(fq + (size_t)(heads + kvh) * hd, fuse.k_norm, fuse.rope + (size_t)newpos * (hd / 2), hd, lane);
            const float *vsrc = fq + (size_t)(heads + kv_heads + kvh) * hd;
#pragma unroll
            for (int k = 0; k < 4; ++k) vin[k] = lane + 64 * k < hd ? vsrc[lane + 64 * k] : 0.0f;
        }
    } else {
        // this lane's 8 values of every q head of the kv head, straight into registers (16-byte loads: hd is a
        // multiple of 8, so a lane's 8 values are aligned)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int rr = min(r, group - 1);
            const size_t at = ((size_t)b * heads + kvh * group + rr) * hd + dl;
            float v[8];
            if constexpr (BF16IO) {
                const u32x4 w = *(g_u32x4 *)(uintptr_t)(reinterpret_cast<const uint16_t *>(qv) + at);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[2 * i] = __uint_as_float(w[i] << 16);
                    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
                }
            } else {
                const uintptr_t base = (uintptr_t)(reinterpret_cast<const float *>(qv) + at);
                const u32x4 w0 = *(g_u32x4 *)base, w1 = *(g_u32x4 *)(base + 16);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] = __uint_as_float(w0[i]);
                    v[4 + i] = __uint_as_float(w1[i]);
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) q[r][i] = (r < group && d + i < hd) ? v[i] : 0.0f;
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the query loads stay ahead of the row loads

    // ---- 3. every key and value row of the chunk
    Raw8<F> kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        // positions past the chunk read the zero row (weighed 0 below) rather than an entry never mapped
        const int rel = wave * PPW + slot + u * STEP;
        const uint32_t p = (uint32_t)(first + rel);
        const bool in = rel < count;
        const uint8_t *row = reinterpret_cast<const uint8_t *>(pg[u] + head_off + (uint64_t)(p & pmask) * hd * es);
        load_raw<F, true, true>(in ? row : zero_row, dl, hd, kr[u]);
    }
    // the value rows after every key row: the scores can start while the values are still in flight
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int rel = wave * PPW + slot + u * STEP;
        const uint32_t p = (uint32_t)(first + rel);
        const bool in = rel < count;
        const uint8_t *row = reinterpret_cast<const uint8_t *>(pg[u] + head_off + (uint64_t)(p & pmask) * hd * es);
        load_raw<F, true, true>(in ? row + geom.value_offset : zero_row, dl, hd, vr[u]);
    }
    __builtin_amdgcn_sched_barrier(0);
    ATT_T(1);

    // ---- 4. FUSE: q and the new key normalized and rotated while the rows are in flight
    if constexpr (FUSE) {
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const int r = wave + j * NW;
            if (r < group) {
                float a2[2], b2[2];
                finish_head_cs(qin[j], hd, fuse.eps, lane, a2, b2);
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int i = lane + 64 * k;
                    if (i < hd / 2) {
                        q_s[r][i] = a2[k];
                        q_s[r][i + hd / 2] = b2[k];
                    }
                }
            }
        }
        if (owns_new && wave == NW - 1) {
            float a2[2], b2[2];
            finish_head_cs(kin, hd, fuse.eps, lane, a2, b2);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int i = lane + 64 * k;
                if (i < hd / 2) {
                    new_s[0][i] = a2[k];
                    new_s[0][i + hd / 2] = b2[k];
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (lane + 64 * k < hd) new_s[1][lane + 64 * k] = vin[k];
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 8; ++i) q[r][i] = (r < group && d + i < hd) ? q_s[r][d + i] : 0.0f;
    }

    ATT_T(2);
    // ---- 5. scores, then one softmax pass over this lane group's positions
    float sc[R][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int p = wave * PPW + slot + u * STEP;
        if (owns_new && first + p == newpos) {
            float kn[8], vn[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                kn[i] = d + i < hd ? new_s[0][d + i] : 0.0f;
                vn[i] = d + i < hd ? new_s[1][d + i] : 0.0f;
            }
            kr[u] = to_raw<F>(kn);
            vr[u] = to_raw<F>(vn);
        }
        const bool valid = p < count;
        if (!valid) {
#pragma unroll
            for (int j = 0; j < (F == MARIN_KV_F32 ? 2 : 1); ++j) kr[u].w[j] = vr[u].w[j] = (u32x4){0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) dot += q[r][i] * elem<F>(kr[u], i);
            dot = group_sum<LPP>(dot);
            sc[r][u] = valid ? dot * scale : -INFINITY;
        }
    }
    float mrow[R], lrow[R], acc[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; ++u) mx = fmaxf(mx, sc[r][u]);
        mrow[r] = mx;
        lrow[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r][i] = 0.0f;
        if (mx != -INFINITY) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float e = sc[r][u] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[r][u] - mx);
                lrow[r] += e;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[r][i] += e * elem<F>(vr[u], i);
            }
        }
    }

    ATT_T(3);
    // ---- 6. the partials of the workgroup (R > 4: lane groups 32 lanes apart combined in registers first, both
    // lanes of a pair computing the same lower-then-upper combination) to LDS; then per row the maximum over the
    // partials, each partial's weight and the weighted sum of the sums, every sum in a fixed order
#pragma unroll
    for (int o = 64 >> PRE; o < 64; o <<= 1) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float m0, m1, l0, l1;
            pair_lanes(mrow[r], o, lane, m0, m1);
            pair_lanes(lrow[r], o, lane, l0, l1);
            const float mn = fmaxf(m0, m1);
            const float fa = m0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m0 - mn);
            const float fb = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - mn);
            lrow[r] = l0 * fa + l1 * fb;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float a0, a1;
                pair_lanes(acc[r][i], o, lane, a0, a1);
                acc[r][i] = a0 * fa + a1 * fb;
            }
            mrow[r] = mn;
        }
    }
    if (slot < (PPW >> PRE)) {
        const int pi = wave * (PPW >> PRE) + slot;
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int i = 0; i < 8; ++i) pacc_s[pi][r][d + i] = acc[r][i];
            if (sub == 0) {
                pm_s[r][pi] = mrow[r];
                pl_s[r][pi] = lrow[r];
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < R) {
        const int r = threadIdx.x;
        float mx = -INFINITY;
#pragma unroll
        for (int p = 0; p < NP; ++p) mx = fmaxf(mx, pm_s[r][p]);
        float l = 0.0f;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float w = pm_s[r][p] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pm_s[r][p] - mx);
            pw_s[r][p] = w;
            l += w * pl_s[r][p];
        }
        rm_s[r] = mx;
        rl_s[r] = l;
    }
    __syncthreads();
    ATT_T(4);
    // the workgroup's weighted values of row r, values e .. e + 3 (e a multiple of 4)
    auto combine4 = [&](int r, int e) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float w = pw_s[r][p];
            const float4 x = *reinterpret_cast<const float4 *>(&pacc_s[p][r][e]);
            a.x += w * x.x;
            a.y += w * x.y;
            a.z += w * x.z;
            a.w += w * x.w;
        }
        return a;
    };

    // the new key and value, stored for later steps (this launch took them from LDS); stored here, after every
    // load of the chunk has been waited for, so the store cannot make those waits drain anything
    if (owns_new && wave == NW - 1) {
        const uint64_t page = table[newpos >> geom.page_shift] + head_off + (uint64_t)(newpos & pmask) * hd * es;
        for (int i = lane; i < hd; i += 64) {
            store_kv<F>(reinterpret_cast<uint8_t *>(page), i, new_s[0][i]);
            store_kv<F>(reinterpret_cast<uint8_t *>(page + geom.value_offset), i, new_s[1][i]);
        }
    }
    if (used == 1) {
        for (int o = threadIdx.x; o < group * (hd / 4); o += NT) {
            const int r = o / (hd / 4), e = 4 * (o % (hd / 4));
            const float4 a = combine4(r, e);
            const float inv = 1.0f / rl_s[r];
            const float v[4] = {a.x * inv, a.y * inv, a.z * inv, a.w * inv};
            const size_t at = ((size_t)b * heads + kvh * group + r) * hd + e;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (BF16IO) {
                    const unsigned u = __float_as_uint(v[j]);
                    reinterpret_cast<uint16_t *>(out)[at + j] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
                } else {
                    reinterpret_cast<float *>(out)[at + j] = v[j];
                }
            }
        }
        return;
    }

    // ---- 7. this chunk's record per row, [max, sum, 0, 0, values, pad] in 16-byte stores; attention_decode_merge
    // combines the records after this launch
    const int RS = rec_floats(hd);
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(part, (short)0, part_bytes, 0x00020000);
    for (int o = threadIdx.x; o < group * (RS / 4); o += NT) {
        const int r = o / (RS / 4), c4 = o % (RS / 4);
        u32x4 v;
        if (c4 == 0) {
            v = (u32x4){__float_as_uint(rm_s[r]), __float_as_uint(rl_s[r]), 0u, 0u};
        } else {
            // hd is a multiple of 8, so every group of 4 values is inside the head
            const float4 a = combine4(r, 4 * (c4 - 1));
            v = (u32x4){__float_as_uint(a.x), __float_as_uint(a.y), __float_as_uint(a.z), __float_as_uint(a.w)};
        }
        const int at = (int)(((((size_t)b * heads + kvh * group + r) * splits) + split) * (size_t)RS * 4) + 16 * c4;
        __builtin_amdgcn_raw_buffer_store_b128(v, prs, at, 0, 0);
    }
    ATT_T(5);
}

// The chunk records of each (sequence, q head) merged after attention_decode: a workgroup per (q head, sequence),
// so each workgroup reads one head's records (a few tens of KB) and the launch spreads over many compute units.
template <bool BF16IO>
__global__ __launch_bounds__(64 * DEC_NW) void attention_decode_merge(const float *__restrict__ part, int part_bytes,
                                                                      const uint32_t *__restrict__ ctx_lens, int hd,
                                                                      int heads, int chunk, int splits,
                                                                      void *__restrict__ out) {
    __shared__ float wt_s[1][DEC_MAX_SPLITS];
    __shared__ float lsum_s[1];
    __shared__ float sh_s[3 * 256];
    const int h = blockIdx.x, b = blockIdx.y;
    const int ctx = (int)ctx_lens[b];
    const int used = (ctx + chunk - 1) / chunk;
    if (used <= 1) return;  // a context of one chunk was written by attention_decode itself
    const int RS = rec_floats(hd);
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(part), (short)0, part_bytes,
                                                                       0x00020000);
    const int rec0 = (int)(((size_t)b * heads + h) * splits * (size_t)RS * 4);
    merge_records<BF16IO, 1, DEC_NW>(prs, rec0, splits * RS * 4, RS * 4, hd, 1, used, wt_s, lsum_s, sh_s, out,
                                     (size_t)b * heads + h);
}

constexpr int NWAVES = 4;         // waves per attention workgroup
constexpr int BLOCKS_PER_CU = 4;  // workgroups the chunk size aims at per compute unit

// Positions per workgroup: about BLOCKS_PER_CU workgroups per compute unit, MIN_CHUNK to MAX_CHUNK positions each,
// rounded up to what one step of the workgroup's lanes covers so no lane group idles.
static int chunk_for(size_t max_ctx, size_t blocks_per_chunk, int cu_count, size_t granule) {
    const size_t target = (size_t)BLOCKS_PER_CU * (size_t)std::max(cu_count, 1);
    const size_t wanted = std::max<size_t>(1, (target + blocks_per_chunk - 1) / std::max<size_t>(blocks_per_chunk, 1));
    size_t chunk = (max_ctx + wanted - 1) / wanted;
    granule = std::min<size_t>(granule, MAX_CHUNK);
    chunk = (chunk + granule - 1) / granule * granule;
    chunk = std::min<size_t>(MAX_CHUNK, std::max<size_t>(MIN_CHUNK, chunk));
    return (int)chunk;
}

static size_t record_count(size_t units, size_t splits) { return units * (splits + groups_of((int)splits)); }

size_t attention_partial_floats(size_t batch, size_t tokens, size_t heads, size_t head_dim, size_t max_ctx,
                                int cu_count) {
    (void)cu_count;
    const size_t splits = std::max<size_t>(std::min<size_t>((max_ctx + MIN_CHUNK - 1) / MIN_CHUNK, MAX_SPLITS), 1);
    return record_count(batch * tokens * heads, splits) * (size_t)rec_floats((int)head_dim);
}

size_t attention_counters(size_t batch, size_t tokens, size_t heads) {
    return std::max<size_t>(batch * tokens * heads, 1) * (1 + MAX_SPLITS / GROUP);
}

static int rows_per_block(const AttentionArgs &a) {
    return a.tokens * (a.heads / a.kv_heads) <= 4 ? 4 : ROWS;
}

template <int F, int LPP, bool VEC, bool BF16IO, int R, bool FUSE>
static void launch_split(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    hipEvent_t t0, t1;
    g->kernel_events(t0, t1);
    auto kern = attention_split<F, LPP, VEC, BF16IO, R, FUSE, NWAVES>;
    if (t0)
        hipExtLaunchKernelGGL(kern, grid, dim3(64 * NWAVES), 0u, g->stream, t0, t1, 0u, a.q, a.fuse, a.tables,
                              a.table_stride, a.ctx, a.geom, (int)a.tokens, (int)a.heads, (int)a.kv_heads, chunk,
                              splits, scale, a.partials, (int)(a.partial_floats * 4), a.counters, a.out);
    else
        kern<<<grid, dim3(64 * NWAVES), 0, g->stream>>>(a.q, a.fuse, a.tables, a.table_stride, a.ctx, a.geom,
                                                        (int)a.tokens, (int)a.heads, (int)a.kv_heads, chunk, splits,
                                                        scale, a.partials, (int)(a.partial_floats * 4), a.counters,
                                                        a.out);
}

template <int F, int LPP, bool VEC, int R>
static void launch_split_r(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    if (a.fuse.qkv) launch_split<F, LPP, VEC, false, R, true>(g, a, grid, chunk, splits, scale);
    else if (a.bf16_io) launch_split<F, LPP, VEC, true, R, false>(g, a, grid, chunk, splits, scale);
    else launch_split<F, LPP, VEC, false, R, false>(g, a, grid, chunk, splits, scale);
}

template <int F, int LPP, bool VEC>
static void launch_split_l(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    if (rows_per_block(a) == 4) launch_split_r<F, LPP, VEC, 4>(g, a, grid, chunk, splits, scale);
    else launch_split_r<F, LPP, VEC, ROWS>(g, a, grid, chunk, splits, scale);
}

// Lanes per position, 8 head values a lane (at least 4 lanes); head sizes that are not a multiple of 8 take the
// element-wise loads with 32 lanes.
static int lanes_for(size_t hd) {
    if (hd % 8) return 32;
    int lanes = 4;
    while ((size_t)lanes * 8 < hd) lanes <<= 1;
    return lanes;
}

template <int F>
static void launch_split_f(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    const size_t hd = a.geom.head_dim;
    switch (lanes_for(hd)) {
        case 4: launch_split_l<F, 4, true>(g, a, grid, chunk, splits, scale); break;
        case 8: launch_split_l<F, 8, true>(g, a, grid, chunk, splits, scale); break;
        case 16: launch_split_l<F, 16, true>(g, a, grid, chunk, splits, scale); break;
        default:
            if (hd % 8) launch_split_l<F, 32, false>(g, a, grid, chunk, splits, scale);
            else launch_split_l<F, 32, true>(g, a, grid, chunk, splits, scale);
    }
}

constexpr int DEC_BLOCKS_PER_CU = 1;  // one-token attention workgroups per compute unit the chunking aims at
constexpr int DEC_ROUND_BLOCKS_PER_CU = 2;  // one-token attention workgroups resident per compute unit

template <int F, int LPP, bool BF16IO, int R, bool FUSE, int U>
static void launch_decode(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    hipEvent_t t0, t1;
    g->kernel_events(t0, t1);
    auto kern = attention_decode<F, LPP, BF16IO, R, FUSE, U>;
    if (t0)
        hipExtLaunchKernelGGL(kern, grid, dim3(64 * DEC_NW), 0u, g->stream, t0, t1, 0u, a.q, a.fuse, a.tables,
                              a.table_stride, (int)a.table_len, (const uint8_t *)g->zero_row, a.ctx, a.geom,
                              (int)a.heads, (int)a.kv_heads, chunk, splits, scale, a.partials,
                              (int)(a.partial_floats * 4), a.out);
    else
        kern<<<grid, dim3(64 * DEC_NW), 0, g->stream>>>(a.q, a.fuse, a.tables, a.table_stride, (int)a.table_len,
                                                        (const uint8_t *)g->zero_row, a.ctx, a.geom, (int)a.heads,
                                                        (int)a.kv_heads, chunk, splits, scale, a.partials,
                                                        (int)(a.partial_floats * 4), a.out);
}

template <int F, int LPP, int R, int U>
static void launch_decode_io(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    if (a.fuse.qkv) launch_decode<F, LPP, false, R, true, U>(g, a, grid, chunk, splits, scale);
    else if (a.bf16_io) launch_decode<F, LPP, true, R, false, U>(g, a, grid, chunk, splits, scale);
    else launch_decode<F, LPP, false, R, false, U>(g, a, grid, chunk, splits, scale);
}

// U: the smallest instantiated step count covering the chunk (2, 4, 6, 8, 10, 12 or 16, at most dec_umax); steps
// past the chunk load its last position again and weigh nothing.
template <int F, int LPP, int R>
static void launch_decode_u(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    constexpr int UMAX = dec_umax<F, R>();
    const int step = DEC_NW * (64 / LPP);
    const int u = (chunk + step - 1) / step;
    if (u > UMAX) shape("decode attention chunk (steps)", (size_t)UMAX, (size_t)u);
    if (u <= 2) launch_decode_io<F, LPP, R, 2>(g, a, grid, chunk, splits, scale);
    else if (u <= 4) launch_decode_io<F, LPP, R, 4>(g, a, grid, chunk, splits, scale);
    else if (u <= 6) launch_decode_io<F, LPP, R, (UMAX < 6 ? UMAX : 6)>(g, a, grid, chunk, splits, scale);
    else if (u <= 8) launch_decode_io<F, LPP, R, (UMAX < 8 ? UMAX : 8)>(g, a, grid, chunk, splits, scale);
    else if (u <= 10) launch_decode_io<F, LPP, R, (UMAX < 10 ? UMAX : 10)>(g, a, grid, chunk, splits, scale);
    else if (u <= 12) launch_decode_io<F, LPP, R, (UMAX < 12 ? UMAX : 12)>(g, a, grid, chunk, splits, scale);
    else launch_decode_io<F, LPP, R, (UMAX < 16 ? UMAX : 16)>(g, a, grid, chunk, splits, scale);
}

template <int F>
static void launch_decode_f(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    const bool r4 = a.heads / a.kv_heads <= 4;
    switch (lanes_for(a.geom.head_dim)) {
        case 4: r4 ? launch_decode_u<F, 4, 4>(g, a, grid, chunk, splits, scale)
                   : launch_decode_u<F, 4, 8>(g, a, grid, chunk, splits, scale); break;
        case 8: r4 ? launch_decode_u<F, 8, 4>(g, a, grid, chunk, splits, scale)
                   : launch_decode_u<F, 8, 8>(g, a, grid, chunk, splits, scale); break;
        case 16: r4 ? launch_decode_u<F, 16, 4>(g, a, grid, chunk, splits, scale)
                    : launch_decode_u<F, 16, 8>(g, a, grid, chunk, splits, scale); break;
        default: r4 ? launch_decode_u<F, 32, 4>(g, a, grid, chunk, splits, scale)
                    : launch_decode_u<F, 32, 8>(g, a, grid, chunk, splits, scale); break;
    }
}

// The one-token kernel's chunking for a context bound: about DEC_BLOCKS_PER_CU workgroups per compute unit in all (a
// few workgroups past a whole number per unit would share units with others and set the launch's tail), chunks of
// any length up to what the largest burst of loads covers. 0 when that needs more chunks
// than the last workgroup merges.
static int decode_chunk(const AttentionArgs &a, int cu_count, int &splits) {
    const int hd = (int)a.geom.head_dim;
    const int step = DEC_NW * (64 / lanes_for((size_t)hd));
    const bool r4 = a.heads / a.kv_heads <= 4;
    const int umax = a.geom.format == MARIN_KV_F32 ? (r4 ? dec_umax<MARIN_KV_F32, 4>() : dec_umax<MARIN_KV_F32, 8>())
                                                   : (r4 ? dec_umax<MARIN_KV_F16, 4>() : dec_umax<MARIN_KV_F16, 8>());
    const size_t units = std::max<size_t>(a.kv_heads * a.batch, 1);
    const size_t per_unit = std::max<size_t>(1, (size_t)DEC_BLOCKS_PER_CU * std::max(cu_count, 1) / units);
    size_t chunk = (a.max_ctx + per_unit - 1) / per_unit;
    chunk = std::min<size_t>(std::max<size_t>(chunk, (size_t)step), (size_t)umax * step);
    size_t n = (a.max_ctx + chunk - 1) / chunk;
    // More workgroups than compute units (large batches, long contexts): they run in rounds of about
    // DEC_ROUND_BLOCKS_PER_CU per unit, so the chunks are shortened until the workgroups fill whole rounds (17
    // chunks per unit on 64 units would leave a third round almost empty; 24 shorter ones fill it).
    const size_t cu = (size_t)std::max(cu_count, 1);
    if (n * units > cu) {
        const size_t cap = (size_t)DEC_ROUND_BLOCKS_PER_CU * cu;
        const size_t rounds = (n * units + cap - 1) / cap;
        const size_t want = std::min<size_t>(rounds * cap / units, (size_t)DEC_MAX_SPLITS);
        if (want > n) {
            chunk = (a.max_ctx + want - 1) / want;
            chunk = std::max<size_t>((chunk + step - 1) / step * step, (size_t)step);
            n = (a.max_ctx + chunk - 1) / chunk;
        }
    }
    if (n > (size_t)DEC_MAX_SPLITS) return 0;
    splits = (int)std::max<size_t>(n, 1);
    return (int)chunk;
}

static bool decode_kernel_fits(const AttentionArgs &a) {
    const size_t hd = a.geom.head_dim, group = a.heads / a.kv_heads;
    return a.tokens == 1 && hd % 8 == 0 && hd >= 8 && group <= 8;
}

void launch_attention(marin_gpu *g, const AttentionArgs &a) {
    const size_t group = a.heads / a.kv_heads;
    const size_t rpb = (size_t)rows_per_block(a);
    const size_t row_groups = (a.tokens * group + rpb - 1) / rpb;
    if (a.geom.head_dim == 0 || a.geom.head_dim > 256) unsupported("head size", 256, a.geom.head_dim);
    if (a.fuse.qkv && a.geom.head_dim % 2) unsupported("head size for RoPE (even)", 256, a.geom.head_dim);
    const size_t per_step = (size_t)NWAVES * (64 / lanes_for(a.geom.head_dim)) * POS_IN_FLIGHT;
    const int chunk = chunk_for(a.max_ctx, a.kv_heads * row_groups * a.batch, g->cu_count, per_step);
    const int splits = (int)((a.max_ctx + chunk - 1) / chunk);
    if (splits > MAX_SPLITS) unsupported("attention context (positions)", (size_t)MAX_SPLITS * MAX_CHUNK, a.max_ctx);
    const size_t need = record_count(a.batch * a.tokens * a.heads, splits) * (size_t)rec_floats((int)a.geom.head_dim);
    if (need > a.partial_floats) shape("attention partial records (floats)", need, a.partial_floats);
    if (a.partial_floats * 4 >= ((size_t)1 << 31))
        unsupported("attention partial bytes", (size_t)1 << 31, a.partial_floats * 4);
    const size_t counters = a.batch * a.kv_heads * row_groups * (1 + groups_of(splits));
    if (counters > a.counter_count) shape("attention chunk counters", counters, a.counter_count);
    // scores in the log2 domain: dot * (1/sqrt(hd)) * log2(e), weights 2^(s - max) with the hardware exp2
    const float scale = (float)(1.4426950408889634 / std::sqrt((double)a.geom.head_dim));
    int dsplits = 0;
    const int dchunk = decode_kernel_fits(a) ? decode_chunk(a, g->cu_count, dsplits) : 0;
    if (dchunk) {
        if (a.fuse.qkv && !a.fuse.rope) unsupported("fused decode attention without a RoPE table", 1, 0);
        if (a.table_len == 0 || a.table_len > 0x7fffffffu) shape("decode attention page table entries", 1, a.table_len);
        if (a.geom.head_dim * kv_elem_bytes((marin_kv_format)a.geom.format) > 4096)
            unsupported("decode attention row bytes", 4096, a.geom.head_dim * kv_elem_bytes((marin_kv_format)a.geom.format));
        const size_t dneed = a.batch * a.heads * (size_t)dsplits * (size_t)rec_floats((int)a.geom.head_dim);
        if (dsplits > 1 && dneed > a.partial_floats) shape("attention partial records (floats)", dneed, a.partial_floats);
        if (a.partial_floats * 4 >= ((size_t)1 << 31))
            unsupported("attention partial bytes", (size_t)1 << 31, a.partial_floats * 4);
        if (!(g->only && strcmp(g->only, "attention_decode"))) {
            dim3 dgrid((unsigned)dsplits, (unsigned)a.kv_heads, (unsigned)a.batch);
            switch (a.geom.format) {
                case MARIN_KV_F32: launch_decode_f<MARIN_KV_F32>(g, a, dgrid, dchunk, dsplits, scale); break;
                case MARIN_KV_F16: launch_decode_f<MARIN_KV_F16>(g, a, dgrid, dchunk, dsplits, scale); break;
                default: launch_decode_f<MARIN_KV_BF16>(g, a, dgrid, dchunk, dsplits, scale); break;
            }
            g->launched(marin_gpu::ATTENTION, a.bytes_hint, "attention_decode");
        }
        if (dsplits > 1 && !(g->only && strcmp(g->only, "attention_decode_merge"))) {
            dim3 mgrid((unsigned)a.heads, (unsigned)a.batch);
            const int pb = (int)(a.partial_floats * 4);
            const int hd = (int)a.geom.head_dim, H = (int)a.heads;
            if (a.bf16_io)
                attention_decode_merge<true><<<mgrid, 64 * DEC_NW, 0, g->stream>>>(a.partials, pb, a.ctx, hd, H, dchunk, dsplits, a.out);
            else
                attention_decode_merge<false><<<mgrid, 64 * DEC_NW, 0, g->stream>>>(a.partials, pb, a.ctx, hd, H, dchunk, dsplits, a.out);
            g->launched(marin_gpu::OTHER, 0.0, "attention_decode_merge");
        }
        return;
    }
    // the fused inputs of attention_split are one sequence's token rows
    if (a.fuse.qkv && a.batch > 1) unsupported("fused attention over a batch (one-token decode only)", 1, a.batch);
    if (prefill_fa_fits(a) && g->fast_attention) {
        if (g->only && strcmp(g->only, "fa_prefill")) return;
        launch_prefill_fa(g, a);
        return;
    }
    if (g->only && strcmp(g->only, "attention_split")) return;
    dim3 grid((unsigned)splits, (unsigned)(a.kv_heads * row_groups), (unsigned)a.batch);
    switch (a.geom.format) {
        case MARIN_KV_F32: launch_split_f<MARIN_KV_F32>(g, a, grid, chunk, splits, scale); break;
        case MARIN_KV_F16: launch_split_f<MARIN_KV_F16>(g, a, grid, chunk, splits, scale); break;
        default: launch_split_f<MARIN_KV_BF16>(g, a, grid, chunk, splits, scale); break;
    }
    g->launched(marin_gpu::ATTENTION, a.bytes_hint, "attention_split");
}

// ---------------------------------------------------------------------------------------------------------------
// kv_store (kv_format.cu:48-72): grid (tokens, kv_heads), one thread per head element; f16 rounds to nearest and
// saturates at the largest finite value, bf16 rounds to nearest even.
template <int F>
__global__ void kv_store_kernel(const float *__restrict__ keys, const float *__restrict__ values,
                                const uint64_t *__restrict__ pages, KvGeom geom, uint32_t start, int kv_heads) {
    const int t = blockIdx.x, kvh = blockIdx.y;
    const int hd = (int)geom.head_dim;
    for (int e = threadIdx.x; e < hd; e += blockDim.x) {
        for (int which = 0; which < 2; ++which) {
            const float x = (which ? values : keys)[((size_t)t * kv_heads + kvh) * hd + e];
            store_kv<F>(const_cast<uint8_t *>(kv_row(pages, geom, which, kvh, start + t)), e, x);
        }
    }
}

void launch_kv_store(marin_gpu *g, const float *keys, const float *values, const uint64_t *pages, const KvGeom &geom,
                     size_t start, size_t tokens, size_t kv_heads) {
    if (!tokens) return;
    dim3 grid((unsigned)tokens, (unsigned)kv_heads);
    dim3 block((unsigned)std::min<size_t>(256, (geom.head_dim + 63) / 64 * 64));
    switch (geom.format) {
        case MARIN_KV_F32: kv_store_kernel<MARIN_KV_F32><<<grid, block, 0, g->stream>>>(keys, values, pages, geom, (uint32_t)start, (int)kv_heads); break;
        case MARIN_KV_F16: kv_store_kernel<MARIN_KV_F16><<<grid, block, 0, g->stream>>>(keys, values, pages, geom, (uint32_t)start, (int)kv_heads); break;
        default: kv_store_kernel<MARIN_KV_BF16><<<grid, block, 0, g->stream>>>(keys, values, pages, geom, (uint32_t)start, (int)kv_heads); break;
    }
    g->launched();
}

}  // namespace marin

using namespace marin;

// ---- DeviceKv (crates/cuda/src/kv.rs) ----
KvGeom marin_kv::geom(size_t layer) const {
    KvGeom g;
    g.page_shift = 6;  // MARIN_PAGE_TOKENS = 64
    g.head_dim = (uint32_t)head_dim;
    g.head_bytes = (uint64_t)MARIN_PAGE_TOKENS * head_dim * kv_elem_bytes(format);
    g.value_offset = g.head_bytes * kv_heads;
    // A slab is [layer][page][K, V][kv head][position][head value]: one layer's pages of a slab are one contiguous
    // run, so a layer's context spans few address-translation regions. A page pointer is its slab plus the page's
    // slot times one page-layer block, and every layer adds its own offset.
    g.layer_offset = (uint64_t)layer * MARIN_SLAB_PAGES * 2 * g.value_offset;
    g.format = (uint32_t)format;
    return g;
}

void marin_kv::reserve(size_t positions) {
    const size_t pages = (positions + MARIN_PAGE_TOKENS - 1) / MARIN_PAGE_TOKENS;
    size_t first_new = 0, needed = 0;
    if (!table.grow_to(pool, pages, first_new, needed)) shape("kv pages", pool.available(), needed);
    try {
        for (size_t i = first_new; i < table.ids.size(); ++i) {
            const size_t id = table.ids[i];
            const size_t slab = id / MARIN_SLAB_PAGES, slot = id % MARIN_SLAB_PAGES;
            if (slabs.size() <= slab) slabs.resize(slab + 1, nullptr);
            if (!slabs[slab]) {
                try {
                    slabs[slab] = gpu->alloc(slab_bytes(), true);
                } catch (const Error &e) {
                    size_t held = 0;
                    for (void *s : slabs) held += s ? slab_bytes() : 0;
                    Error k(MARIN_KV_MEMORY,
                            "the GPU could not allocate " + std::to_string(slab_bytes()) +
                                " more bytes for the KV cache, which holds " + std::to_string(held) + " bytes for " +
                                std::to_string(len) + " positions: " + e.what(),
                            held, slab_bytes(), len);
                    k.oom = e.oom;
                    throw k;
                }
            }
            host_ptrs[i] = (uint64_t)(uintptr_t)slabs[slab] + (uint64_t)slot * (page_bytes() / layers);
        }
        if (table.ids.size() > first_new) {
            const size_t n = table.ids.size() - first_new;
            void *staged = gpu->stage(&host_ptrs[first_new], n * 8);
            HIP_CHECK(hipMemcpyAsync(page_ptrs + first_new, staged, n * 8, hipMemcpyHostToDevice, gpu->stream));
            gpu->traffic.uploads++;
            gpu->traffic.upload_bytes += n * 8;
        }
    } catch (...) {
        table.shrink_to(pool, first_new);
        throw;
    }
}

extern "C" {

size_t marin_kv_startup_bytes(size_t layers, size_t heads, size_t kv_heads, size_t head_dim, size_t capacity,
                              marin_kv_format format) {
    const size_t row = kv_heads * head_dim * kv_elem_bytes(format);
    size_t slab, table, scratch;
    if (__builtin_mul_overflow(row, (size_t)MARIN_PAGE_TOKENS * MARIN_SLAB_PAGES * 2, &slab)) return 0;
    if (__builtin_mul_overflow(slab, layers, &slab)) return 0;
    table = std::max<size_t>(1, (capacity + MARIN_PAGE_TOKENS - 1) / MARIN_PAGE_TOKENS) * 8;
    scratch = attention_partial_floats(1, 8, heads, head_dim, capacity, 0) * 4 + attention_counters(1, 8, heads) * 4;
    return slab + table + scratch + 4;
}

marin_status marin_kv_new(marin_gpu *g, size_t layers, size_t heads, size_t kv_heads, size_t head_dim,
                          size_t capacity, marin_kv_format format, marin_kv **out) {
    return guard([&] {
        if (head_dim == 0 || head_dim > 256 || kv_heads == 0 || heads == 0 || heads % kv_heads != 0)
            unsupported("head layout", 256, head_dim);
        if (format != MARIN_KV_F32 && format != MARIN_KV_F16 && format != MARIN_KV_BF16)
            shape("kv format", 3, (size_t)format);
        size_t check;
        if (__builtin_mul_overflow(kv_heads * head_dim * 4, (size_t)MARIN_PAGE_TOKENS * MARIN_SLAB_PAGES * 2 * layers,
                                   &check))
            overflow("kv cache");
        auto *kv = new marin_kv();
        kv->gpu = g;
        kv->format = format;
        kv->layers = layers;
        kv->heads = heads;
        kv->kv_heads = kv_heads;
        kv->head_dim = head_dim;
        kv->capacity = capacity;
        kv->pool.limit = (capacity + MARIN_PAGE_TOKENS - 1) / MARIN_PAGE_TOKENS;
        kv->host_ptrs.assign(std::max<size_t>(kv->pool.limit, 1), 0);
        try {
            kv->page_ptrs = (uint64_t *)g->alloc(std::max<size_t>(kv->pool.limit, 1) * 8, true);
            kv->ctx = (uint32_t *)g->alloc(4, true);
            kv->partial_floats = attention_partial_floats(1, 8, heads, head_dim, std::max<size_t>(capacity, 1), g->cu_count);
            kv->partials = (float *)g->alloc(kv->partial_floats * 4, false);
            kv->counters = (uint32_t *)g->alloc(attention_counters(1, 8, heads) * 4, true);
        } catch (...) {
            marin_kv_free(kv);
            throw;
        }
        *out = kv;
    });
}

void marin_kv_free(marin_kv *kv) {
    if (!kv) return;
    (void)hipStreamSynchronize(kv->gpu->stream);
    for (void *s : kv->slabs) kv->gpu->release(s);
    kv->gpu->release(kv->page_ptrs);
    kv->gpu->release(kv->ctx);
    kv->gpu->release(kv->partials);
    kv->gpu->release(kv->counters);
    delete kv;
}

marin_status marin_kv_write(marin_gpu *g, marin_kv *kv, size_t layer, const marin_buffer *keys,
                            const marin_buffer *values) {
    return guard([&] {
        const size_t stride = kv->kv_heads * kv->head_dim;
        const size_t tokens = keys->len / stride;
        if (keys->len != tokens * stride || values->len != keys->len) shape("kv chunk", tokens * stride, keys->len);
        if (keys->dtype != MARIN_F32 || values->dtype != MARIN_F32) shape("kv chunk element size", 4, 2);
        const size_t end = kv->len + tokens;
        if (end > kv->capacity) shape("kv positions", kv->capacity, end);
        if (layer >= kv->layers) shape("kv layer", kv->layers, layer);
        kv->reserve(end);
        if (!tokens) return;
        launch_kv_store(g, (const float *)keys->data, (const float *)values->data, kv->page_ptrs, kv->geom(layer),
                        kv->len, tokens, kv->kv_heads);
    });
}

marin_status marin_kv_advance(marin_kv *kv, size_t tokens) {
    return guard([&] {
        if (kv->len + tokens > kv->capacity || kv->len + tokens < kv->len)
            shape("kv positions", kv->capacity, kv->len + tokens);
        kv->len += tokens;
    });
}

marin_status marin_kv_truncate(marin_kv *kv, size_t len) {
    return guard([&] {
        if (len > kv->len) shape("kv rollback", kv->len, len);
        kv->len = len;
        kv->table.shrink_to(kv->pool, (len + MARIN_PAGE_TOKENS - 1) / MARIN_PAGE_TOKENS);
    });
}

void marin_kv_clear(marin_kv *kv) {
    kv->len = 0;
    kv->table.shrink_to(kv->pool, 0);
}

size_t marin_kv_len(const marin_kv *kv) { return kv->len; }
int marin_kv_is_empty(const marin_kv *kv) { return kv->len == 0; }
marin_kv_format marin_kv_format_of(const marin_kv *kv) { return kv->format; }
size_t marin_kv_auxiliary_bytes(const marin_kv *kv) {
    // the split-attention scratch (partial records and chunk counters), the device page table and the context word
    return kv->partial_floats * 4 + attention_counters(1, 8, kv->heads) * 4 + std::max<size_t>(kv->pool.limit, 1) * 8 +
           4;
}
size_t marin_kv_capacity(const marin_kv *kv) { return kv->capacity; }
size_t marin_kv_pages_in_use(const marin_kv *kv) { return kv->table.ids.size(); }
size_t marin_kv_page_bytes(const marin_kv *kv) { return kv->page_bytes(); }
size_t marin_kv_slab_bytes(const marin_kv *kv) { return kv->slab_bytes(); }

size_t marin_kv_pages_held(const marin_kv *kv) {
    size_t held = 0;
    for (size_t i = 0; i < kv->slabs.size(); ++i) {
        if (!kv->slabs[i]) continue;
        const size_t first = i * MARIN_SLAB_PAGES;
        held += std::min<size_t>(MARIN_SLAB_PAGES, kv->pool.issued > first ? kv->pool.issued - first : 0);
    }
    return held;
}

size_t marin_kv_bytes_held(const marin_kv *kv) {
    size_t n = 0;
    for (void *s : kv->slabs) n += s ? 1 : 0;
    return n * kv->slab_bytes();
}

size_t marin_kv_page_ids(const marin_kv *kv, size_t *out, size_t cap) {
    for (size_t i = 0; i < kv->table.ids.size() && i < cap; ++i) out[i] = kv->table.ids[i];
    return kv->table.ids.size();
}

marin_status marin_attention(marin_gpu *g, const marin_buffer *q, marin_kv *kv, size_t layer, size_t heads,
                             size_t tokens, marin_buffer *out) {
    return guard([&] {
        const size_t hd = kv->head_dim;
        if (heads != kv->heads) shape("attention heads", kv->heads, heads);
        const size_t qlen = mul(mul(tokens, heads, "attention queries"), hd, "attention queries");
        check_len("attention queries", qlen, q->len);
        check_len("attention output", qlen, out->len);
        if (q->dtype != MARIN_F32 || out->dtype != MARIN_F32) shape("attention element size", 4, 2);
        const size_t visible = kv->len + tokens;
        if (visible > kv->capacity) shape("attention positions", kv->capacity, visible);
        if (layer >= kv->layers) shape("kv layer", kv->layers, layer);
        if (tokens == 0 || visible == 0) return;
        const size_t pages = (visible + MARIN_PAGE_TOKENS - 1) / MARIN_PAGE_TOKENS;
        if (pages > kv->table.ids.size()) shape("attention pages", pages, kv->table.ids.size());
        // Tokens go in groups of at most 8 (the partial scratch is sized for that); group j sees its own prefix.
        for (size_t t0 = 0; t0 < tokens; t0 += 8) {
            const size_t nt = std::min<size_t>(8, tokens - t0);
            const uint32_t ctx = (uint32_t)(kv->len + t0 + nt);
            void *staged = g->stage(&ctx, 4);
            HIP_CHECK(hipMemcpyAsync(kv->ctx, staged, 4, hipMemcpyHostToDevice, g->stream));
            AttentionArgs a{};
            a.q = (const float *)q->data + t0 * heads * hd;
            a.bf16_io = false;
            a.out = (float *)out->data + t0 * heads * hd;
            a.tables = kv->page_ptrs;
            a.table_stride = 0;
            a.table_len = std::max<size_t>(kv->pool.limit, 1);
            a.ctx = kv->ctx;
            a.batch = 1;
            a.tokens = nt;
            a.heads = heads;
            a.kv_heads = kv->kv_heads;
            a.geom = kv->geom(layer);
            a.max_ctx = ctx;
            a.partials = kv->partials;
            a.partial_floats = kv->partial_floats;
            a.counters = kv->counters;
            a.counter_count = attention_counters(1, 8, heads);
            launch_attention(g, a);
        }
    });
}

// ---- page pool shared by a batch of sequences ----
}  // extern "C"

struct marin_page_pool {
    marin_gpu *gpu = nullptr;
    size_t pages = 0, page_tokens = 0, kv_heads = 0, head_dim = 0;
    marin_kv_format format = MARIN_KV_BF16;
    uint8_t *base = nullptr;
    size_t page_bytes = 0;
    uint64_t *tables = nullptr;
    size_t table_cap = 0;
    uint32_t *ctx = nullptr;
    size_t ctx_cap = 0;
    float *partials = nullptr;
    size_t partial_floats = 0;
    uint32_t *counters = nullptr;
    size_t counter_count = 0;
    std::vector<uint64_t> last_tables;  // what the device copies hold, to skip unchanged uploads
    std::vector<uint32_t> last_ctx;
};

extern "C" {

marin_status marin_page_pool_new(marin_gpu *g, size_t pages, size_t page_tokens, size_t kv_heads, size_t head_dim,
                                 marin_kv_format format, marin_page_pool **out) {
    return guard([&] {
        if (page_tokens == 0 || (page_tokens & (page_tokens - 1)) != 0 || page_tokens > 4096)
            unsupported("page tokens (a power of two)", 4096, page_tokens);
        if (head_dim == 0 || head_dim > 256) unsupported("head size", 256, head_dim);
        auto *p = new marin_page_pool();
        p->gpu = g;
        p->pages = pages;
        p->page_tokens = page_tokens;
        p->kv_heads = kv_heads;
        p->head_dim = head_dim;
        p->format = format;
        p->page_bytes = mul(mul(2 * kv_heads, page_tokens, "page"), head_dim * kv_elem_bytes(format), "page");
        try {
            p->base = (uint8_t *)g->alloc(mul(pages, p->page_bytes, "page pool"), true);
        } catch (...) {
            delete p;
            throw;
        }
        *out = p;
    });
}

void marin_page_pool_free(marin_page_pool *p) {
    if (!p) return;
    (void)hipStreamSynchronize(p->gpu->stream);
    p->gpu->release(p->base);
    p->gpu->release(p->tables);
    p->gpu->release(p->ctx);
    p->gpu->release(p->partials);
    p->gpu->release(p->counters);
    delete p;
}

marin_status marin_page_pool_write(marin_gpu *g, marin_page_pool *p, size_t page, const void *data, size_t bytes) {
    return guard([&] {
        if (page >= p->pages) shape("page id", p->pages, page);
        check_len("page bytes", p->page_bytes, bytes);
        g->upload(p->base + page * p->page_bytes, data, bytes);
    });
}

marin_status marin_paged_attention_batch(marin_gpu *g, const marin_buffer *q, marin_page_pool *p,
                                         const uint32_t *tables, size_t table_stride, const uint32_t *ctx_lens,
                                         size_t batch, size_t heads, marin_buffer *out) {
    return guard([&] {
        const size_t hd = p->head_dim;
        if (heads == 0 || heads % p->kv_heads != 0) shape("attention heads", p->kv_heads, heads);
        const size_t qlen = mul(mul(batch, heads, "queries"), hd, "queries");
        check_len("attention queries", qlen, q->len);
        check_len("attention output", qlen, out->len);
        if (q->dtype != MARIN_BF16 || out->dtype != MARIN_BF16) shape("attention element size", 2, 4);
        size_t max_ctx = 0;
        std::vector<uint64_t> addr(batch * table_stride, 0);
        for (size_t b = 0; b < batch; ++b) {
            const size_t n = ctx_lens[b];
            if (n == 0) shape("context length", 1, 0);
            const size_t need = (n + p->page_tokens - 1) / p->page_tokens;
            if (need > table_stride) shape("page table length", table_stride, need);
            for (size_t i = 0; i < need; ++i) {
                const uint32_t id = tables[b * table_stride + i];
                if (id >= p->pages) shape("page id", p->pages, id);
                addr[b * table_stride + i] = (uint64_t)(uintptr_t)(p->base + (size_t)id * p->page_bytes);
            }
            max_ctx = std::max(max_ctx, n);
        }
        if (!batch) return;
        if (addr.size() > p->table_cap) {
            g->release(p->tables);
            p->tables = nullptr;
            p->tables = (uint64_t *)g->alloc(addr.size() * 8, false);
            p->table_cap = addr.size();
            p->last_tables.clear();
        }
        if (batch > p->ctx_cap) {
            g->release(p->ctx);
            p->ctx = nullptr;
            p->ctx = (uint32_t *)g->alloc(batch * 4, false);
            p->ctx_cap = batch;
            p->last_ctx.clear();
        }
        const size_t need_partials = attention_partial_floats(batch, 1, heads, hd, max_ctx, g->cu_count);
        if (need_partials > p->partial_floats) {
            g->release(p->partials);
            p->partials = nullptr;
            p->partials = (float *)g->alloc(need_partials * 4, false);
            p->partial_floats = need_partials;
        }
        const size_t need_counters = attention_counters(batch, 1, heads);
        if (need_counters > p->counter_count) {
            g->release(p->counters);
            p->counters = nullptr;
            p->counters = (uint32_t *)g->alloc(need_counters * 4, true);
            p->counter_count = need_counters;
        }
        if (p->last_tables != addr) {
            g->upload(p->tables, addr.data(), addr.size() * 8);
            p->last_tables = addr;
        }
        std::vector<uint32_t> ctxv(ctx_lens, ctx_lens + batch);
        if (p->last_ctx != ctxv) {
            g->upload(p->ctx, ctx_lens, batch * 4);
            p->last_ctx = ctxv;
        }
        AttentionArgs a{};
        a.q = q->data;
        a.bf16_io = true;
        a.out = out->data;
        a.tables = p->tables;
        a.table_stride = table_stride;
        a.table_len = table_stride;
        a.ctx = p->ctx;
        a.batch = batch;
        a.tokens = 1;
        a.heads = heads;
        a.kv_heads = p->kv_heads;
        a.geom.page_shift = (uint32_t)__builtin_ctzll(p->page_tokens);
        a.geom.head_dim = (uint32_t)hd;
        a.geom.head_bytes = (uint64_t)p->page_tokens * hd * kv_elem_bytes(p->format);
        a.geom.value_offset = a.geom.head_bytes * p->kv_heads;
        a.geom.layer_offset = 0;
        a.geom.format = (uint32_t)p->format;
        a.max_ctx = max_ctx;
        a.partials = p->partials;
        a.partial_floats = p->partial_floats;
        a.counters = p->counters;
        a.counter_count = p->counter_count;
        launch_attention(g, a);
    });
}

}  // extern "C"
