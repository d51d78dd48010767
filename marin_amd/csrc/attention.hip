// Paged KV cache and grouped-query decode attention on CDNA4 (crates/cuda/src/kv.rs, pages.rs, attention.rs and
// attention.cu of the reference, redesigned).
//
// Attention splits the visible context into chunks; a workgroup takes one chunk of one kv head for up to 8 query rows
// (the heads sharing that kv head, times the new tokens). Lanes are grouped per position: a group of LPP lanes covers
// one position's head with 8 contiguous values per lane (16-byte loads for bf16/f16), so a wave reads 64/LPP rows of
// a page per step and each key or value row is read once for all the rows of the group. Scores go to LDS; each chunk
// leaves its maximum, sum of weights and weighted values, and a merge kernel combines the chunks (log-sum-exp).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "attention.hpp"

namespace marin {

size_t kv_elem_bytes(marin_kv_format f) { return f == MARIN_KV_F32 ? 4 : 2; }

constexpr int ROWS = 8;         // query rows per workgroup
constexpr int MAX_CHUNK = 256;  // positions per workgroup
constexpr int MIN_CHUNK = 64;
constexpr int UNR = 8;  // position steps whose rows are loaded before any is used

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((unsigned)b << 16); }

// Eight values of a row starting at element d (d + 8 <= head_dim when VEC).
template <int F, bool VEC>
__device__ __forceinline__ void load8(const uint8_t *row, int d, int hd, float v[8]) {
    if constexpr (VEC) {
        if constexpr (F == MARIN_KV_F32) {
            const float4 a = *reinterpret_cast<const float4 *>(row + (size_t)d * 4);
            const float4 b = *reinterpret_cast<const float4 *>(row + (size_t)d * 4 + 16);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 u = *reinterpret_cast<const uint4 *>(row + (size_t)d * 2);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (F == MARIN_KV_F16) {
                    v[2 * i] = f16_bits_to_f32((uint16_t)(w[i] & 0xffffu));
                    v[2 * i + 1] = f16_bits_to_f32((uint16_t)(w[i] >> 16));
                } else {
                    v[2 * i] = __uint_as_float(w[i] << 16);
                    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
                }
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = d + i;
            float x = 0.0f;
            if (e < hd) {
                if constexpr (F == MARIN_KV_F32) x = reinterpret_cast<const float *>(row)[e];
                else if constexpr (F == MARIN_KV_F16) x = f16_bits_to_f32(reinterpret_cast<const uint16_t *>(row)[e]);
                else x = bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(row)[e]);
            }
            v[i] = x;
        }
    }
}

__device__ __forceinline__ const uint8_t *kv_row(const uint64_t *table, const KvGeom &g, int which, int kvh,
                                                 uint32_t pos) {
    const uint64_t page = table[pos >> g.page_shift];
    const uint32_t in_page = pos & ((1u << g.page_shift) - 1u);
    const size_t es = g.format == MARIN_KV_F32 ? 4 : 2;
    return reinterpret_cast<const uint8_t *>(page + g.layer_offset + (which ? g.value_offset : 0) +
                                             (uint64_t)kvh * g.head_bytes + (uint64_t)in_page * g.head_dim * es);
}

// grid: x = chunk (split), y = kv_head * row_groups + row_group, z = sequence. LPP lanes per position, R query rows
// (the heads of one kv head times the new tokens, in groups of R). The chunk's page addresses are read into LDS
// first, so every row address is computed without another memory round trip.
template <int F, int LPP, bool VEC, bool QBF16, int R>
__global__ __launch_bounds__(256) void attention_partial(const void *__restrict__ qv, const uint64_t *__restrict__ tables,
                                                         size_t table_stride, const uint32_t *__restrict__ ctx_lens,
                                                         KvGeom geom, int tokens, int heads, int kv_heads, int chunk,
                                                         int splits, float scale, float *__restrict__ part) {
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
    const int count = min(chunk, ctx - first);
    const int r0 = rg * R;
    const int nrows = min(R, total_rows - r0);
    const uint64_t *table = tables + (size_t)b * table_stride;
    const int d = sub * 8;
    const size_t es = F == MARIN_KV_F32 ? 4 : 2;
    const uint64_t head_off = (uint64_t)kvh * geom.head_bytes + geom.layer_offset;
    const uint32_t pmask = (1u << geom.page_shift) - 1u;

    __shared__ float w_s[R][MAX_CHUNK];
    __shared__ float red[4][R][8 * 32];  // wave partial accumulators (only head_dim used)
    __shared__ float ml_s[R][2];
    __shared__ uint64_t pages_s[MAX_CHUNK + 1];

    const int page0 = first >> geom.page_shift;
    const int npages = ((first + count - 1) >> geom.page_shift) - page0 + 1;
    for (int i = threadIdx.x; i < npages; i += 256) pages_s[i] = table[page0 + i] + head_off;

    // Query rows: row r = (token r / group, head kvh * group + r % group).
    float q[R][8];
    int visible[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int rr = r0 + r;
        const int t = rr / group, h = kvh * group + rr % group;
        visible[r] = ctx - tokens + t + 1;
#pragma unroll
        for (int i = 0; i < 8; ++i) q[r][i] = 0.0f;
        if (r < nrows && d < hd) {
            const size_t base = (((size_t)b * tokens + t) * heads + h) * hd;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (d + i < hd) {
                    if constexpr (QBF16) q[r][i] = bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(qv)[base + d + i]);
                    else q[r][i] = reinterpret_cast<const float *>(qv)[base + d + i];
                }
            }
        }
    }
    __syncthreads();
    auto row_ptr = [&](int which, int p) {
        const uint32_t pos = (uint32_t)(first + p);
        return reinterpret_cast<const uint8_t *>(pages_s[(pos >> geom.page_shift) - page0] +
                                                 (which ? geom.value_offset : 0) + (uint64_t)(pos & pmask) * hd * es);
    };

    // Scores: UNR rows per lane group are loaded before the dots, so each wave keeps UNR * 16 bytes per lane in flight.
    for (int p0 = wave * PPW; p0 < count; p0 += 4 * PPW * UNR) {
        float k[UNR][8];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int p = p0 + u * 4 * PPW + slot;
#pragma unroll
            for (int i = 0; i < 8; ++i) k[u][i] = 0.0f;
            if (p < count && d < hd) load8<F, VEC>(row_ptr(0, p), d, hd, k[u]);
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int p = p0 + u * 4 * PPW + slot;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float sc = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) sc += q[r][i] * k[u][i];
#pragma unroll
                for (int o = 1; o < LPP; o <<= 1) sc += __shfl_xor(sc, o);
                if (sub == 0 && p < count && r < nrows)
                    w_s[r][p] = (first + p < visible[r]) ? sc * scale : -INFINITY;
            }
        }
    }
    __syncthreads();

    // Softmax pieces per row: the chunk maximum, exp(score - max), their sum.
    for (int r = wave; r < nrows; r += 4) {
        float m = -INFINITY;
        for (int i = lane; i < count; i += 64) m = fmaxf(m, w_s[r][i]);
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        float l = 0.0f;
        for (int i = lane; i < count; i += 64) {
            const float e = m == -INFINITY ? 0.0f : expf(w_s[r][i] - m);
            w_s[r][i] = e;
            l += e;
        }
        for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o);
        if (lane == 0) {
            ml_s[r][0] = m;
            ml_s[r][1] = l;
        }
    }
    __syncthreads();

    // Weighted values.
    float acc[R][8];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[r][i] = 0.0f;
    for (int p0 = wave * PPW; p0 < count; p0 += 4 * PPW * UNR) {
        float v[UNR][8];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int p = p0 + u * 4 * PPW + slot;
#pragma unroll
            for (int i = 0; i < 8; ++i) v[u][i] = 0.0f;
            if (p < count && d < hd) load8<F, VEC>(row_ptr(1, p), d, hd, v[u]);
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int p = p0 + u * 4 * PPW + slot;
            if (p < count) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float wgt = w_s[r][p];
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[r][i] += wgt * v[u][i];
                }
            }
        }
    }
    // Reduce over the position slots of the wave (lanes with the same sub), then over the waves.
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int o = LPP; o < 64; o <<= 1) acc[r][i] += __shfl_xor(acc[r][i], o);
    if (slot == 0 && d < hd) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (d + i < 8 * 32) red[wave][r][d + i] = acc[r][i];
    }
    __syncthreads();
    for (int o = threadIdx.x; o < nrows * hd; o += 256) {
        const int r = o / hd, e = o % hd;
        const float v = (red[0][r][e] + red[1][r][e]) + (red[2][r][e] + red[3][r][e]);
        const int rr = r0 + r;
        const int t = rr / group, h = kvh * group + rr % group;
        const size_t unit = (((size_t)b * tokens + t) * heads + h) * splits + split;
        part[unit * (hd + 2) + 2 + e] = v;
        if (e == 0) {
            part[unit * (hd + 2)] = ml_s[r][0];
            part[unit * (hd + 2) + 1] = ml_s[r][1];
        }
    }
}

// Combines the chunks of one (sequence, token, head): out = sum_s acc_s e^{m_s - M} / sum_s l_s e^{m_s - M}. The
// chunks' weights e^{m_s - M} are computed once into LDS, then each thread sums one element over the chunks.
template <int OUT>
__global__ __launch_bounds__(256) void attention_merge(const float *__restrict__ part,
                                                       const uint32_t *__restrict__ ctx_lens, int tokens, int heads,
                                                       int hd, int chunk, int splits, void *__restrict__ out) {
    extern __shared__ float ws[];  // [splits] weights, then the total
    const int unit = blockIdx.x;  // (b * tokens + t) * heads + h
    const int b = unit / (tokens * heads);
    const int used = min(splits, (int)((ctx_lens[b] + chunk - 1) / chunk));
    const float *p = part + (size_t)unit * splits * (hd + 2);
    __shared__ float red[4];
    float m = -INFINITY;
    for (int s = threadIdx.x; s < used; s += blockDim.x) m = fmaxf(m, p[(size_t)s * (hd + 2)]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) m = fmaxf(m, red[w]);
    for (int s = threadIdx.x; s < used; s += blockDim.x) {
        const float ms = p[(size_t)s * (hd + 2)];
        ws[s] = ms == -INFINITY ? 0.0f : expf(ms - m);
    }
    __syncthreads();
    float total = 0.0f;
    for (int s = 0; s < used; ++s) total += p[(size_t)s * (hd + 2) + 1] * ws[s];
    for (int e = threadIdx.x; e < hd; e += blockDim.x) {
        float acc = 0.0f;
        for (int s = 0; s < used; ++s) acc += p[(size_t)s * (hd + 2) + 2 + e] * ws[s];
        const float v = acc / total;
        const size_t at = (size_t)unit * hd + e;
        if constexpr (OUT == 0) reinterpret_cast<float *>(out)[at] = v;
        if constexpr (OUT == 1) {
            const unsigned u = __float_as_uint(v);
            reinterpret_cast<uint16_t *>(out)[at] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        }
    }
}

// Positions per workgroup: enough workgroups for about two per compute unit, 64 to 256 positions each.
static int chunk_for(size_t max_ctx, size_t blocks_per_chunk, int cu_count) {
    const size_t wanted = std::max<size_t>(1, (2 * (size_t)std::max(cu_count, 1) + blocks_per_chunk - 1) /
                                                  std::max<size_t>(blocks_per_chunk, 1));
    size_t chunk = (max_ctx + wanted - 1) / wanted;
    chunk = std::min<size_t>(MAX_CHUNK, std::max<size_t>(MIN_CHUNK, chunk));
    return (int)chunk;
}

size_t attention_partial_floats(size_t batch, size_t tokens, size_t heads, size_t head_dim, size_t max_ctx,
                                int cu_count) {
    (void)cu_count;
    const size_t splits = (max_ctx + MIN_CHUNK - 1) / MIN_CHUNK;
    return batch * tokens * heads * std::max<size_t>(splits, 1) * (head_dim + 2);
}

template <int F, int LPP, bool VEC, int R>
static void launch_partial_r(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    if (a.q_bf16)
        attention_partial<F, LPP, VEC, true, R><<<grid, dim3(256), 0, g->stream>>>(
            a.q, a.tables, a.table_stride, a.ctx, a.geom, (int)a.tokens, (int)a.heads, (int)a.kv_heads, chunk, splits,
            scale, a.partials);
    else
        attention_partial<F, LPP, VEC, false, R><<<grid, dim3(256), 0, g->stream>>>(
            a.q, a.tables, a.table_stride, a.ctx, a.geom, (int)a.tokens, (int)a.heads, (int)a.kv_heads, chunk, splits,
            scale, a.partials);
}

static int rows_per_block(const AttentionArgs &a) {
    const size_t rows = a.tokens * (a.heads / a.kv_heads);
    return rows <= 2 ? 2 : (rows <= 4 ? 4 : ROWS);
}

template <int F, int LPP, bool VEC>
static void launch_partial(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    const int r = rows_per_block(a);
    if (r == 2) launch_partial_r<F, LPP, VEC, 2>(g, a, grid, chunk, splits, scale);
    else if (r == 4) launch_partial_r<F, LPP, VEC, 4>(g, a, grid, chunk, splits, scale);
    else launch_partial_r<F, LPP, VEC, ROWS>(g, a, grid, chunk, splits, scale);
}

template <int F>
static void launch_partial_f(marin_gpu *g, const AttentionArgs &a, dim3 grid, int chunk, int splits, float scale) {
    const int hd = (int)a.geom.head_dim;
    const bool vec = hd % 8 == 0;
    int lpp = 1;
    while (lpp * 8 < hd) lpp <<= 1;
#define MARIN_P(L)                                                                    \
    do {                                                                              \
        if (vec) launch_partial<F, L, true>(g, a, grid, chunk, splits, scale);        \
        else launch_partial<F, L, false>(g, a, grid, chunk, splits, scale);           \
    } while (0)
    switch (lpp) {
        case 1: MARIN_P(1); break;
        case 2: MARIN_P(2); break;
        case 4: MARIN_P(4); break;
        case 8: MARIN_P(8); break;
        case 16: MARIN_P(16); break;
        default: MARIN_P(32); break;
    }
#undef MARIN_P
}

void launch_attention(marin_gpu *g, const AttentionArgs &a) {
    const size_t group = a.heads / a.kv_heads;
    const size_t rpb = (size_t)rows_per_block(a);
    const size_t row_groups = (a.tokens * group + rpb - 1) / rpb;
    const int chunk = chunk_for(a.max_ctx, a.kv_heads * row_groups * a.batch, g->cu_count);
    const int splits = (int)((a.max_ctx + chunk - 1) / chunk);
    if ((size_t)splits * a.batch * a.tokens * a.heads * (a.geom.head_dim + 2) > a.partial_floats)
        shape("attention partial sums", (size_t)splits * a.batch * a.tokens * a.heads * (a.geom.head_dim + 2),
              a.partial_floats);
    const float scale = 1.0f / sqrtf((float)a.geom.head_dim);
    dim3 grid((unsigned)splits, (unsigned)(a.kv_heads * row_groups), (unsigned)a.batch);
    switch (a.geom.format) {
        case MARIN_KV_F32: launch_partial_f<MARIN_KV_F32>(g, a, grid, chunk, splits, scale); break;
        case MARIN_KV_F16: launch_partial_f<MARIN_KV_F16>(g, a, grid, chunk, splits, scale); break;
        default: launch_partial_f<MARIN_KV_BF16>(g, a, grid, chunk, splits, scale); break;
    }
    g->launched(marin_gpu::ATTENTION, a.bytes_hint);
    const dim3 mgrid((unsigned)(a.batch * a.tokens * a.heads));
    const dim3 mblock((unsigned)std::min<size_t>(256, (a.geom.head_dim + 63) / 64 * 64));
    const size_t mlds = (size_t)splits * 4;
    if (a.out_kind == 0)
        attention_merge<0><<<mgrid, mblock, mlds, g->stream>>>(a.partials, a.ctx, (int)a.tokens, (int)a.heads,
                                                               (int)a.geom.head_dim, chunk, splits, a.out);
    else
        attention_merge<1><<<mgrid, mblock, mlds, g->stream>>>(a.partials, a.ctx, (int)a.tokens, (int)a.heads,
                                                               (int)a.geom.head_dim, chunk, splits, a.out);
    g->launched(marin_gpu::ATTENTION, 0.0);
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
            uint8_t *row = const_cast<uint8_t *>(kv_row(pages, geom, which, kvh, start + t));
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
    g.layer_offset = (uint64_t)layer * 2 * g.value_offset;
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
            host_ptrs[i] = (uint64_t)(uintptr_t)slabs[slab] + (uint64_t)slot * page_bytes();
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
    scratch = attention_partial_floats(1, 8, heads, head_dim, capacity, 0) * 4;
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
            a.q_bf16 = false;
            a.out = (float *)out->data + t0 * heads * hd;
            a.out_kind = 0;
            a.tables = kv->page_ptrs;
            a.table_stride = 0;
            a.ctx = kv->ctx;
            a.batch = 1;
            a.tokens = nt;
            a.heads = heads;
            a.kv_heads = kv->kv_heads;
            a.geom = kv->geom(layer);
            a.max_ctx = ctx;
            a.partials = kv->partials;
            a.partial_floats = kv->partial_floats;
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
        a.q_bf16 = true;
        a.out = out->data;
        a.out_kind = 1;
        a.tables = p->tables;
        a.table_stride = table_stride;
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
        launch_attention(g, a);
    });
}

}  // extern "C"
