// Paged KV storage and the split-context decode attention kernels.
#pragma once

#include <vector>

#include "common.hpp"

namespace marin {

// Where a layer's keys and values are for the kernels. A page holds `1 << page_shift` positions laid out
// [layer][keys, values][kv_head][position in page][head_dim], so one kv head's rows of a page are contiguous.
struct KvGeom {
    uint32_t page_shift;
    uint32_t head_dim;
    uint64_t layer_offset;  // bytes from a page's start to this layer's keys
    uint64_t value_offset;  // bytes from a layer's keys to its values
    uint64_t head_bytes;    // bytes of one kv head's rows in a page
    uint32_t format;        // marin_kv_format
};

// The reference's page bookkeeping (crates/cuda/src/pages.rs:20-110): freed pages are handed out again before any
// new id, most recently freed first; grow_to is all-or-nothing; shrink_to gives pages back lowest position first.
struct PagePool {
    size_t limit = 0, issued = 0;
    std::vector<size_t> freed;
    size_t available() const { return freed.size() + (limit - issued); }
    size_t take() {
        if (!freed.empty()) {
            size_t id = freed.back();
            freed.pop_back();
            return id;
        }
        return issued++;
    }
    void give(size_t id) { freed.push_back(id); }
};

struct PageTable {
    std::vector<size_t> ids;
    // Returns where the new pages start; changes nothing (returns false) when the pool cannot supply them all.
    bool grow_to(PagePool &pool, size_t pages, size_t &first_new, size_t &needed) {
        first_new = ids.size();
        needed = pages > ids.size() ? pages - ids.size() : 0;
        if (needed > pool.available()) return false;
        for (size_t i = 0; i < needed; ++i) ids.push_back(pool.take());
        return true;
    }
    void shrink_to(PagePool &pool, size_t pages) {
        while (ids.size() > pages) {
            // lowest position first: pop from the front of the removed range
            size_t first = pages;
            pool.give(ids[first]);
            ids.erase(ids.begin() + first);
        }
    }
};

size_t kv_elem_bytes(marin_kv_format f);

// Attention of `tokens` new tokens of `batch` sequences. q/out: [batch][tokens][heads][head_dim] in q_bf16/out_*
// types. tables: device u64 page addresses [batch][table_stride]. ctx: device u32 [batch] (visible positions
// including the new tokens). Partials must hold batch*tokens*heads*splits*(head_dim+2) floats.
// Raw projections for the fused path: q and the new tokens' keys and values as [tokens][heads + 2 kv_heads][hd] f32,
// with the q/k RMSNorm weights and the RoPE frequency table (batch 1).
struct AttnFuse {
    const float *qkv = nullptr;
    const float *q_norm = nullptr, *k_norm = nullptr, *freq = nullptr;
    const float2 *rope = nullptr;  // cos/sin of every position, [pos][hd/2] (required by the one-token kernel)
    float eps = 0.0f;
};

struct AttentionArgs {
    const void *q;   // [batch][tokens][heads][head_dim], f32 or bf16 (bf16_io); unused with fuse.qkv
    bool bf16_io;    // q and out in bf16 instead of f32
    void *out;
    AttnFuse fuse;   // fuse.qkv set: q/k norm + RoPE + the store of the new keys/values happen in the kernel
    const uint64_t *tables;
    size_t table_stride;
    size_t table_len = 0;  // entries of one sequence's table (the one-token kernel reads its entries before ctx)
    const uint32_t *ctx;  // device
    size_t batch, tokens, heads, kv_heads;
    KvGeom geom;
    size_t max_ctx;  // bound on every ctx[b], sets the grid
    float *partials;
    size_t partial_floats;
    uint32_t *counters;  // zero-initialized; every launch leaves them zero
    size_t counter_count;
    double bytes_hint = 0.0;  // algorithmic bytes, for launch accounting only
};
size_t attention_partial_floats(size_t batch, size_t tokens, size_t heads, size_t head_dim, size_t max_ctx,
                                int cu_count);
// Chunk counters a launch of `batch` sequences of `tokens` new tokens can use.
size_t attention_counters(size_t batch, size_t tokens, size_t heads);

// Prompt attention on the matrix cores (attention_fa.hip): one sequence, 16+ tokens, f16 cache, head size 64 or 128,
// 1, 2, 4 or 8 q heads per kv head; its q scratch lives in the partial records.
size_t prefill_fa_scratch(size_t tokens, size_t heads, size_t hd);
bool prefill_fa_fits(const AttentionArgs &a);
void launch_prefill_fa(marin_gpu *g, const AttentionArgs &a);
void launch_attention(marin_gpu *g, const AttentionArgs &a);

// Stores f32 keys/values [tokens][kv_heads*head_dim] at positions start.. of one layer.
void launch_kv_store(marin_gpu *g, const float *keys, const float *values, const uint64_t *pages, const KvGeom &geom,
                     size_t start, size_t tokens, size_t kv_heads);

}  // namespace marin

struct marin_kv {
    marin_gpu *gpu = nullptr;
    marin_kv_format format = MARIN_KV_F32;
    size_t layers = 0, heads = 0, kv_heads = 0, head_dim = 0, capacity = 0, len = 0;
    marin::PagePool pool;
    marin::PageTable table;
    std::vector<void *> slabs;
    uint64_t *page_ptrs = nullptr;  // device, pool.limit entries
    std::vector<uint64_t> host_ptrs;
    uint32_t *ctx = nullptr;  // device scalar used by the kernels
    float *partials = nullptr;
    size_t partial_floats = 0;
    uint32_t *counters = nullptr;

    size_t row_bytes() const { return kv_heads * head_dim * marin::kv_elem_bytes(format); }
    size_t page_bytes() const { return row_bytes() * MARIN_PAGE_TOKENS * layers * 2; }
    size_t slab_bytes() const { return page_bytes() * MARIN_SLAB_PAGES; }
    marin::KvGeom geom(size_t layer) const;
    void reserve(size_t positions);  // maps pages for positions [0, positions); all-or-nothing
};
