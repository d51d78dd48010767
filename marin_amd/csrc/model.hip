// The Qwen3 decode pass over this backend (model/src/qwen3/gpu.rs:222-377 Qwen3Gpu::pass, weight.rs, workspace.rs of
// the reference), with MI355X-first fusion:
//  - q, k and v are one matrix (rows q | k | v), so the three projections are one weight stream;
//  - gate and up are interleaved row by row, so the GEMV epilogue sees (gate_i, up_i) in one lane and writes
//    silu(gate) * up straight into the f16 split the down projection reads;
//  - the o and down projections add into the residual stream in their epilogue;
//  - q/k RMSNorm, RoPE and the KV-cache store are one kernel;
//  - the input RMSNorm, post-attention RMSNorm and final norm run inside the prologue of the product that consumes
//    them (each block normalizes the row while its first weights are in flight), so no norm kernel remains;
//  - the greedy choice is an atomic max in the output head's epilogue, and one small kernel then records the token,
//    advances the positions and embeds the token for the next step.
// A decode step is 7 launches per layer plus 2. Positions live in device memory (pos, ctx), so a step has no host
// arguments and replays as a HIP graph: the greedy loop never returns to the host.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <string>

#include "attention.hpp"
#include "ops.hpp"
#include "gemm.hpp"
#include "gemv.hpp"

using namespace marin;

namespace marin {

constexpr size_t MAX_ROWS = 8;  // tokens of a forward_rows pass (model/src/qwen3/gpu.rs:118-119)
constexpr size_t CHUNK = 512;  // tokens per prompt pass through the layers (the products run as GEMMs)

// One decode step's bookkeeping, after the output head left the greedy choice in *best as (total-order key, ~id)
// (sampler/src/lib.rs:40-48: largest logit, lowest id on ties): record the token, clear the choice for the next
// head, advance the state (pos += 1, ctx = pos + 1, step += 1) and embed the token's table row into hidden.
// One int8 embedding row (code x scale, the windowed layout) written by a block: every thread issues all the loads of
// a pass before its first store, so the pass costs one memory round trip instead of one per element.
__device__ __forceinline__ void embed_row(const uint8_t *__restrict__ codes, const float *__restrict__ scales,
                                          size_t row, int cols, int group, float *__restrict__ dst) {
    constexpr int U = 8;
    const int groups = cols / group;
    const float *srow = scales + (row / 16) * (size_t)groups * 16 + (row % 16);
    for (int base = 0; base < cols; base += U * (int)blockDim.x) {
        int cv[U];
        float sv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = min(base + (int)threadIdx.x + u * (int)blockDim.x, cols - 1);
            cv[u] = (int8_t)codes[code_offset(row, i, cols, true, 16)];
            sv[u] = srow[(i / group) * 16];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = base + (int)threadIdx.x + u * (int)blockDim.x;
            if (i < cols) dst[i] = (float)cv[u] * sv[u];
        }
    }
}

__global__ __launch_bounds__(512) void advance(unsigned long long *best, uint32_t *ids, uint32_t *tokens_out,
                                               uint32_t *state, const uint8_t *__restrict__ codes,
                                               const float *__restrict__ scales, float *__restrict__ hidden, int cols,
                                               int group, uint32_t vocab) {
    __shared__ uint32_t id_s;
    if (threadIdx.x == 0) {
        // an empty choice word (no head block wrote one) would decode to 0xffffffff: the id is kept inside the table
        const uint32_t id = min(0xffffffffu - (uint32_t)(*best & 0xffffffffull), vocab - 1);
        *best = 0ull;
        ids[0] = id;
        tokens_out[state[2]] = id;
        state[0] += 1;
        state[1] = state[0] + 1;
        state[2] += 1;
        id_s = id;
    }
    __syncthreads();
    embed_row(codes, scales, id_s, cols, group, hidden);
}

// The greedy choice of one logits row (sampler/src/lib.rs:40-48: largest under f32's total order, lowest index on
// ties), as the key the products' fused argmax leaves: (total-order key << 32) | ~index. One block.
__global__ __launch_bounds__(1024) void argmax_row(const float *__restrict__ row, int n, unsigned long long *best) {
    __shared__ unsigned long long part[16];
    unsigned long long k = 0ull;
    for (int i = threadIdx.x; i < n; i += 1024) {
        const int b = __float_as_int(row[i]);
        const unsigned key = (unsigned)(b ^ (int)(((unsigned)(b >> 31)) >> 1)) ^ 0x80000000u;
        const unsigned long long v = (unsigned long long)key << 32 | (unsigned long long)(0xffffffffu - (unsigned)i);
        k = v > k ? v : k;
    }
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long other = __shfl_xor(k, o);
        k = other > k ? other : k;
    }
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w) k = part[w] > k ? part[w] : k;
        *best = k;
    }
}

// Sets the device state for a pass of `count` tokens at `pos` (pos, ctx = pos + count) and clears the greedy choice
// the pass's output head will make.
__global__ void set_state(uint32_t *state, uint32_t pos, uint32_t count, unsigned long long *best) {
    state[0] = pos;
    state[1] = pos + count;
    *best = 0ull;
}

__global__ void embed_device_ids(const uint8_t *__restrict__ codes, const float *__restrict__ scales,
                                 const uint32_t *__restrict__ ids, float *__restrict__ out, int cols, int group) {
    const size_t row = ids[blockIdx.x];
    const int groups = cols / group;
    const float *srow = scales + (row / 16) * (size_t)groups * 16 + (row % 16);
    for (int i = threadIdx.x; i < cols; i += blockDim.x)
        out[(size_t)blockIdx.x * cols + i] =
            (float)(int8_t)codes[code_offset(row, i, cols, true, 16)] * srow[(i / group) * 16];
}

// A decode batch's bookkeeping (one workgroup per sequence b): the greedy choice best[b] of the last pass becomes
// the sequence's token (recorded at tokens_out[step * batch + b]), the choice is cleared, the sequence's position
// advances (pos[b] += 1, ctx[b] = pos[b] + 1, step[b] += 1) and the token's table row is embedded into hidden[b].
// state: pos [batch] | ctx [batch] | step [batch].
__global__ __launch_bounds__(512) void advance_batch(unsigned long long *best, uint32_t *tokens_out, uint32_t *state,
                                                     int batch, const uint8_t *__restrict__ codes,
                                                     const float *__restrict__ scales, float *__restrict__ hidden,
                                                     int cols, int group, uint32_t vocab) {
    __shared__ uint32_t id_s;
    const int b = blockIdx.x;
    if (threadIdx.x == 0) {
        const uint32_t id = min(0xffffffffu - (uint32_t)(best[b] & 0xffffffffull), vocab - 1);
        best[b] = 0ull;
        tokens_out[(size_t)state[2 * batch + b] * batch + b] = id;
        state[b] += 1;
        state[batch + b] = state[b] + 1;
        state[2 * batch + b] += 1;
        id_s = id;
    }
    __syncthreads();
    embed_row(codes, scales, id_s, cols, group, hidden + (size_t)b * cols);
}

}  // namespace marin

struct Layer {
    marin_quant_matrix *qkv = nullptr, *o = nullptr, *gate_up = nullptr, *down = nullptr;
    float *input_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

struct marin_qwen3 {
    marin_gpu *gpu = nullptr;
    marin_qwen3_config cfg{};
    std::vector<Layer> layers;
    marin_quant_matrix *embed = nullptr, *lm_head = nullptr;
    float *final_norm = nullptr;
    float *freq = nullptr;
    size_t qd() const { return cfg.heads * cfg.head_dim; }
    size_t kvd() const { return cfg.kv_heads * cfg.head_dim; }
    const marin_quant_matrix *head() const { return lm_head ? lm_head : embed; }
};

struct marin_qwen3_cache {
    marin_qwen3 *model = nullptr;
    marin_kv *kv = nullptr;
    // device workspace, CHUNK tokens
    float *hidden = nullptr, *qkv = nullptr, *ctx = nullptr, *act = nullptr, *logits = nullptr;
    uint32_t *ids = nullptr, *state = nullptr, *tokens_out = nullptr;
    unsigned long long *best = nullptr;  // greedy choice of the last pass (key, ~id)
    size_t tokens_cap = 0;
    float *attn_partials = nullptr;
    size_t attn_partial_floats = 0;
    uint32_t *attn_counters = nullptr;
    float2 *rope = nullptr;  // RoPE cos/sin of every position of the capacity
    float *rows = nullptr;   // forward_rows: logits of every row of a pass, [MAX_ROWS][vocab]
    hipGraphExec_t graph = nullptr;
    size_t graph_capacity_ctx = 0;
};

// A decode batch: `seqs` sequences, each with its own KV cache (prefilled one at a time through its own cache),
// decoded together: one token per sequence per step, every product over the whole batch (weights read once), one
// attention launch over all sequences through a combined page-address table.
struct marin_qwen3_batch {
    marin_qwen3 *model = nullptr;
    std::vector<marin_qwen3_cache *> seqs;
    float *hidden = nullptr, *qkv = nullptr, *ctx = nullptr, *act = nullptr, *logits = nullptr;
    unsigned long long *best = nullptr;  // [batch] greedy choices
    uint32_t *state = nullptr;           // pos [batch] | ctx [batch] | step [batch]
    uint64_t *tables = nullptr;          // [batch][table_stride] page addresses
    size_t table_stride = 0;
    std::vector<uint64_t> host_tables;
    uint32_t *tokens_out = nullptr;  // [steps][batch]
    size_t tokens_cap = 0;           // steps
    float *partials = nullptr;
    size_t partial_floats = 0;
    uint32_t *counters = nullptr;
    size_t counter_count = 0;
    size_t capacity = 0;
    hipGraphExec_t graph = nullptr;
};

static void check_config(const marin_qwen3_config *c) {
    if (!c->layers || !c->hidden || !c->heads || !c->kv_heads || !c->head_dim || !c->ffn || !c->vocab)
        shape("qwen3 config", 1, 0);
    if (c->heads % c->kv_heads) shape("attention heads", c->kv_heads, c->heads);
    if (c->head_dim > 256 || c->head_dim % 2) unsupported("head size (even)", 256, c->head_dim);
    if (c->group == 0 || c->group % 64 || c->hidden % c->group || c->ffn % c->group ||
        (c->heads * c->head_dim) % c->group)
        shape("quantization group (a multiple of 64 dividing every width)", c->group, c->hidden);
}

static float *device_ones(marin_gpu *g, size_t n) {
    std::vector<float> ones(n, 1.0f);
    float *d = (float *)g->alloc(n * 4, false);
    g->upload(d, ones.data(), n * 4);
    return d;
}

static marin_qwen3 *alloc_model(marin_gpu *g, const marin_qwen3_config *cfg) {
    check_config(cfg);
    auto m = std::make_unique<marin_qwen3>();
    m->gpu = g;
    m->cfg = *cfg;
    const size_t H = cfg->hidden, qd = cfg->heads * cfg->head_dim, kvd = cfg->kv_heads * cfg->head_dim;
    m->layers.resize(cfg->layers);
    try {
        for (auto &L : m->layers) {
            L.qkv = new_quant_matrix(g, qd + 2 * kvd, H, 8, cfg->group, false);
            L.o = new_quant_matrix(g, H, qd, 8, cfg->group, false);
            L.gate_up = new_quant_matrix(g, 2 * cfg->ffn, H, 8, cfg->group, false);
            L.down = new_quant_matrix(g, H, cfg->ffn, 8, cfg->group, false);
            L.input_norm = device_ones(g, H);
            L.post_norm = device_ones(g, H);
            L.q_norm = device_ones(g, cfg->head_dim);
            L.k_norm = device_ones(g, cfg->head_dim);
        }
        m->embed = new_quant_matrix(g, cfg->vocab, H, 8, cfg->group, false);
        if (!cfg->tie_embeddings) m->lm_head = new_quant_matrix(g, cfg->vocab, H, 8, cfg->group, false);
        m->final_norm = device_ones(g, H);
        m->freq = make_rope_frequencies(g, cfg->head_dim, cfg->rope_theta);
    } catch (...) {
        marin_qwen3_free(m.release());
        throw;
    }
    return m.release();
}

// Where tensor `tensor` of a layer lands in the fused matrices: (matrix, first row, row step).
static void placement(marin_qwen3 *m, int layer, int tensor, marin_quant_matrix *&mat, size_t &row0, size_t &step,
                      size_t &rows, size_t &cols) {
    const size_t H = m->cfg.hidden, qd = m->qd(), kvd = m->kvd(), F = m->cfg.ffn;
    step = 1;
    row0 = 0;
    if (layer < 0) {
        if (tensor == 0) mat = m->embed;
        else if (tensor == 1 && m->lm_head) mat = m->lm_head;
        else shape("model tensor", 1, (size_t)tensor);
        rows = m->cfg.vocab;
        cols = H;
        return;
    }
    if ((size_t)layer >= m->layers.size()) shape("layer", m->layers.size(), (size_t)layer);
    Layer &L = m->layers[layer];
    switch (tensor) {
        case 0: mat = L.qkv; rows = qd; cols = H; break;
        case 1: mat = L.qkv; row0 = qd; rows = kvd; cols = H; break;
        case 2: mat = L.qkv; row0 = qd + kvd; rows = kvd; cols = H; break;
        case 3: mat = L.o; rows = H; cols = qd; break;
        case 4: mat = L.gate_up; row0 = 0; step = 2; rows = F; cols = H; break;
        case 5: mat = L.gate_up; row0 = 1; step = 2; rows = F; cols = H; break;
        case 6: mat = L.down; rows = H; cols = F; break;
        default: shape("layer tensor", 7, (size_t)tensor);
    }
}

// Synthetic tensor streams (same numbering as oracle/qwen3_synth.c): embed 1, lm_head 2, layer l tensor i:
// ((l + 1) << 8) | i.
static uint64_t synth_stream(int layer, int tensor) {
    if (layer < 0) return tensor == 0 ? 1u : 2u;
    return ((uint64_t)(layer + 1) << 8) | (uint64_t)tensor;
}

static void free_cache_graph(marin_qwen3_cache *c) {
    if (c->graph) {
        unregister_graph(c->graph);
        (void)hipGraphExecDestroy(c->graph);
        c->graph = nullptr;
    }
}

// What a pass reads and writes: `batch` sequences of `tokens` tokens each (rows batch * tokens, sequence-major),
// their embeddings in `hidden`; attention through `tables` (sequence b's page addresses at b * table_stride) with
// the sequences' context lengths in `ctx_lens`.
struct PassIo {
    float *hidden, *qkv, *ctx, *act, *logits;
    unsigned long long *best;
    const uint64_t *tables;
    size_t table_stride;
    const uint32_t *ctx_lens;
    size_t batch, tokens;
    const marin_kv *kv;  // geometry and format (shared by every sequence)
    float *partials;
    size_t partial_floats;
    uint32_t *counters;
    size_t counter_count;
    const float2 *rope;
    float *rows;  // set: the head runs over every row into rows [tokens][vocab] (one sequence)
};

static PassIo io_of(marin_qwen3_cache *c, size_t n) {
    return PassIo{c->hidden, c->qkv, c->ctx, c->act, c->logits, c->best, c->kv->page_ptrs, 0, c->state + 1, 1, n,
                  c->kv, c->attn_partials, c->attn_partial_floats, c->attn_counters,
                  attention_counters(1, CHUNK, c->model->cfg.heads), c->rope, nullptr};
}

// One pass at the positions in the device state, whose embeddings are already in io.hidden. With one sequence,
// writes the last token's logits and greedy choice; with a batch (one token per sequence), every sequence's logits
// and greedy choice (best[b]). `max_ctx` bounds the context for the attention grid; `host_ctx` (when known) only
// feeds launch accounting.
static void pass(marin_qwen3 *m, const PassIo &io, size_t max_ctx, size_t host_ctx = 0, bool head_out = true) {
    marin_gpu *g = m->gpu;
    const auto &cfg = m->cfg;
    const size_t H = cfg.hidden, qd = m->qd(), kvd = m->kvd(), F = cfg.ffn;
    const size_t n = io.batch * io.tokens;  // rows of every product
    for (size_t l = 0; l < m->layers.size(); ++l) {
        Layer &L = m->layers[l];
        GemvIn norm_in;
        norm_in.mode = IN_NORM;
        norm_in.x = io.hidden;
        norm_in.x_stride = H;
        norm_in.norm = L.input_norm;
        norm_in.eps = cfg.rms_eps;
        GemvOut qkv_out;
        qkv_out.mode = OUT_F32;
        qkv_out.y = io.qkv;
        qkv_out.y_stride = qd + 2 * kvd;
        launch_product(g, L.qkv, norm_in, qkv_out, n);
        AttentionArgs a{};
        a.q = nullptr;
        a.bf16_io = false;
        a.out = io.ctx;
        a.fuse.qkv = io.qkv;
        a.fuse.q_norm = L.q_norm;
        a.fuse.k_norm = L.k_norm;
        a.fuse.freq = m->freq;
        a.fuse.rope = io.rope;
        a.fuse.eps = cfg.rms_eps;
        a.tables = io.tables;
        a.table_stride = io.table_stride;
        a.table_len = io.table_stride ? io.table_stride : std::max<size_t>(io.kv->pool.limit, 1);
        a.ctx = io.ctx_lens;
        a.batch = io.batch;
        a.tokens = io.tokens;
        a.heads = cfg.heads;
        a.kv_heads = cfg.kv_heads;
        a.geom = io.kv->geom(l);
        a.max_ctx = max_ctx;
        a.partials = io.partials;
        a.partial_floats = io.partial_floats;
        a.counters = io.counters;
        a.counter_count = io.counter_count;
        a.bytes_hint = (double)io.batch * host_ctx * 2 * kvd * kv_elem_bytes(io.kv->format) + 2.0 * n * qd * 4;
        launch_attention(g, a);
        GemvIn ctx_in;
        ctx_in.mode = IN_F32;
        ctx_in.x = io.ctx;
        ctx_in.x_stride = qd;
        GemvOut add_out;
        add_out.mode = OUT_ADD;
        add_out.y = io.hidden;
        add_out.y_stride = H;
        launch_product(g, L.o, ctx_in, add_out, n);
        GemvIn post_in = norm_in;
        post_in.norm = L.post_norm;
        GemvOut silu_out;
        silu_out.mode = OUT_SILU;
        silu_out.y = io.act;
        silu_out.y_stride = F;
        launch_product(g, L.gate_up, post_in, silu_out, n);
        GemvIn act_in;
        act_in.mode = IN_F32;
        act_in.x = io.act;
        act_in.x_stride = F;
        launch_product(g, L.down, act_in, add_out, n);
    }
    if (!head_out) return;  // a prompt's earlier chunks need no logits
    if (io.rows && io.batch == 1) {
        // every row's logits (forward_rows), then the last row's greedy choice for the decode that may follow
        GemvIn all;
        all.mode = IN_NORM;
        all.x = io.hidden;
        all.x_stride = H;
        all.norm = m->final_norm;
        all.eps = cfg.rms_eps;
        GemvOut rows;
        rows.mode = OUT_F32;
        rows.y = io.rows;
        rows.y_stride = cfg.vocab;
        launch_product(g, m->head(), all, rows, n);
        argmax_row<<<1, 1024, 0, g->stream>>>(io.rows + (n - 1) * cfg.vocab, (int)cfg.vocab, io.best);
        g->launched();
        return;
    }
    GemvIn last;
    last.mode = IN_NORM;
    last.x = io.batch == 1 ? io.hidden + (n - 1) * H : io.hidden;
    last.x_stride = H;
    last.norm = m->final_norm;
    last.eps = cfg.rms_eps;
    GemvOut head;
    head.mode = OUT_F32;
    head.y = io.logits;
    head.y_stride = cfg.vocab;
    head.argmax = io.best;
    if (io.batch == 1) {
        launch_gemv(g, m->head(), last, head, 1);
    } else {
        head.argmax_each = true;
        launch_product(g, m->head(), last, head, io.batch);
    }
}

static void run_prompt(marin_qwen3 *m, marin_qwen3_cache *c, const uint32_t *ids, size_t n, bool all_rows = false) {
    marin_gpu *g = m->gpu;
    const size_t start = c->kv->len;
    if (n == 0) throw Error(MARIN_SHAPE, "no tokens", 1, 0);
    if (start + n > c->kv->capacity) shape("kv positions", c->kv->capacity, start + n);
    for (size_t i = 0; i < n; ++i)
        if (ids[i] >= m->cfg.vocab) shape("token id", m->cfg.vocab, ids[i]);
    c->kv->reserve(start + n);
    for (size_t t0 = 0; t0 < n; t0 += CHUNK) {
        const size_t nt = std::min(CHUNK, n - t0);
        void *staged = g->stage(ids + t0, nt * 4);
        HIP_CHECK(hipMemcpyAsync(c->ids, staged, nt * 4, hipMemcpyHostToDevice, g->stream));
        set_state<<<1, 1, 0, g->stream>>>(c->state, (uint32_t)(start + t0), (uint32_t)nt, c->best);
        g->launched();
        embed_device_ids<<<dim3((unsigned)nt), dim3(256), 0, g->stream>>>(
            m->embed->codes, (const float *)m->embed->scales, c->ids, c->hidden, (int)m->cfg.hidden, (int)m->cfg.group);
        g->launched();
        PassIo io = io_of(c, nt);
        if (all_rows) io.rows = c->rows;
        pass(m, io, start + t0 + nt, 0, t0 + nt == n);
        c->kv->len = start + t0 + nt;
    }
}

extern "C" {

marin_status marin_qwen3_new_empty(marin_gpu *g, const marin_qwen3_config *cfg, marin_qwen3 **out) {
    return guard([&] { *out = alloc_model(g, cfg); });
}

marin_status marin_qwen3_new_synthetic(marin_gpu *g, const marin_qwen3_config *cfg, uint64_t seed, marin_qwen3 **out) {
    return guard([&] {
        marin_qwen3 *m = alloc_model(g, cfg);
        try {
            for (int l = -1; l < (int)cfg->layers; ++l) {
                const int tensors = l < 0 ? (cfg->tie_embeddings ? 1 : 2) : 7;
                for (int t = 0; t < tensors; ++t) {
                    marin_quant_matrix *mat;
                    size_t row0, step, rows, cols;
                    placement(m, l, t, mat, row0, step, rows, cols);
                    launch_synth_quantize(g, mat, seed, synth_stream(l, t), 0.02, rows, row0, step);
                }
            }
            HIP_CHECK(hipStreamSynchronize(g->stream));
        } catch (...) {
            marin_qwen3_free(m);
            throw;
        }
        *out = m;
    });
}

marin_status marin_qwen3_load_matrix(marin_qwen3 *m, int layer, int tensor, size_t rows, size_t cols,
                                     const uint8_t *codes, const float *scales) {
    return guard([&] {
        marin_quant_matrix *mat;
        size_t row0, step, r, c;
        placement(m, layer, tensor, mat, row0, step, r, c);
        if (rows != r || cols != c) shape("tensor rows", r, rows);
        upload_rows(mat, codes, scales, rows, row0, step);
    });
}

marin_status marin_qwen3_load_vector(marin_qwen3 *m, int layer, int which, const float *values, size_t len) {
    return guard([&] {
        float *dst = nullptr;
        size_t want = m->cfg.hidden;
        if (layer < 0) {
            if (which != 0) shape("model vector", 1, (size_t)which);
            dst = m->final_norm;
        } else {
            if ((size_t)layer >= m->layers.size()) shape("layer", m->layers.size(), (size_t)layer);
            Layer &L = m->layers[layer];
            switch (which) {
                case 0: dst = L.input_norm; break;
                case 1: dst = L.post_norm; break;
                case 2: dst = L.q_norm; want = m->cfg.head_dim; break;
                case 3: dst = L.k_norm; want = m->cfg.head_dim; break;
                default: shape("layer vector", 4, (size_t)which);
            }
        }
        check_len("vector length", want, len);
        m->gpu->upload(dst, values, len * 4);
    });
}

void marin_qwen3_free(marin_qwen3 *m) {
    if (!m) return;
    marin_gpu *g = m->gpu;
    (void)hipStreamSynchronize(g->stream);
    for (auto &L : m->layers) {
        free_quant_matrix(L.qkv);
        free_quant_matrix(L.o);
        free_quant_matrix(L.gate_up);
        free_quant_matrix(L.down);
        g->release(L.input_norm);
        g->release(L.post_norm);
        g->release(L.q_norm);
        g->release(L.k_norm);
    }
    free_quant_matrix(m->embed);
    free_quant_matrix(m->lm_head);
    g->release(m->final_norm);
    g->release(m->freq);
    delete m;
}

marin_status marin_qwen3_cache_new(marin_qwen3 *m, size_t capacity, marin_kv_format format, marin_qwen3_cache **out) {
    return guard([&] {
        marin_gpu *g = m->gpu;
        const auto &cfg = m->cfg;
        auto c = std::make_unique<marin_qwen3_cache>();
        c->model = m;
        marin_status s = marin_kv_new(g, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, capacity, format, &c->kv);
        if (s != MARIN_OK) throw Error(s, marin_last_error());
        try {
            const size_t H = cfg.hidden, qd = m->qd(), kvd = m->kvd();
            c->hidden = (float *)g->alloc(CHUNK * H * 4, true);
            c->qkv = (float *)g->alloc(CHUNK * (qd + 2 * kvd) * 4, true);
            c->logits = (float *)g->alloc(cfg.vocab * 4, true);
            c->ctx = (float *)g->alloc(CHUNK * qd * 4, true);
            c->act = (float *)g->alloc(CHUNK * cfg.ffn * 4, true);
            c->best = (unsigned long long *)g->alloc(8, true);
            c->ids = (uint32_t *)g->alloc(CHUNK * 4, true);
            c->state = (uint32_t *)g->alloc(16, true);
            c->tokens_out = (uint32_t *)g->alloc(std::max<size_t>(capacity, 1) * 4, true);
            c->tokens_cap = std::max<size_t>(capacity, 1);
            c->attn_partial_floats = attention_partial_floats(1, CHUNK, cfg.heads, cfg.head_dim, capacity, g->cu_count);
            c->attn_partials = (float *)g->alloc(c->attn_partial_floats * 4, false);
            c->attn_counters = (uint32_t *)g->alloc(attention_counters(1, CHUNK, cfg.heads) * 4, true);
            c->rope = make_rope_table(g, m->freq, cfg.head_dim, capacity);
            c->rows = (float *)g->alloc(MAX_ROWS * cfg.vocab * 4, false);
        } catch (...) {
            marin_qwen3_cache_free(c.release());
            throw;
        }
        *out = c.release();
    });
}

void marin_qwen3_cache_free(marin_qwen3_cache *c) {
    if (!c) return;
    marin_gpu *g = c->model->gpu;
    (void)hipStreamSynchronize(g->stream);
    free_cache_graph(c);
    marin_kv_free(c->kv);
    for (void *p : {(void *)c->hidden, (void *)c->qkv, (void *)c->logits, (void *)c->ctx, (void *)c->act,
                    (void *)c->best, (void *)c->ids, (void *)c->state, (void *)c->attn_partials, (void *)c->attn_counters,
                    (void *)c->tokens_out, (void *)c->rope, (void *)c->rows})
        g->release(p);
    delete c;
}

size_t marin_qwen3_cache_len(const marin_qwen3_cache *c) { return c->kv->len; }

marin_status marin_qwen3_cache_truncate(marin_qwen3_cache *c, size_t len) { return marin_kv_truncate(c->kv, len); }

marin_status marin_qwen3_forward(marin_qwen3 *m, marin_qwen3_cache *c, const uint32_t *ids, size_t n, float *logits) {
    return guard([&] {
        run_prompt(m, c, ids, n);
        m->gpu->download(logits, c->logits, m->cfg.vocab * 4);
    });
}

marin_status marin_qwen3_forward_rows(marin_qwen3 *m, marin_qwen3_cache *c, const uint32_t *ids, size_t n,
                                      float *logits) {
    return guard([&] {
        if (n > MAX_ROWS) unsupported("forward_rows tokens", MAX_ROWS, n);
        run_prompt(m, c, ids, n, true);
        m->gpu->download(logits, c->rows, n * m->cfg.vocab * 4);
    });
}

// One decode step on the device: choose the next token from the last pass's logits, then run it through the model.
static void decode_step(marin_qwen3 *m, marin_qwen3_cache *c, size_t host_ctx) {
    marin_gpu *g = m->gpu;
    advance<<<1, 512, 0, g->stream>>>(c->best, c->ids, c->tokens_out, c->state, m->embed->codes,
                                      (const float *)m->embed->scales, c->hidden, (int)m->cfg.hidden,
                                      (int)m->cfg.group, (uint32_t)m->cfg.vocab);
    g->launched();
    pass(m, io_of(c, 1), c->kv->capacity, host_ctx);
}

static bool graphs_enabled() {
    const char *v = getenv("MARIN_NO_GRAPH");
    return !(v && *v && *v != '0');
}

// Greedy decoding of `steps` tokens from the cache's last logits; each chosen token is fed through the model, so the
// cache then holds the logits after the last one. The per-step launches are captured once into a HIP graph.
static void decode(marin_qwen3 *m, marin_qwen3_cache *c, size_t steps, uint32_t *tokens_out) {
    marin_gpu *g = m->gpu;
    if (steps == 0) return;
    const size_t len = c->kv->len;
    if (len == 0) throw Error(MARIN_SHAPE, "decode needs a forward pass first", 1, 0);
    if (len + steps > c->kv->capacity) shape("kv positions", c->kv->capacity, len + steps);
    c->kv->reserve(len + steps);
    if (steps > c->tokens_cap) {
        HIP_CHECK(hipStreamSynchronize(g->stream));
        free_cache_graph(c);  // the graph holds the old tokens_out address
        g->release(c->tokens_out);
        c->tokens_out = nullptr;
        c->tokens_out = (uint32_t *)g->alloc(steps * 4, false);
        c->tokens_cap = steps;
    }
    // state: pos = len - 1 (advanced to len by the first choice), ctx = len, step 0
    const uint32_t init[3] = {(uint32_t)(len - 1), (uint32_t)len, 0u};
    void *staged = g->stage(init, sizeof(init));
    HIP_CHECK(hipMemcpyAsync(c->state, staged, sizeof(init), hipMemcpyHostToDevice, g->stream));
    if (graphs_enabled()) {
        if (!c->graph) {
            hipGraph_t graph;
            HIP_CHECK(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal));
            try {
                decode_step(m, c, 0);
            } catch (...) {
                hipGraph_t junk;
                (void)hipStreamEndCapture(g->stream, &junk);
                if (junk) (void)hipGraphDestroy(junk);
                throw;
            }
            HIP_CHECK(hipStreamEndCapture(g->stream, &graph));
            hipError_t e = hipGraphInstantiate(&c->graph, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            hip_check(e, "hipGraphInstantiate");
            register_graph(c->graph);
        }
        for (size_t s = 0; s < steps; ++s) {
            HIP_CHECK(hipGraphLaunch(c->graph, g->stream));
            g->traffic.launches++;
        }
    } else {
        for (size_t s = 0; s < steps; ++s) decode_step(m, c, 0);
    }
    c->kv->len = len + steps;
    if (tokens_out) g->download(tokens_out, c->tokens_out, steps * 4);
}

marin_status marin_qwen3_generate(marin_qwen3 *m, marin_qwen3_cache *c, const uint32_t *prompt, size_t n,
                                  size_t steps, uint32_t *tokens_out) {
    return guard([&] {
        if (c->kv->len + n + steps > c->kv->capacity) shape("kv positions", c->kv->capacity, c->kv->len + n + steps);
        run_prompt(m, c, prompt, n);
        decode(m, c, steps, tokens_out);
    });
}

marin_status marin_qwen3_decode(marin_qwen3 *m, marin_qwen3_cache *c, size_t steps, uint32_t *tokens_out) {
    return guard([&] { decode(m, c, steps, tokens_out); });
}

// Runs one decode step with an event after every launch (and before every product and attention launch) and
// returns the launches in order; products and attention are timed by their own start and end events.
static std::vector<marin_launch_record> profile_launches(marin_qwen3 *m, marin_qwen3_cache *c) {
    marin_gpu *g = m->gpu;
    const size_t len = c->kv->len;
    if (len == 0) throw Error(MARIN_SHAPE, "decode needs a forward pass first", 1, 0);
    if (len + 1 > c->kv->capacity) shape("kv positions", c->kv->capacity, len + 1);
    c->kv->reserve(len + 1);
    if (!c->tokens_out) {
        c->tokens_out = (uint32_t *)g->alloc(4, false);
        c->tokens_cap = 1;
    }
    const uint32_t init[3] = {(uint32_t)(len - 1), (uint32_t)len, 0u};
    void *staged = g->stage(init, sizeof(init));
    HIP_CHECK(hipMemcpyAsync(c->state, staged, sizeof(init), hipMemcpyHostToDevice, g->stream));
    std::vector<marin_gpu::ProfileEntry> entries;
    entries.reserve(1024);
    g->events_used = 0;
    hipEvent_t start = g->next_event();
    HIP_CHECK(hipEventRecord(start, g->stream));
    g->profile = &entries;
    try {
        decode_step(m, c, len + 1);
    } catch (...) {
        g->profile = nullptr;
        g->pending_start = g->pending_stop = nullptr;
        throw;
    }
    g->profile = nullptr;
    HIP_CHECK(hipStreamSynchronize(g->stream));
    std::vector<marin_launch_record> out;
    out.reserve(entries.size());
    hipEvent_t prev = start;
    for (const auto &en : entries) {
        float ms = 0.0f;
        HIP_CHECK(hipEventElapsedTime(&ms, en.start ? en.start : prev, en.event));
        marin_launch_record r{};
        r.kind = (uint32_t)en.kind;
        r.bytes = en.bytes;
        r.seconds = ms * 1e-3;
        snprintf(r.name, sizeof(r.name), "%s", en.name ? en.name : "");
        out.push_back(r);
        prev = en.event;
    }
    c->kv->len = len + 1;
    return out;
}

marin_status marin_qwen3_profile_step(marin_qwen3 *m, marin_qwen3_cache *c, marin_step_profile *out) {
    return guard([&] {
        marin_step_profile p{};
        for (const auto &r : profile_launches(m, c)) {
            if (r.kind == marin_gpu::GEMV) {
                p.gemv_seconds += r.seconds;
                p.gemv_bytes += r.bytes;
                p.gemv_launches++;
            } else if (r.kind == marin_gpu::ATTENTION) {
                p.attention_seconds += r.seconds;
                p.attention_bytes += r.bytes;
                p.attention_launches++;
            } else {
                p.other_seconds += r.seconds;
                p.other_launches++;
            }
            p.step_seconds += r.seconds;
        }
        *out = p;
    });
}

marin_status marin_qwen3_time_kernel(marin_qwen3 *m, marin_qwen3_cache *c, const char *name, int reps,
                                     double *seconds_per_launch, uint32_t *launches_per_pass) {
    return guard([&] {
        marin_gpu *g = m->gpu;
        if (!name || !*name) shape("kernel name", 1, 0);
        if (reps < 1) shape("timing repetitions", 1, (size_t)reps);
        if (c->kv->len == 0) throw Error(MARIN_SHAPE, "timing needs a forward pass first", 1, 0);
        const std::string only = name;
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        const uint64_t before = g->traffic.launches;
        HIP_CHECK(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal));
        g->only = only.c_str();
        try {
            pass(m, io_of(c, 1), c->kv->capacity, 0);
        } catch (...) {
            g->only = nullptr;
            g->skipped = false;
            hipGraph_t junk = nullptr;
            (void)hipStreamEndCapture(g->stream, &junk);
            if (junk) (void)hipGraphDestroy(junk);
            throw;
        }
        g->only = nullptr;
        HIP_CHECK(hipStreamEndCapture(g->stream, &graph));
        const uint64_t launches = g->traffic.launches - before;
        if (launches == 0) {
            (void)hipGraphDestroy(graph);
            throw Error(MARIN_SHAPE, "no launch of that kernel in a decode pass", 1, 0);
        }
        hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        hip_check(e, "hipGraphInstantiate");
        hipEvent_t a = g->next_event(), b = g->next_event();
        float ms = 0.0f;
        e = hipGraphLaunch(exec, g->stream);  // warm-up
        if (e == hipSuccess) e = hipEventRecord(a, g->stream);
        for (int r = 0; r < reps && e == hipSuccess; ++r) e = hipGraphLaunch(exec, g->stream);
        if (e == hipSuccess) e = hipEventRecord(b, g->stream);
        if (e == hipSuccess) e = hipEventSynchronize(b);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
        (void)hipGraphExecDestroy(exec);
        hip_check(e, "timed kernel graph");
        *seconds_per_launch = ms * 1e-3 / ((double)reps * (double)launches);
        *launches_per_pass = (uint32_t)launches;
    });
}

marin_status marin_qwen3_profile_launches(marin_qwen3 *m, marin_qwen3_cache *c, marin_launch_record *out,
                                          size_t cap, size_t *count) {
    return guard([&] {
        const auto recs = profile_launches(m, c);
        for (size_t i = 0; i < recs.size() && i < cap; ++i) out[i] = recs[i];
        *count = recs.size();
    });
}

static void free_batch_graph(marin_qwen3_batch *b) {
    if (b->graph) {
        unregister_graph(b->graph);
        (void)hipGraphExecDestroy(b->graph);
        b->graph = nullptr;
    }
}

static PassIo io_of(marin_qwen3_batch *b) {
    return PassIo{b->hidden, b->qkv, b->ctx, b->act, b->logits, b->best, b->tables, b->table_stride,
                  b->state + b->seqs.size(), b->seqs.size(), 1, b->seqs[0]->kv, b->partials, b->partial_floats,
                  b->counters, b->counter_count, b->seqs[0]->rope, nullptr};
}

// One batch decode step: every sequence's choice becomes its token, then one pass of the batch.
static void batch_step(marin_qwen3 *m, marin_qwen3_batch *b) {
    marin_gpu *g = m->gpu;
    advance_batch<<<(unsigned)b->seqs.size(), 512, 0, g->stream>>>(
        b->best, b->tokens_out, b->state, (int)b->seqs.size(), m->embed->codes, (const float *)m->embed->scales,
        b->hidden, (int)m->cfg.hidden, (int)m->cfg.group, (uint32_t)m->cfg.vocab);
    g->launched();
    pass(m, io_of(b), b->capacity, 0);
}


void marin_qwen3_batch_free(marin_qwen3_batch *b) {
    if (!b) return;
    marin_gpu *g = b->model->gpu;
    (void)hipStreamSynchronize(g->stream);
    free_batch_graph(b);
    for (auto *c : b->seqs) marin_qwen3_cache_free(c);
    for (void *p : {(void *)b->hidden, (void *)b->qkv, (void *)b->ctx, (void *)b->act, (void *)b->logits,
                    (void *)b->best, (void *)b->state, (void *)b->tables, (void *)b->tokens_out, (void *)b->partials,
                    (void *)b->counters})
        g->release(p);
    delete b;
}

marin_status marin_qwen3_batch_new(marin_qwen3 *m, size_t batch, size_t capacity, marin_kv_format format,
                                   marin_qwen3_batch **out) {
    return guard([&] {
        if (batch < 1 || batch > MOE_BATCH) unsupported("decode batch (sequences)", MOE_BATCH, batch);
        marin_gpu *g = m->gpu;
        const auto &cfg = m->cfg;
        auto b = std::make_unique<marin_qwen3_batch>();
        b->model = m;
        b->capacity = capacity;
        try {
            for (size_t i = 0; i < batch; ++i) {
                marin_qwen3_cache *c = nullptr;
                marin_status st = marin_qwen3_cache_new(m, capacity, format, &c);
                if (st != MARIN_OK) throw Error(st, marin_last_error());
                b->seqs.push_back(c);
            }
            const size_t H = cfg.hidden, qd = m->qd(), kvd = m->kvd();
            b->hidden = (float *)g->alloc(batch * H * 4, true);
            b->qkv = (float *)g->alloc(batch * (qd + 2 * kvd) * 4, true);
            b->ctx = (float *)g->alloc(batch * qd * 4, true);
            b->act = (float *)g->alloc(batch * cfg.ffn * 4, true);
            b->logits = (float *)g->alloc(batch * cfg.vocab * 4, true);
            b->best = (unsigned long long *)g->alloc(batch * 8, true);
            b->state = (uint32_t *)g->alloc(3 * batch * 4, true);
            b->table_stride = b->seqs[0]->kv->pool.limit;
            b->tables = (uint64_t *)g->alloc(std::max<size_t>(batch * b->table_stride, 1) * 8, true);
            b->host_tables.assign(batch * b->table_stride, 0);
            b->partial_floats = attention_partial_floats(batch, 1, cfg.heads, cfg.head_dim, capacity, g->cu_count);
            b->partials = (float *)g->alloc(b->partial_floats * 4, false);
            b->counter_count = attention_counters(batch, 1, cfg.heads);
            b->counters = (uint32_t *)g->alloc(b->counter_count * 4, true);
        } catch (...) {
            marin_qwen3_batch_free(b.release());
            throw;
        }
        *out = b.release();
    });
}

size_t marin_qwen3_batch_len(const marin_qwen3_batch *b, size_t seq) {
    return seq < b->seqs.size() ? b->seqs[seq]->kv->len : 0;
}

marin_status marin_qwen3_batch_prefill(marin_qwen3_batch *b, size_t seq, const uint32_t *ids, size_t n) {
    return guard([&] {
        if (seq >= b->seqs.size()) shape("batch sequence", b->seqs.size(), seq);
        marin_qwen3_cache *c = b->seqs[seq];
        run_prompt(b->model, c, ids, n);
        // the prompt's greedy choice is the sequence's first decoded token
        HIP_CHECK(hipMemcpyAsync(b->best + seq, c->best, 8, hipMemcpyDeviceToDevice, b->model->gpu->stream));
    });
}

// Greedy decoding of `steps` tokens for every sequence; tokens_out is [batch][steps].
marin_status marin_qwen3_batch_decode(marin_qwen3_batch *b, size_t steps, uint32_t *tokens_out) {
    return guard([&] {
        marin_qwen3 *m = b->model;
        marin_gpu *g = m->gpu;
        const size_t B = b->seqs.size();
        if (steps == 0) return;
        std::vector<uint32_t> init(3 * B, 0u);
        for (size_t i = 0; i < B; ++i) {
            marin_kv *kv = b->seqs[i]->kv;
            if (kv->len == 0) throw Error(MARIN_SHAPE, "every sequence of a batch needs its prompt first", 1, 0);
            if (kv->len + steps > kv->capacity) shape("kv positions", kv->capacity, kv->len + steps);
            kv->reserve(kv->len + steps);
            std::copy(kv->host_ptrs.begin(), kv->host_ptrs.begin() + std::min(kv->host_ptrs.size(), b->table_stride),
                      b->host_tables.begin() + i * b->table_stride);
            init[i] = (uint32_t)(kv->len - 1);  // advanced to len by the first choice
            init[B + i] = (uint32_t)kv->len;
        }
        g->upload(b->tables, b->host_tables.data(), b->host_tables.size() * 8);
        g->upload(b->state, init.data(), init.size() * 4);
        if (steps > b->tokens_cap) {
            HIP_CHECK(hipStreamSynchronize(g->stream));
            free_batch_graph(b);  // the graph holds the old tokens_out address
            g->release(b->tokens_out);
            b->tokens_out = nullptr;
            b->tokens_out = (uint32_t *)g->alloc(steps * B * 4, false);
            b->tokens_cap = steps;
        }
        // the products' activation limbs: grown before a capture (a capture may not allocate)
        const auto &cfg = m->cfg;
        g->workspace(moe_gate_up_workspace((B + 3) / 4 * 4, std::max(std::max(cfg.hidden, cfg.ffn), m->qd()), cfg.group));
        if (graphs_enabled()) {
            if (!b->graph) {
                hipGraph_t graph;
                HIP_CHECK(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal));
                try {
                    batch_step(m, b);
                } catch (...) {
                    hipGraph_t junk;
                    (void)hipStreamEndCapture(g->stream, &junk);
                    if (junk) (void)hipGraphDestroy(junk);
                    throw;
                }
                HIP_CHECK(hipStreamEndCapture(g->stream, &graph));
                hipError_t e = hipGraphInstantiate(&b->graph, graph, nullptr, nullptr, 0);
                (void)hipGraphDestroy(graph);
                hip_check(e, "hipGraphInstantiate");
                register_graph(b->graph);
            }
            for (size_t s = 0; s < steps; ++s) {
                HIP_CHECK(hipGraphLaunch(b->graph, g->stream));
                g->traffic.launches++;
            }
        } else {
            for (size_t s = 0; s < steps; ++s) batch_step(m, b);
        }
        for (auto *c : b->seqs) c->kv->len += steps;
        if (tokens_out) {
            std::vector<uint32_t> t(steps * B);
            g->download(t.data(), b->tokens_out, t.size() * 4);
            for (size_t s = 0; s < steps; ++s)
                for (size_t i = 0; i < B; ++i) tokens_out[i * steps + s] = t[s * B + i];
        }
    });
}

}  // extern "C"
