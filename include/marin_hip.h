/*
 * marin_hip: the MI355X (gfx950) backend of Marin's quantized decode path, behind a C ABI.
 *
 * Every entry point mirrors a public item of the reference's `cuda` crate, the backend that crates/model and
 * crates/runtime call (cited per declaration as crates/cuda/src/<file>:<line>). A Rust crate `hip` that wraps these
 * functions with the same method names can stand in for `cuda`, published under that name to crates/model.
 *
 * Conventions (crates/cuda/src/error.rs:6-36, gpu.rs:68-76):
 *  - Every fallible call returns a marin_status. On failure the calling thread's last error (marin_last_error*) holds
 *    the message and the fields of the matching CudaError variant. Sizes are checked before any launch: a call that
 *    fails its checks launches nothing and changes nothing.
 *  - Handles are opaque and owned by the caller; each *_new has a matching *_free. Device memory lives until freed.
 *  - All work is issued in order on the context's one stream; only downloads, marin_gpu_synchronize and
 *    marin_mark_since block.
 *  - Buffers hold f32 unless created with a dtype (extensions for the benchmark layouts).
 */
#ifndef MARIN_HIP_H
#define MARIN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- errors: crates/cuda/src/error.rs:6-49 (enum CudaError, is_out_of_memory) ---- */
typedef enum marin_status {
    MARIN_OK = 0,
    MARIN_UNAVAILABLE = 1, /* CudaError::Unavailable: no gfx950 device / runtime */
    MARIN_DRIVER = 2,      /* CudaError::Driver: a HIP runtime call failed */
    MARIN_SHAPE = 3,       /* CudaError::Shape { what, expected, actual } */
    MARIN_KV_MEMORY = 4,   /* CudaError::KvMemory { held, needed, positions } */
    MARIN_OVERFLOW = 5,    /* CudaError::Overflow { what } */
    MARIN_SELF_CHECK = 6,  /* CudaError::SelfCheck { what } */
    MARIN_UNSUPPORTED = 7  /* CudaError::Unsupported { what, max, actual } */
} marin_status;

/* Message of the calling thread's last failure ("" after success is not guaranteed; check the status). */
const char *marin_last_error(void);
/* The numeric fields of the last failure: Shape (expected, actual), Unsupported (max, actual), KvMemory (held,
 * needed, positions in extra). Unused fields are 0. */
void marin_last_error_fields(size_t *expected, size_t *actual, size_t *extra);
/* CudaError::is_out_of_memory (error.rs:40-49): the last failure was a device allocation that ran out of memory. */
int marin_last_error_is_oom(void);

/* ---- device context: crates/cuda/src/gpu.rs:68-76 (struct Gpu), gpu.rs:149-244 ---- */
typedef struct marin_gpu marin_gpu;
typedef struct marin_gpu_info {
    char name[256];
    char arch[64];
    int compute_units;
    size_t free_bytes, total_bytes;
} marin_gpu_info;

marin_status marin_gpu_new(marin_gpu **out);                          /* Gpu::new, gpu.rs:149 (device 0) */
void marin_gpu_free(marin_gpu *gpu);                                  /* Drop for Gpu */
marin_status marin_gpu_info_get(marin_gpu *gpu, marin_gpu_info *out); /* Gpu::info, gpu.rs:228 */
marin_status marin_gpu_synchronize(marin_gpu *gpu);                   /* Gpu::synchronize, gpu.rs:244 */
/* The context's stream (hipStream_t), for interop only. */
void *marin_gpu_stream(marin_gpu *gpu);
/* Gpu::bind_to_thread (gpu.rs:238-242): makes the context's device current on the calling thread. */
marin_status marin_gpu_bind_to_thread(marin_gpu *gpu);
/* Gpu::set_fast_attention (attention.rs:81-86): whether prompt passes over an f16 cache with head size 64 or 128 use
 * the matrix-core attention (the default); off, they take the vector-ALU kernel, as other caches always do. */
void marin_set_fast_attention(marin_gpu *gpu, int on);

/* Traffic counters: crates/cuda/src/counters.rs:10-89 (struct Traffic, Gpu::traffic :102). */
typedef struct marin_traffic {
    uint64_t launches, allocations, uploads, upload_bytes, downloads, download_bytes;
} marin_traffic;
marin_status marin_gpu_traffic(marin_gpu *gpu, marin_traffic *out);

/* Events: counters.rs:91-111 (Mark, Gpu::mark, Mark::since). */
typedef struct marin_mark marin_mark;
marin_status marin_mark_new(marin_gpu *gpu, marin_mark **out); /* records an event on the stream now */
marin_status marin_mark_since(marin_mark *later, marin_mark *earlier, double *seconds); /* waits for `later` */
void marin_mark_free(marin_mark *mark);

/* ---- buffers: gpu.rs:87-123 (Buffer, Tokens), gpu.rs:270-392 ---- */
typedef enum marin_dtype { MARIN_F32 = 0, MARIN_BF16 = 1, MARIN_F16 = 2, MARIN_U8 = 3, MARIN_U32 = 4 } marin_dtype;
typedef struct marin_buffer marin_buffer;

marin_status marin_buffer_zeros(marin_gpu *gpu, size_t len, marin_buffer **out);                 /* Gpu::zeros :295 */
marin_status marin_buffer_upload(marin_gpu *gpu, const float *values, size_t len, marin_buffer **out); /* :270 */
marin_status marin_buffer_upload_into(marin_gpu *gpu, const float *values, size_t len, marin_buffer *dst); /* :281 */
marin_status marin_buffer_download(marin_gpu *gpu, const marin_buffer *buf, float *dst, size_t len); /* :303 */
marin_status marin_buffer_download_range(marin_gpu *gpu, const marin_buffer *buf, size_t start, size_t len,
                                         float *dst);                                            /* :326 */
marin_status marin_buffer_copy_range_into(marin_gpu *gpu, const marin_buffer *src, size_t start,
                                          marin_buffer *dst);                                    /* :346 */
marin_status marin_buffer_copy_into_range(marin_gpu *gpu, const marin_buffer *src, marin_buffer *dst,
                                          size_t start);                                         /* :366 */
size_t marin_buffer_len(const marin_buffer *buf);
void marin_buffer_free(marin_buffer *buf);
/* Extension (no reference counterpart): typed buffers for the benchmark layouts (bf16 activations, bf16 outputs). */
marin_status marin_buffer_new_typed(marin_gpu *gpu, marin_dtype dtype, size_t len, const void *host,
                                    marin_buffer **out);
marin_status marin_buffer_download_raw(marin_gpu *gpu, const marin_buffer *buf, void *dst, size_t bytes);
marin_dtype marin_buffer_dtype(const marin_buffer *buf);
void *marin_buffer_device_ptr(const marin_buffer *buf);

typedef struct marin_tokens marin_tokens;
marin_status marin_tokens_new(marin_gpu *gpu, size_t capacity, marin_tokens **out); /* Gpu::tokens, gpu.rs:386 */
void marin_tokens_free(marin_tokens *tokens);

/* ---- quantized matrices: crates/cuda/src/quant.rs:16-293 ---- */
typedef struct marin_quant_matrix marin_quant_matrix; /* DeviceQuantMatrix, quant.rs:16 */

/* Gpu::upload_quantized (quant.rs:56-97): `codes` as tensor::Quantized holds them (int8 row-major; int4 two per
 * byte, even column low, +8), `scales[row * cols/group + g]` f32. Checks group % 32 == 0, cols % group == 0 and
 * both lengths (CudaError::Shape) before touching the device. bits is 8 or 4. */
marin_status marin_upload_quantized(marin_gpu *gpu, size_t rows, size_t cols, int bits, size_t group,
                                    const uint8_t *codes, size_t codes_len, const float *scales, size_t scales_len,
                                    marin_quant_matrix **out);
/* Extension: bf16 scales (the benchmark layout of the isolated-linear config). Same checks. */
marin_status marin_upload_quantized_bf16_scales(marin_gpu *gpu, size_t rows, size_t cols, int bits, size_t group,
                                                const uint8_t *codes, size_t codes_len, const uint16_t *scales,
                                                size_t scales_len, marin_quant_matrix **out);
void marin_quant_matrix_free(marin_quant_matrix *m);
void marin_quant_matrix_shape(const marin_quant_matrix *m, size_t *rows, size_t *cols, int *bits, size_t *group);
/* Bytes of codes plus scales held on the device (QuantScheme::matrix_bytes, tensor/src/quant.rs:86-92). */
size_t marin_quant_matrix_bytes(const marin_quant_matrix *m);

/* Gpu::embed_quant (quant.rs:100-129): out[t] = row ids[t] of an int8 table, dequantized. Refuses int4 tables
 * (Unsupported), ids >= rows (Shape), more ids than `scratch` holds (Shape), out.len != n * cols (Shape). */
marin_status marin_embed_quant(marin_gpu *gpu, const marin_quant_matrix *table, const uint32_t *ids, size_t n,
                               marin_tokens *scratch, marin_buffer *out);

/* Gpu::matmul_quant (quant.rs:131-139): out[t][r] = dot(dequantized w[r], x[t]) for `tokens` rows of x; f32
 * activations, f32 accumulation. Checks x.len == tokens*cols and out.len == tokens*rows (Shape). */
marin_status marin_matmul_quant(marin_gpu *gpu, const marin_quant_matrix *w, const marin_buffer *x, size_t tokens,
                                marin_buffer *out);
/* Gpu::matmul_quant_precise (quant.rs:141-154): same product, with the f32-grade path at every token count. */
marin_status marin_matmul_quant_precise(marin_gpu *gpu, const marin_quant_matrix *w, const marin_buffer *x,
                                        size_t tokens, marin_buffer *out);
/* Extension (no reference counterpart): the isolated-linear benchmark layout, x bf16 [tokens][cols] and out bf16
 * [tokens][rows], f32 accumulation. */
marin_status marin_matmul_quant_bf16(marin_gpu *gpu, const marin_quant_matrix *w, const marin_buffer *x,
                                     size_t tokens, marin_buffer *out);

/* ---- dense bf16 matrices: crates/cuda/src/gpu.rs:87-93 (DeviceMatrix), gpu.rs:248-268, matmul.rs:16-205 ---- */
typedef struct marin_matrix marin_matrix; /* DeviceMatrix: bf16 bits, row-major [rows][cols] */

/* Gpu::upload_matrix (gpu.rs:248-268): checks len == rows * cols (Shape) and the product (Overflow). */
marin_status marin_upload_matrix(marin_gpu *gpu, size_t rows, size_t cols, const uint16_t *bits, size_t len,
                                 marin_matrix **out);
void marin_matrix_free(marin_matrix *m);
void marin_matrix_shape(const marin_matrix *m, size_t *rows, size_t *cols);
/* Gpu::embed (ops.rs:55-73): out[t] = row ids[t] of a bf16 table as f32. Ids >= rows, more ids than `scratch`
 * holds, or out.len != n * cols are refused (Shape) before anything is copied. */
marin_status marin_embed(marin_gpu *gpu, const marin_matrix *table, const uint32_t *ids, size_t n,
                         marin_tokens *scratch, marin_buffer *out);
/* Gpu::matmul (matmul.rs:16-24): out[t][r] = dot(w[r], x[t]); f32 activations, f32 accumulation; from 16 tokens with
 * cols a multiple of 16 on the matrix cores with the activations split into three bf16 parts, so every product is
 * exact (matmul.rs:51 chooses the kernel the same way). */
marin_status marin_matmul(marin_gpu *gpu, const marin_matrix *w, const marin_buffer *x, size_t tokens,
                          marin_buffer *out);
/* Gpu::matmul_precise (matmul.rs:26-35): the same product on the vector ALUs in f32 at every token count. */
marin_status marin_matmul_precise(marin_gpu *gpu, const marin_matrix *w, const marin_buffer *x, size_t tokens,
                                  marin_buffer *out);
/* Gpu::matmul_pair / matmul_triple (matmul.rs:101-166): matrices sharing x, each with its own output; the same bits
 * as separate matmuls. Mismatched columns or buffer sizes are refused (Shape) before any launch. */
marin_status marin_matmul_pair(marin_gpu *gpu, const marin_matrix *w0, const marin_matrix *w1, const marin_buffer *x,
                               size_t tokens, marin_buffer *y0, marin_buffer *y1);
marin_status marin_matmul_triple(marin_gpu *gpu, const marin_matrix *w0, const marin_matrix *w1,
                                 const marin_matrix *w2, const marin_buffer *x, size_t tokens, marin_buffer *y0,
                                 marin_buffer *y1, marin_buffer *y2);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc): marin_matmul_quant_bf16 with the multi-token products' scratch
 * (activation limbs, exponents, per-token factors) in a fixed 4 MiB device array of the library, one per device for
 * the life of the process, instead of memory the library allocates. Calls no allocating routine. Refuses (Unsupported)
 * a product whose scratch would exceed 4 MiB (about 64 tokens of 12288 columns). Every call on a device shares the
 * array: calls that overlap on one device (contexts whose streams run at once) race. */
marin_status marin_matmul_quant_bf16_noalloc(marin_gpu *gpu, const marin_quant_matrix *w, const marin_buffer *x,
                                             size_t tokens, marin_buffer *out);

/* ---- elementwise ops: crates/cuda/src/ops.rs:110-236 ---- */
marin_status marin_rms_norm(marin_gpu *gpu, marin_buffer *x, const marin_buffer *weight, float eps); /* ops.rs:110 */
marin_status marin_rms_norm_into(marin_gpu *gpu, const marin_buffer *x, const marin_buffer *weight,
                                 marin_buffer *out, float eps);                                     /* ops.rs:128 */
marin_status marin_rope(marin_gpu *gpu, marin_buffer *x, size_t heads, size_t head_dim, size_t start,
                        float theta);                                                               /* ops.rs:157 */
marin_status marin_silu_mul(marin_gpu *gpu, marin_buffer *gate, const marin_buffer *up);           /* ops.rs:207 */
marin_status marin_add(marin_gpu *gpu, marin_buffer *a, const marin_buffer *b);                    /* ops.rs:212 */

/* ---- paged KV cache: crates/cuda/src/kv.rs:11-346, pages.rs:1-110, kv_format.rs:1-46 ---- */
typedef enum marin_kv_format { MARIN_KV_F32 = 0, MARIN_KV_F16 = 1, MARIN_KV_BF16 = 2 } marin_kv_format;
#define MARIN_PAGE_TOKENS 64 /* pages.rs:4 PAGE_TOKENS */
#define MARIN_SLAB_PAGES 8   /* pages.rs:7 SLAB_PAGES */
typedef struct marin_kv marin_kv;

/* DeviceKv::new (kv.rs:43-70). heads / kv_heads must divide; head_dim <= 256. Allocates the page table and the
 * split-attention scratch for `capacity` positions now, slabs of pages on first use. */
marin_status marin_kv_new(marin_gpu *gpu, size_t layers, size_t heads, size_t kv_heads, size_t head_dim,
                          size_t capacity, marin_kv_format format, marin_kv **out);
void marin_kv_free(marin_kv *kv);
/* DeviceKv::write (kv.rs:273-332): stores keys/values (f32 [tokens][kv_heads*head_dim]) of `layer` for the
 * positions from len on, mapping pages as needed. A failed page reservation leaves the table unchanged. */
marin_status marin_kv_write(marin_gpu *gpu, marin_kv *kv, size_t layer, const marin_buffer *keys,
                            const marin_buffer *values);
marin_status marin_kv_advance(marin_kv *kv, size_t tokens);  /* kv.rs:186 */
marin_status marin_kv_truncate(marin_kv *kv, size_t len);    /* kv.rs:176 */
void marin_kv_clear(marin_kv *kv);                            /* kv.rs:170 */
size_t marin_kv_len(const marin_kv *kv);                      /* kv.rs:85 */
int marin_kv_is_empty(const marin_kv *kv);                    /* kv.rs:89 */
marin_kv_format marin_kv_format_of(const marin_kv *kv);       /* DeviceKv::format, kv.rs:81 */
/* DeviceKv::auxiliary_bytes (kv.rs:144-150): the split-attention scratch and the device page table. */
size_t marin_kv_auxiliary_bytes(const marin_kv *kv);
size_t marin_kv_capacity(const marin_kv *kv);                 /* kv.rs:93 */
size_t marin_kv_pages_held(const marin_kv *kv);               /* kv.rs:98 */
size_t marin_kv_pages_in_use(const marin_kv *kv);             /* kv.rs:111 */
size_t marin_kv_bytes_held(const marin_kv *kv);               /* kv.rs:135 */
size_t marin_kv_page_bytes(const marin_kv *kv);               /* kv.rs:120 */
size_t marin_kv_slab_bytes(const marin_kv *kv);               /* kv.rs:128 */
/* DeviceKv::page_ids (kv.rs:115): copies up to `cap` ids, returns how many the table holds. */
size_t marin_kv_page_ids(const marin_kv *kv, size_t *out, size_t cap);
/* DeviceKv::startup_bytes (kv.rs:151-166); 0 on overflow. */
size_t marin_kv_startup_bytes(size_t layers, size_t heads, size_t kv_heads, size_t head_dim, size_t capacity,
                              marin_kv_format format);

/* Gpu::attention (attention.rs:90-221): causal grouped-query attention of the `tokens` new tokens (q f32
 * [tokens][heads][head_dim]) against `layer`'s cached keys and values, which must already include them. */
marin_status marin_attention(marin_gpu *gpu, const marin_buffer *q, marin_kv *kv, size_t layer, size_t heads,
                             size_t tokens, marin_buffer *out);

/* ---- extension: a page pool shared by a batch of sequences (the paged-attention benchmark layout) ----
 * No reference counterpart: Marin runs one sequence per DeviceKv. Pages hold `page_tokens` positions of
 * [kv_heads][page_tokens][head_dim] keys, then the same for values, in `format`. */
typedef struct marin_page_pool marin_page_pool;
marin_status marin_page_pool_new(marin_gpu *gpu, size_t pages, size_t page_tokens, size_t kv_heads,
                                 size_t head_dim, marin_kv_format format, marin_page_pool **out);
void marin_page_pool_free(marin_page_pool *pool);
/* Writes one page's keys and values from host data already in the pool's format (2 * kv_heads * page_tokens *
 * head_dim elements: keys then values). */
marin_status marin_page_pool_write(marin_gpu *gpu, marin_page_pool *pool, size_t page, const void *data,
                                   size_t bytes);
/* Decode attention for `batch` sequences, one new token each, q bf16 [batch][heads][head_dim] -> out bf16.
 * tables[b * table_stride + i] is the page holding positions [i*page_tokens, (i+1)*page_tokens) of sequence b;
 * ctx_lens[b] positions are visible (the last is the query's own). Host arrays; checked before launching. */
marin_status marin_paged_attention_batch(marin_gpu *gpu, const marin_buffer *q, marin_page_pool *pool,
                                         const uint32_t *tables, size_t table_stride, const uint32_t *ctx_lens,
                                         size_t batch, size_t heads, marin_buffer *out);

/* ---- extension: the Qwen3 decode driver over this backend (model/src/qwen3/gpu.rs:222-395 Qwen3Gpu::pass) ---- */
typedef struct marin_qwen3 marin_qwen3;
typedef struct marin_qwen3_config {
    size_t layers, hidden, heads, kv_heads, head_dim, ffn, vocab;
    float rms_eps, rope_theta;
    int tie_embeddings;
    size_t group; /* int8 group size (multiple of 64 for the fused path) */
} marin_qwen3_config;

/* Random-init model of the given shape built on the device (weights N(0, 0.02) from the generator that
 * oracle/marin_oracle.c restates, quantized int8 with the reference's rule; norms 1.0). */
marin_status marin_qwen3_new_synthetic(marin_gpu *gpu, const marin_qwen3_config *cfg, uint64_t seed,
                                       marin_qwen3 **out);
/* Empty model; fill each tensor with marin_qwen3_load_* (tensor: 0 q, 1 k, 2 v, 3 o, 4 gate, 5 up, 6 down for
 * layer >= 0; layer -1: 0 embed, 1 lm_head). Vectors: 0 input_norm, 1 post_norm, 2 q_norm, 3 k_norm; layer -1: 0
 * final norm. */
marin_status marin_qwen3_new_empty(marin_gpu *gpu, const marin_qwen3_config *cfg, marin_qwen3 **out);
marin_status marin_qwen3_load_matrix(marin_qwen3 *m, int layer, int tensor, size_t rows, size_t cols,
                                     const uint8_t *codes, const float *scales);
marin_status marin_qwen3_load_vector(marin_qwen3 *m, int layer, int which, const float *values, size_t len);
void marin_qwen3_free(marin_qwen3 *m);
/* Sequence state (GpuCache, model/src/qwen3/gpu.rs:56-100): paged KV cache plus the decode workspace. */
typedef struct marin_qwen3_cache marin_qwen3_cache;
marin_status marin_qwen3_cache_new(marin_qwen3 *m, size_t capacity, marin_kv_format format,
                                   marin_qwen3_cache **out);
void marin_qwen3_cache_free(marin_qwen3_cache *c);
size_t marin_qwen3_cache_len(const marin_qwen3_cache *c);
marin_status marin_qwen3_cache_truncate(marin_qwen3_cache *c, size_t len);
/* CausalLm::forward (runtime/src/lib.rs:67-100): one pass over `n` tokens; the last token's logits into `logits`
 * (vocab floats, host memory). */
marin_status marin_qwen3_forward(marin_qwen3 *m, marin_qwen3_cache *c, const uint32_t *ids, size_t n,
                                 float *logits);
/* CausalLm::forward_rows (runtime/src/lib.rs:86-99; Qwen3Gpu::forward_rows, model/src/qwen3/gpu.rs:212-236): one pass
 * over n <= 8 tokens (more: Unsupported, nothing run) that commits them and writes the logits after every token,
 * [n][vocab] floats in host memory; a decode that follows continues from the last row's greedy choice. */
marin_status marin_qwen3_forward_rows(marin_qwen3 *m, marin_qwen3_cache *c, const uint32_t *ids, size_t n,
                                      float *logits);
/* runtime::generate_reusing greedy (generate.rs:105-284, sampler lowest-index argmax): the prompt, then `steps`
 * greedy tokens chosen on the device; no host round trip per token. */
marin_status marin_qwen3_generate(marin_qwen3 *m, marin_qwen3_cache *c, const uint32_t *prompt, size_t n,
                                  size_t steps, uint32_t *tokens_out);

/* Extension (config 3 at batch 8; the reference decodes one sequence at a time): a decode batch of `batch` (1..8)
 * sequences, each with its own KV cache of `capacity` positions. Prompts go in one sequence at a time; decoding then
 * advances every sequence by one greedy token per step with each product over the whole batch (its weights read
 * once per step) and one attention launch over all sequences. */
typedef struct marin_qwen3_batch marin_qwen3_batch;
marin_status marin_qwen3_batch_new(marin_qwen3 *m, size_t batch, size_t capacity, marin_kv_format format,
                                   marin_qwen3_batch **out);
void marin_qwen3_batch_free(marin_qwen3_batch *b);
size_t marin_qwen3_batch_len(const marin_qwen3_batch *b, size_t seq);
/* The prompt of sequence `seq` (a forward pass through its cache); its greedy choice is the sequence's next token. */
marin_status marin_qwen3_batch_prefill(marin_qwen3_batch *b, size_t seq, const uint32_t *ids, size_t n);
/* `steps` greedy tokens for every sequence (each must have had its prompt); tokens_out is [batch][steps]. */
marin_status marin_qwen3_batch_decode(marin_qwen3_batch *b, size_t steps, uint32_t *tokens_out);

/* Extension: continues greedy decoding for `steps` more tokens after a forward/generate on this cache (the
 * choice from the last pass's logits is the first token written). */
marin_status marin_qwen3_decode(marin_qwen3 *m, marin_qwen3_cache *c, size_t steps, uint32_t *tokens_out);
/* Extension (measurement): one decode step like marin_qwen3_decode(steps = 1), with an event between every launch.
 * Reports the summed durations and algorithmic bytes of the quantized products (weights + scales + activations +
 * outputs) and of attention (keys + values read, queries, outputs), and the whole step. */
typedef struct marin_step_profile {
    double gemv_seconds, gemv_bytes;
    double attention_seconds, attention_bytes;
    double other_seconds, step_seconds;
    uint32_t gemv_launches, attention_launches, other_launches;
} marin_step_profile;
marin_status marin_qwen3_profile_step(marin_qwen3 *m, marin_qwen3_cache *c, marin_step_profile *out);
/* Extension (measurement, the role of GpuProbe + Gpu::mark, model/src/qwen3/gpu_probe.rs, cuda/src/counters.rs:91-111):
 * one decode step with events around every launch; the launches in order, `count` of them (at most `cap` written).
 * kind: 0 other, 1 quantized product, 2 attention; seconds between the launch's own events (products and
 * attention) or from the previous launch's event; name: the kernel instantiation as profilers print it. */
typedef struct marin_launch_record {
    uint32_t kind;
    double bytes, seconds;
    char name[96];
} marin_launch_record;
marin_status marin_qwen3_profile_launches(marin_qwen3 *m, marin_qwen3_cache *c, marin_launch_record *out,
                                          size_t cap, size_t *count);
/* Extension (measurement): one decode pass captured into a HIP graph with only the launches of kernel `name` (as
 * marin_launch_record names it), replayed `reps` times between two events on the stream: mean seconds per launch
 * (kernel time plus the graph's gap to the next launch) and launches per pass. The pass's matrices, inputs and
 * outputs are the decode step's; it leaves the cache's activations (not its keys and values) unspecified. */
marin_status marin_qwen3_time_kernel(marin_qwen3 *m, marin_qwen3_cache *c, const char *name, int reps,
                                     double *seconds_per_launch, uint32_t *launches_per_pass);

/* ---- Mixture of experts (config 4, Qwen3-30B-A3B shape; no reference counterpart for Qwen3-MoE: the analogue is
 * Granite's route/experts/mix, crates/cuda/src/granite.cu:12-118 and granite.rs:1-194) ----
 * Routing: per token, probabilities = softmax over the `experts` logits; the k largest (lowest expert id on ties) in
 * descending order into `ids` (u32 buffer [tokens][k]) and their probabilities into `weights` ([tokens][k]),
 * renormalized to sum to 1 when `renorm` (norm_topk_prob). */
marin_status marin_moe_route(marin_gpu *gpu, const marin_buffer *logits, size_t tokens, size_t experts, size_t k,
                             int renorm, marin_buffer *ids, marin_buffer *weights);
/* Expert FFN: gate_up is the experts' stacked [experts * 2F][H] int8 matrix (expert e's rows at e * 2F, gate and up
 * interleaved row by row), down the stacked [experts * H][F] one. For every token t:
 * out[t] += sum_j weights[t][j] * down_e(silu(gate_e x) * up_e x), e = ids[t][j], x = RMSNorm(x[t]) * norm when
 * `norm` is given (eps), else x[t]. `act` is scratch of tokens * k * F floats. k <= 8, F a multiple of 64 up to
 * 1024, groups 64 or 128. */
marin_status marin_moe_ffn(marin_gpu *gpu, const marin_quant_matrix *gate_up, const marin_quant_matrix *down,
                           const marin_buffer *x, const marin_buffer *norm, float eps, const marin_buffer *ids,
                           const marin_buffer *weights, size_t tokens, size_t experts, size_t k, marin_buffer *act,
                           marin_buffer *out);
/* Measurement: the expert FFNs of `layers` layers (gate_ups[l], downs[l]; ids and weights [layers][tokens][k])
 * captured into one HIP graph and replayed `reps` times between two events: mean seconds per replay. `part` 0 times
 * the whole FFN, 1 only the gate_up products, 2 only the down products (whose inputs are then last call's `act`). */
marin_status marin_moe_stack_time(marin_gpu *gpu, size_t layers, const marin_quant_matrix *const *gate_ups,
                                  const marin_quant_matrix *const *downs, const marin_buffer *x,
                                  const marin_buffer *norm, float eps, const marin_buffer *ids,
                                  const marin_buffer *weights, size_t tokens, size_t experts, size_t k,
                                  marin_buffer *act, marin_buffer *out, int part, int reps, double *seconds);

/* Extension (measurement, config 1): `reps` bf16-in/bf16-out products (marin_matmul_quant_bf16) cycling through `n`
 * same-shaped matrices, captured into one HIP graph and replayed between two events: mean seconds per product. */
marin_status marin_time_matmul_bf16(marin_gpu *gpu, const marin_quant_matrix *const *mats, size_t n,
                                    const marin_buffer *x, size_t tokens, marin_buffer *out, int reps,
                                    double *seconds);

/* Extension (bandwidth probe, the role of cuda/src/probe.rs:145-314): `reps` device-to-device copies of `bytes`
 * (a multiple of 16) through a plain streaming kernel; the mean seconds per copy. */
marin_status marin_probe_copy(marin_gpu *gpu, size_t bytes, int reps, double *seconds);

/* Extension: a rows x cols int8 matrix from the synthetic generator (seed, stream), N(0, std), quantized on the
 * device with the reference's rule (tensor/src/quant.rs:181-234); the oracle restates both bit for bit. */
marin_status marin_quantized_synthetic(marin_gpu *gpu, size_t rows, size_t cols, size_t group, uint64_t seed,
                                       uint64_t stream, double std_dev, marin_quant_matrix **out);

#ifdef __cplusplus
}
#endif
#endif
