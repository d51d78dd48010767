/*
 * CPU oracle for the quantized decode path: a plain-C restatement of Marin's CPU arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or, for the baseline, as the thing timed on the host). The HIP product path
 * never calls it.
 *
 * Pinning status of each function is recorded next to its declaration. "pinned" means a test checks it against the
 * reference's own known answers or golden fixtures, or against a closed form / brute force chosen so a plausible
 * mistake fails.
 */
#ifndef MARIN_ORACLE_H
#define MARIN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Threads for the row-parallel helpers (results do not depend on the count). Default 1, as Marin's one-token path. */
void or_set_threads(int n);

/* bf16 <-> f32 (tensor/src/matrix.rs:31 bf16_to_f32; f32 -> bf16 round-to-nearest-even). pinned: exhaustive. */
float or_bf16_to_f32(uint16_t bits);
uint16_t or_f32_to_bf16(float value);
/* f32 -> f16 bits, round to nearest even, saturating at 65504 like cuda/tests/kv_round/mod.rs:3-18. */
uint16_t or_f32_to_f16_sat(float value);
float or_f16_to_f32(uint16_t bits);

/* tensor::quantize / quantize_rows (tensor/src/quant.rs:120-234). bits is 8 or 4. Returns -1 on success, or the first
 * row holding a NaN/Inf (the reference reports that row), or -2 for a bad shape/group. pinned: known answers of
 * tensor/tests/quant.rs:69-123 + exhaustive bf16 sweep. */
long or_quantize(const uint16_t *weights, size_t rows, size_t cols, int bits, size_t group, uint8_t *codes,
                 float *scales);

/* Quantized::dequantize_row (tensor/src/quant.rs:259-299): code as f32 times its group's scale. pinned. */
void or_dequantize_row(const uint8_t *codes, const float *scales, size_t cols, int bits, size_t group, size_t row,
                       float *out);

/* The one-token int8 product in Marin's AVX2 order (tensor/src/q8_gemv.rs:28-76, q8.rs:65-131): per group, four
 * 8-lane accumulators over the bytes of each 32-bit word, summed, then fused into the running total with the scale.
 * pinned: tolerance vs f64 dot of dequantized rows (cuda/tests/quant.rs:19-37) and hand values. */
void or_q8_gemv(const uint8_t *codes, const float *scales, const float *x, float *out, size_t rows, size_t cols,
                size_t group);

/* Any token count, int8 or int4: dequantize the row (a2) then the f64-accumulating `dot` of tensor/src/ops.rs:5-21
 * per token; this is q8.rs:117-128's scalar path. pinned. */
void or_matmul_dot(const uint8_t *codes, const float *scales, const float *x, float *out, size_t rows, size_t cols,
                   int bits, size_t group, size_t tokens);

/* tensor/src/ops.rs:5-21: eight f64 lanes, remainder, then the lane sum. pinned: ops.rs test dot 1..10 = 385. */
float or_dot(const float *a, const float *b, size_t n);

/* The vector exp of tensor/src/kernel.rs:73-98 (Cephes polynomial, input clamped to [-87.3, 88]). pinned: within a
 * few ulp of libm exp over a sweep. */
float or_exp(float x);

/* rms_norm_rows (tensor/src/norm.rs:6-58) in the 8-lane SIMD order. pinned: norm.rs hand values. */
void or_rms_norm_rows(float *x, size_t len, const float *weight, size_t dim, float eps);

/* rope_tokens (tensor/src/ops.rs:56-95): pairs (i, i + size/2), angle = pos * theta^(-2i/size). pinned: ops.rs hand
 * values. */
void or_rope_tokens(float *x, size_t len, size_t token_dim, size_t head_size, size_t start, float theta);

/* silu_mul (tensor/src/silu.rs:8-60) with the vector exp. pinned: silu.rs hand value. */
void or_silu_mul(float *gate, const float *up, size_t n);

/* softmax (tensor/src/ops.rs:23-33, libm exp). pinned: ops.rs hand values. */
void or_softmax(float *x, size_t n);

/* Grouped-query causal attention (tensor/src/attention.rs:39-173). One token takes AttendOne's order
 * (attention_one.rs:20-112: 4-accumulator vector dots, vector-exp softmax, values streamed in position order); more
 * tokens take attend_scalar (attention.rs:139-173). queries [tokens][heads][hd], keys/values [pos][kv_heads][hd].
 * pinned: attention.rs/qwen3 attention hand cases + f64 reference (cuda/tests/attention_reference/mod.rs). */
void or_attention(const float *queries, const float *keys, const float *values, float *out, size_t heads,
                  size_t kv_heads, size_t head_dim, size_t start, size_t tokens);

/* Plain f64 attention exactly as cuda/tests/attention_reference/mod.rs:1-49 (the reference's own test oracle). */
void or_attention_f64(const float *queries, const float *keys, const float *values, float *out, size_t heads,
                      size_t kv_heads, size_t head_dim, size_t start, size_t tokens);

/* Greedy choice: largest under f32 total order, lowest index on ties (sampler/src/lib.rs:40-48). pinned. */
uint32_t or_argmax(const float *values, size_t n);

/* Seeded synthetic weights: Irwin-Hall(12) approximation of N(0, std), computed in exact integer and one IEEE
 * double multiply, rounded to f32 then bf16. The GPU generator computes the same bits. Not from the reference
 * (which loads checkpoints); pinned by moments and by equality with the device generator. */
uint16_t or_synth_bf16(uint64_t seed, uint64_t stream, uint64_t index, double std_dev);
void or_synth_fill(uint64_t seed, uint64_t stream, double std_dev, uint16_t *out, size_t count);
/* Values start .. start + count - 1 of the same stream (a row range of a synthetic matrix). */
void or_synth_fill_at(uint64_t seed, uint64_t stream, double std_dev, uint64_t start, uint16_t *out, size_t count);

/* ---- Qwen3 forward (model/src/qwen3/model.rs:81-131, layer.rs:39-105, mlp.rs) over a contiguous f32 KV cache
 * (crates/kv). Weights are int8-quantized (Q8 path) or dense f32 (f64-dot path). ---- */
typedef struct or_matrix {
    size_t rows, cols, group;
    int bits;             /* 8 (int8 codes), or 0 for dense f32 */
    const uint8_t *codes; /* bits == 8 */
    const float *scales;
    const float *dense; /* bits == 0: [rows][cols] */
} or_matrix;

typedef struct or_layer {
    or_matrix q, k, v, o, gate, up, down;
    const float *input_norm, *post_norm, *q_norm, *k_norm;
} or_layer;

typedef struct or_qwen3 {
    size_t layers, hidden, heads, kv_heads, head_dim, ffn, vocab, capacity;
    float eps, theta;
    int kv_f16; /* store keys/values rounded to f16 (KvFormat::F16) */
    const or_layer *layer;
    or_matrix embed;   /* int8 table or dense */
    or_matrix lm_head; /* rows == 0 means tied to embed */
    const float *final_norm;
    /* cache: [layer][pos][kv_heads*head_dim] for keys and values */
    float *keys, *values;
    size_t len;
} or_qwen3;

/* One pass over `count` tokens at position model->len; writes the last token's logits. 0 on success. */
int or_qwen3_forward(or_qwen3 *model, const uint32_t *tokens, size_t count, float *logits);

/* ---- Synthetic Qwen3-shaped models (the benchmark configs). Tensor streams: embed 1, lm_head 2, layer l tensor i
 * ((l + 1) << 8 | i) with q 0, k 1, v 2, o 3, gate 4, up 5, down 6. Linear weights N(0, 0.02) via or_synth_bf16,
 * quantized int8 with `group`; norm weights are 1.0. The device library uses the same streams. ---- */
typedef struct or_synth_config {
    size_t layers, hidden, heads, kv_heads, head_dim, ffn, vocab, group, capacity;
    float eps, theta;
    int tied, kv_f16;
    uint64_t seed;
} or_synth_config;

uint64_t or_synth_stream(int layer, int tensor); /* layer -1: embed (tensor 0) or lm_head (tensor 1) */
uint32_t or_synth_prompt(uint64_t seed, uint64_t index, uint32_t vocab);
void *or_qwen3_synth_new(const or_synth_config *cfg);
or_qwen3 *or_qwen3_synth_model(void *handle);
void or_qwen3_synth_free(void *handle);
/* Prompt pass then `steps` greedy tokens. tokens_out[steps]; gaps_out[steps] = top-1 minus top-2 logit of each step
 * (how far the choice is from a tie); top_ids/top_vals[steps * 5] (optional) the five best logits of each step.
 * Returns 0 on success. */
/* The CPU baseline: seconds of one decode token of a model of this shape (constant weight codes, a filled cache of
 * `ctx` positions in the config's KV format) through or_qwen3_forward on one thread; negative on failure. */
double or_qwen3_time_token(const or_synth_config *cfg, size_t ctx);
int or_qwen3_greedy(void *handle, const uint32_t *prompt, size_t prompt_len, size_t steps, uint32_t *tokens_out,
                    float *gaps_out, size_t prefill_chunk, uint32_t *top_ids, float *top_vals);

#ifdef __cplusplus
}
#endif
#endif
