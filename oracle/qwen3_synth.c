/*
 * Synthetic Qwen3-shaped models for the oracle (TEST INFRASTRUCTURE; see marin_oracle.c). Weights come from
 * or_synth_bf16 and go through the same quantizer (tensor/src/quant.rs:120-234) as a checkpoint would in
 * model/src/qwen3/gpu.rs:26-45: the embedding table and head with scheme.table() (int8), the projections with the
 * scheme. Generation follows runtime/src/generate.rs:105-284 for greedy sampling: one pass over the prompt, then one
 * pass per token, choosing with the lowest-index argmax.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "marin_oracle.h"

#include <string.h>
#include <time.h>

static inline uint64_t mix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

uint64_t or_synth_stream(int layer, int tensor) {
    if (layer < 0) return tensor == 0 ? 1u : 2u;
    return ((uint64_t)(layer + 1) << 8) | (uint64_t)tensor;
}

uint32_t or_synth_prompt(uint64_t seed, uint64_t index, uint32_t vocab) {
    return (uint32_t)(mix(mix(seed ^ 0x70726F6D7074ull) + index) % vocab);
}

typedef struct synth {
    or_qwen3 model;
    or_layer *layers;
    void **owned;
    size_t n_owned, cap_owned;
} synth;

static void *own(synth *s, size_t bytes) {
    if (s->n_owned == s->cap_owned) {
        s->cap_owned = s->cap_owned ? 2 * s->cap_owned : 64;
        s->owned = (void **)realloc(s->owned, s->cap_owned * sizeof(void *));
    }
    void *p = calloc(1, bytes ? bytes : 1);
    s->owned[s->n_owned++] = p;
    return p;
}

static void own_ptr(synth *s, void *p) {
    if (s->n_owned == s->cap_owned) {
        s->cap_owned = s->cap_owned ? 2 * s->cap_owned : 64;
        s->owned = (void **)realloc(s->owned, s->cap_owned * sizeof(void *));
    }
    s->owned[s->n_owned++] = p;
}

static int make_matrix(synth *s, uint64_t seed, uint64_t stream, size_t rows, size_t cols, size_t group,
                       or_matrix *m) {
    uint16_t *bits = (uint16_t *)malloc(rows * cols * sizeof(uint16_t));
    or_synth_fill(seed, stream, 0.02, bits, rows * cols);
    uint8_t *codes = (uint8_t *)own(s, rows * cols);
    float *scales = (float *)own(s, rows * (cols / group) * sizeof(float));
    /* Rows are quantized independently (tensor/src/quant.rs:134-170 splits them across threads the same way). */
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(| : bad)
    for (long r0 = 0; r0 < (long)rows; r0 += 256) {
        size_t n = rows - (size_t)r0 < 256 ? rows - (size_t)r0 : 256;
        if (or_quantize(bits + (size_t)r0 * cols, n, cols, 8, group, codes + (size_t)r0 * cols,
                        scales + (size_t)r0 * (cols / group)) != -1)
            bad = 1;
    }
    long rc = bad ? 0 : -1;
    free(bits);
    m->rows = rows;
    m->cols = cols;
    m->group = group;
    m->bits = 8;
    m->codes = codes;
    m->scales = scales;
    m->dense = NULL;
    return rc == -1 ? 0 : 1;
}

void *or_qwen3_synth_new(const or_synth_config *c) {
    synth *s = (synth *)calloc(1, sizeof(synth));
    or_qwen3 *M = &s->model;
    M->layers = c->layers;
    M->hidden = c->hidden;
    M->heads = c->heads;
    M->kv_heads = c->kv_heads;
    M->head_dim = c->head_dim;
    M->ffn = c->ffn;
    M->vocab = c->vocab;
    M->capacity = c->capacity;
    M->eps = c->eps;
    M->theta = c->theta;
    M->kv_f16 = c->kv_f16;
    const size_t H = c->hidden, qd = c->heads * c->head_dim, kvd = c->kv_heads * c->head_dim, F = c->ffn;
    float *ones = (float *)own(s, (H > qd ? H : qd) * sizeof(float));
    for (size_t i = 0; i < (H > qd ? H : qd); ++i) ones[i] = 1.0f;
    s->layers = (or_layer *)own(s, c->layers * sizeof(or_layer));
    int bad = 0;
    for (size_t l = 0; l < c->layers; ++l) {
        or_layer *L = &s->layers[l];
        bad |= make_matrix(s, c->seed, or_synth_stream((int)l, 0), qd, H, c->group, &L->q);
        bad |= make_matrix(s, c->seed, or_synth_stream((int)l, 1), kvd, H, c->group, &L->k);
        bad |= make_matrix(s, c->seed, or_synth_stream((int)l, 2), kvd, H, c->group, &L->v);
        bad |= make_matrix(s, c->seed, or_synth_stream((int)l, 3), H, qd, c->group, &L->o);
        bad |= make_matrix(s, c->seed, or_synth_stream((int)l, 4), F, H, c->group, &L->gate);
        bad |= make_matrix(s, c->seed, or_synth_stream((int)l, 5), F, H, c->group, &L->up);
        bad |= make_matrix(s, c->seed, or_synth_stream((int)l, 6), H, F, c->group, &L->down);
        L->input_norm = L->post_norm = L->q_norm = L->k_norm = ones;
    }
    M->layer = s->layers;
    bad |= make_matrix(s, c->seed, or_synth_stream(-1, 0), c->vocab, H, c->group, &M->embed);
    if (!c->tied) bad |= make_matrix(s, c->seed, or_synth_stream(-1, 1), c->vocab, H, c->group, &M->lm_head);
    M->final_norm = ones;
    M->keys = (float *)own(s, c->layers * c->capacity * kvd * sizeof(float));
    M->values = (float *)own(s, c->layers * c->capacity * kvd * sizeof(float));
    if (bad) {
        or_qwen3_synth_free(s);
        return NULL;
    }
    return s;
}

or_qwen3 *or_qwen3_synth_model(void *handle) { return &((synth *)handle)->model; }

void or_qwen3_synth_free(void *handle) {
    synth *s = (synth *)handle;
    if (!s) return;
    for (size_t i = 0; i < s->n_owned; ++i) free(s->owned[i]);
    free(s->owned);
    free(s);
}

int or_qwen3_greedy(void *handle, const uint32_t *prompt, size_t prompt_len, size_t steps, uint32_t *tokens_out,
                    float *gaps_out, size_t prefill_chunk, uint32_t *top_ids, float *top_vals) {
    or_qwen3 *M = &((synth *)handle)->model;
    float *logits = (float *)malloc(M->vocab * sizeof(float));
    if (prefill_chunk == 0) prefill_chunk = prompt_len;
    int rc = 0;
    for (size_t i = 0; i < prompt_len && !rc; i += prefill_chunk) {
        size_t n = prompt_len - i < prefill_chunk ? prompt_len - i : prefill_chunk;
        rc = or_qwen3_forward(M, prompt + i, n, logits);
    }
    for (size_t s = 0; s < steps && !rc; ++s) {
        uint32_t best = or_argmax(logits, M->vocab);
        float second = -3.4e38f;
        for (size_t i = 0; i < M->vocab; ++i)
            if (i != best && logits[i] > second) second = logits[i];
        tokens_out[s] = best;
        if (gaps_out) gaps_out[s] = logits[best] - second;
        if (top_ids) { /* the five largest, ties to the lower id */
            for (int k = 0; k < 5; ++k) {
                uint32_t pick = 0;
                int found = 0;
                for (size_t i = 0; i < M->vocab; ++i) {
                    int taken = 0;
                    for (int j = 0; j < k; ++j) taken |= top_ids[s * 5 + j] == i;
                    if (taken) continue;
                    if (!found || logits[i] > logits[pick]) { pick = (uint32_t)i; found = 1; }
                }
                top_ids[s * 5 + k] = pick;
                top_vals[s * 5 + k] = logits[pick];
            }
        }
        if (s + 1 < steps) rc = or_qwen3_forward(M, &best, 1, logits);
    }
    free(logits);
    return rc;
}

/* ---- the CPU baseline's timed token ----
 * One decode token of a model of the given shape through or_qwen3_forward after `ctx` cached positions, on one thread
 * (Marin decodes one token on one core, crates/tensor/src/q8.rs:67-74). The weights are a constant code pattern with
 * small scales and the cache a deterministic pattern already rounded to the cache format: the arithmetic, and so the
 * time, does not depend on the values, and filling memory is much cheaper than generating and quantizing the
 * synthetic weights. Every byte is written before the clock starts, so no page is first touched while timed.
 * Returns the seconds of the forward, or a negative value when memory runs out. */
static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

static int fill_matrix(synth *s, size_t rows, size_t cols, size_t group, or_matrix *m) {
    uint8_t *codes = (uint8_t *)malloc(rows * cols);
    float *scales = (float *)malloc(rows * (cols / group) * sizeof(float));
    if (!codes || !scales) {
        free(codes);
        free(scales);
        return 1;
    }
    own_ptr(s, codes);
    own_ptr(s, scales);
    memset(codes, 0x11, rows * cols);
    for (size_t i = 0; i < rows * (cols / group); ++i) scales[i] = 1e-3f;
    m->rows = rows;
    m->cols = cols;
    m->group = group;
    m->bits = 8;
    m->codes = codes;
    m->scales = scales;
    m->dense = NULL;
    return 0;
}

double or_qwen3_time_token(const or_synth_config *c, size_t ctx) {
    synth *s = (synth *)calloc(1, sizeof(synth));
    if (!s) return -1.0;
    or_qwen3 *M = &s->model;
    M->layers = c->layers;
    M->hidden = c->hidden;
    M->heads = c->heads;
    M->kv_heads = c->kv_heads;
    M->head_dim = c->head_dim;
    M->ffn = c->ffn;
    M->vocab = c->vocab;
    M->capacity = ctx + 1;
    M->eps = c->eps;
    M->theta = c->theta;
    M->kv_f16 = c->kv_f16;
    const size_t H = c->hidden, qd = c->heads * c->head_dim, kvd = c->kv_heads * c->head_dim, F = c->ffn;
    float *ones = (float *)own(s, (H > qd ? H : qd) * sizeof(float));
    for (size_t i = 0; i < (H > qd ? H : qd); ++i) ones[i] = 1.0f;
    s->layers = (or_layer *)own(s, c->layers * sizeof(or_layer));
    int bad = 0;
    for (size_t l = 0; l < c->layers && !bad; ++l) {
        or_layer *L = &s->layers[l];
        bad |= fill_matrix(s, qd, H, c->group, &L->q);
        bad |= fill_matrix(s, kvd, H, c->group, &L->k);
        bad |= fill_matrix(s, kvd, H, c->group, &L->v);
        bad |= fill_matrix(s, H, qd, c->group, &L->o);
        bad |= fill_matrix(s, F, H, c->group, &L->gate);
        bad |= fill_matrix(s, F, H, c->group, &L->up);
        bad |= fill_matrix(s, H, F, c->group, &L->down);
        L->input_norm = L->post_norm = L->q_norm = L->k_norm = ones;
    }
    M->layer = s->layers;
    if (!bad) bad |= fill_matrix(s, c->vocab, H, c->group, &M->embed);
    if (!bad && !c->tied) bad |= fill_matrix(s, c->vocab, H, c->group, &M->lm_head);
    M->final_norm = ones;
    const size_t kv_len = c->layers * M->capacity * kvd;
    M->keys = bad ? NULL : (float *)malloc(kv_len * sizeof(float));
    M->values = bad ? NULL : (float *)malloc(kv_len * sizeof(float));
    if (bad || !M->keys || !M->values) {
        free(M->keys);
        free(M->values);
        or_qwen3_synth_free(s);
        return -1.0;
    }
    own_ptr(s, M->keys);
    own_ptr(s, M->values);
    /* small values that an f16 cache holds exactly: multiples of 2^-8 in (-1, 1) */
    for (size_t i = 0; i < kv_len; ++i) {
        M->keys[i] = (float)((int)((i * 2654435761u) >> 24 & 0xff) - 128) * 0.00390625f;
        M->values[i] = (float)((int)((i * 40503u + 7u) >> 8 & 0xff) - 128) * 0.00390625f;
    }
    M->len = ctx;
    float *logits = (float *)malloc(c->vocab * sizeof(float));
    if (!logits) {
        or_qwen3_synth_free(s);
        return -1.0;
    }
    memset(logits, 0, c->vocab * sizeof(float));
    const uint32_t token = 17;
    or_set_threads(1);
    const double t0 = now_s();
    const int rc = or_qwen3_forward(M, &token, 1, logits);
    const double sec = now_s() - t0;
    free(logits);
    or_qwen3_synth_free(s);
    return rc ? -2.0 : sec;
}
