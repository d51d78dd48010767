// Dense bf16 matrices: the DeviceMatrix half of the reference's `cuda` crate (crates/cuda/src/gpu.rs:248-268
// upload_matrix, matmul.rs:16-205 matmul / matmul_precise / matmul_pair / matmul_triple, ops.rs:55-73 embed).
//
// Two products, chosen as the reference chooses (matmul.rs:51): from MMA_MIN_TOKENS tokens with columns a multiple of
// 16, `matmul` runs on the matrix cores; every other pass, and `matmul_precise` always, runs on the vector ALUs.
//  - dense_rows: a wave per weight row, 8 tokens per workgroup column. A lane owns 8 consecutive columns per 512-column
//    step (one 16-byte load of bf16 weights, f32 FMA with the tokens' activations), then the wave sums its lanes in a
//    fixed butterfly. Grouped launches (pair, triple) take the concatenation of their matrices' rows with exactly the
//    same per-row arithmetic, so they give the same bits as separate launches (the reference's own test,
//    cuda/tests/ops.rs:57-110).
//  - dense_mfma: 64 rows x 64 tokens per workgroup of 4 waves on v_mfma_f32_16x16x32_bf16. The f32 activations are
//    split into three bf16 parts (8 + 8 + 8 significant bits, the whole f32 significand) and all three are
//    multiplied, so every product is exact and only the f32 accumulation rounds (the split mma.cu:1-9 describes; two
//    parts, 16 bits, miss the 1e-4 tolerance on 4096-column rows). Weight and activation tiles of 32 columns are
//    staged through LDS, the next tile's global loads in flight while the current one is multiplied.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "common.hpp"

struct marin_matrix {
    marin_gpu *gpu = nullptr;
    size_t rows = 0, cols = 0;
    uint16_t *data = nullptr;  // bf16 bits, row-major [rows][cols] (DeviceMatrix, gpu.rs:87-93)
};

namespace marin {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef short bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int ROWS_PER_BLOCK = 4;   // waves (rows) per vector workgroup
constexpr int TOKEN_TILE = 8;       // tokens per vector workgroup
constexpr size_t MMA_MIN_TOKENS = 16;  // matmul.rs:13
constexpr int MT = 64;              // rows per matrix-core workgroup
constexpr int NTOK = 64;            // tokens per matrix-core workgroup
constexpr int KT = 32;              // columns per staged tile
constexpr int KP = KT + 8;          // LDS row pitch in bf16 (16 bytes of padding)

__device__ __forceinline__ float bf16_f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__device__ __forceinline__ uint16_t f_bf16_rne(float v) {
    const uint32_t u = __float_as_uint(v);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Up to three matrices over one input: rows [0, r0) of the launch are matrix 0's, then matrix 1's, then matrix 2's.
struct DenseSet {
    const uint16_t *w[3];
    float *y[3];
    uint32_t rows[3];
};

}  // namespace

__global__ __launch_bounds__(64 * ROWS_PER_BLOCK) void dense_rows(DenseSet set, const float *__restrict__ x,
                                                                  uint32_t cols, uint32_t tokens) {
    const uint32_t lane = threadIdx.x & 63;
    uint32_t row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6);
    int m = 0;
    if (row >= set.rows[0]) {
        row -= set.rows[0];
        m = 1;
        if (row >= set.rows[1]) {
            row -= set.rows[1];
            m = 2;
            if (row >= set.rows[2]) return;
        }
    }
    const uint32_t rows = set.rows[m];
    const uint16_t *wrow = set.w[m] + (size_t)row * cols;
    const uint32_t t0 = blockIdx.y * TOKEN_TILE;
    const uint32_t nt = min((uint32_t)TOKEN_TILE, tokens - t0);
    float acc[TOKEN_TILE];
#pragma unroll
    for (int j = 0; j < TOKEN_TILE; ++j) acc[j] = 0.0f;
    if ((cols & 7u) == 0u) {
        for (uint32_t c = lane * 8; c < cols; c += 512) {
            const u32x4 p = *reinterpret_cast<const u32x4 *>(wrow + c);
            float wf[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                wf[2 * i] = bf16_f(p[i] & 0xffffu);
                wf[2 * i + 1] = __uint_as_float(p[i] & 0xffff0000u);
            }
#pragma unroll
            for (int j = 0; j < TOKEN_TILE; ++j) {
                if ((uint32_t)j >= nt) break;
                const float4 *xv = reinterpret_cast<const float4 *>(x + (size_t)(t0 + j) * cols + c);
                const float4 a = xv[0], b = xv[1];
                float s = acc[j];
                s = fmaf(wf[0], a.x, s);
                s = fmaf(wf[1], a.y, s);
                s = fmaf(wf[2], a.z, s);
                s = fmaf(wf[3], a.w, s);
                s = fmaf(wf[4], b.x, s);
                s = fmaf(wf[5], b.y, s);
                s = fmaf(wf[6], b.z, s);
                s = fmaf(wf[7], b.w, s);
                acc[j] = s;
            }
        }
    } else {
        for (uint32_t c = lane; c < cols; c += 64) {
            const float wf = bf16_f(wrow[c]);
#pragma unroll
            for (int j = 0; j < TOKEN_TILE; ++j) {
                if ((uint32_t)j >= nt) break;
                acc[j] = fmaf(wf, x[(size_t)(t0 + j) * cols + c], acc[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < TOKEN_TILE; ++j) {
        float v = acc[j];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0 && (uint32_t)j < nt) set.y[m][(size_t)(t0 + j) * rows + row] = v;
    }
}

// grid: (rows / 64, tokens / 64), 4 waves; wave w computes rows 16 w .. + 15 of the tile for all 64 tokens.
// Operand layouts of v_mfma_f32_16x16x32_bf16 (lane l, c = l % 16, q = l / 16): A row c, columns 8 q .. + 7; B token
// c, columns 8 q .. + 7; C row 4 q + i, token c.
__global__ __launch_bounds__(256) void dense_mfma(const uint16_t *__restrict__ w, const float *__restrict__ x,
                                                  float *__restrict__ y, uint32_t rows, uint32_t cols,
                                                  uint32_t tokens) {
    __shared__ __align__(16) uint16_t ws[MT][KP];
    __shared__ __align__(16) uint16_t xh[NTOK][KP];
    __shared__ __align__(16) uint16_t xm[NTOK][KP];
    __shared__ __align__(16) uint16_t xl[NTOK][KP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 15, q = lane >> 4;
    const uint32_t row0 = blockIdx.x * MT, tok0 = blockIdx.y * NTOK;
    // staging: thread t takes row / token t / 4, columns 8 (t % 4) .. + 7 of the tile
    const int sr = tid >> 2, sk = (tid & 3) * 8;
    const bool wrow_ok = row0 + sr < rows, xtok_ok = tok0 + sr < tokens;
    const uint16_t *wp = w + (size_t)min(row0 + sr, rows - 1) * cols;
    const float *xp = x + (size_t)min(tok0 + sr, tokens - 1) * cols;
    u32x4 wv;
    float4 xa, xb;
    auto load = [&](uint32_t k0) {
        const uint32_t k = k0 + sk;
        const bool in = k < cols;  // cols is a multiple of 8
        const uint32_t kc = in ? k : 0;
        wv = *reinterpret_cast<const u32x4 *>(wp + kc);
        xa = *reinterpret_cast<const float4 *>(xp + kc);
        xb = *reinterpret_cast<const float4 *>(xp + kc + 4);
        if (!(in && wrow_ok)) wv = (u32x4){0u, 0u, 0u, 0u};
        if (!(in && xtok_ok)) xa = xb = make_float4(0.f, 0.f, 0.f, 0.f);
    };
    floatx4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = (floatx4){0.f, 0.f, 0.f, 0.f};
    load(0);
    for (uint32_t k0 = 0; k0 < cols; k0 += KT) {
        *reinterpret_cast<u32x4 *>(&ws[sr][sk]) = wv;
        {
            const float v[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            u32x4 hi, mid, lo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint16_t p[2][3];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float x = v[2 * i + j];
                    p[j][0] = f_bf16_rne(x);
                    const float r1 = x - bf16_f(p[j][0]);  // exact
                    p[j][1] = f_bf16_rne(r1);
                    p[j][2] = f_bf16_rne(r1 - bf16_f(p[j][1]));
                }
                hi[i] = (uint32_t)p[0][0] | ((uint32_t)p[1][0] << 16);
                mid[i] = (uint32_t)p[0][1] | ((uint32_t)p[1][1] << 16);
                lo[i] = (uint32_t)p[0][2] | ((uint32_t)p[1][2] << 16);
            }
            *reinterpret_cast<u32x4 *>(&xh[sr][sk]) = hi;
            *reinterpret_cast<u32x4 *>(&xm[sr][sk]) = mid;
            *reinterpret_cast<u32x4 *>(&xl[sr][sk]) = lo;
        }
        __syncthreads();
        if (k0 + KT < cols) load(k0 + KT);  // the next tile in flight during the products
        const bf16x8 a = *reinterpret_cast<const bf16x8 *>(&ws[16 * wave + c][8 * q]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bf16x8 bh = *reinterpret_cast<const bf16x8 *>(&xh[16 * j + c][8 * q]);
            const bf16x8 bm = *reinterpret_cast<const bf16x8 *>(&xm[16 * j + c][8 * q]);
            const bf16x8 bl = *reinterpret_cast<const bf16x8 *>(&xl[16 * j + c][8 * q]);
            // smallest part first: the exact products of the low parts are added before the large ones
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bm, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh, acc[j], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t t = tok0 + 16 * j + c;
        if (t >= tokens) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = row0 + 16 * wave + 4 * q + i;
            if (r < rows) y[(size_t)t * rows + r] = acc[j][i];
        }
    }
}

// out[t][i] = table[ids[t]][i] as f32 (kernels.cu embed: a block per token).
__global__ __launch_bounds__(256) void dense_embed(const uint16_t *__restrict__ table, const uint32_t *__restrict__ ids,
                                                   float *__restrict__ out, uint32_t cols) {
    const uint16_t *row = table + (size_t)ids[blockIdx.x] * cols;
    float *o = out + (size_t)blockIdx.x * cols;
    for (uint32_t i = threadIdx.x; i < cols; i += 256) o[i] = bf16_f(row[i]);
}

static void launch_rows(marin_gpu *g, const DenseSet &set, size_t total_rows, const float *x, size_t cols,
                        size_t tokens) {
    dim3 grid(to_u32((total_rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK, "grid size"),
              to_u32((tokens + TOKEN_TILE - 1) / TOKEN_TILE, "grid size"));
    dense_rows<<<grid, 64 * ROWS_PER_BLOCK, 0, g->stream>>>(set, x, to_u32(cols, "cols"), to_u32(tokens, "tokens"));
    g->launched();
}

static void launch_one(marin_gpu *g, const marin_matrix *w, const float *x, size_t tokens, float *y, bool mma) {
    if (mma && tokens >= MMA_MIN_TOKENS && w->cols % 16 == 0) {
        dim3 grid(to_u32((w->rows + MT - 1) / MT, "grid size"), to_u32((tokens + NTOK - 1) / NTOK, "grid size"));
        dense_mfma<<<grid, 256, 0, g->stream>>>(w->data, x, y, to_u32(w->rows, "rows"), to_u32(w->cols, "cols"),
                                                to_u32(tokens, "tokens"));
        g->launched();
        return;
    }
    DenseSet set{};
    set.w[0] = w->data;
    set.y[0] = y;
    set.rows[0] = to_u32(w->rows, "rows");
    launch_rows(g, set, w->rows, x, w->cols, tokens);
}

static void check_f32(const marin_buffer *b, const char *what, size_t len) {
    if (b->dtype != MARIN_F32) shape(what, 4, dtype_bytes(b->dtype));
    check_len(what, len, b->len);
}

// matmul.rs:168-205 (grouped_plan): every matrix has the input's columns and an output of tokens x its rows.
static void grouped(marin_gpu *g, const marin_matrix *const *ws, marin_buffer *const *ys, int n, const marin_buffer *x,
                    size_t tokens) {
    const size_t cols = ws[0]->cols;
    size_t total = 0;
    for (int i = 0; i < n; ++i) {
        if (ws[i]->cols != cols) shape("grouped matmul columns", cols, ws[i]->cols);
        check_f32(ys[i], "matmul output", mul(tokens, ws[i]->rows, "matmul output"));
        total += ws[i]->rows;
    }
    check_f32(x, "matmul input", mul(tokens, cols, "matmul input"));
    if (!tokens || !total || !cols) return;
    if (tokens >= MMA_MIN_TOKENS && cols % 16 == 0) {  // Plan::Each: the matrix-core kernel per matrix
        for (int i = 0; i < n; ++i)
            if (ws[i]->rows) launch_one(g, ws[i], (const float *)x->data, tokens, (float *)ys[i]->data, true);
        return;
    }
    DenseSet set{};
    for (int i = 0; i < n; ++i) {
        set.w[i] = ws[i]->data;
        set.y[i] = (float *)ys[i]->data;
        set.rows[i] = to_u32(ws[i]->rows, "rows");
    }
    launch_rows(g, set, total, (const float *)x->data, cols, tokens);
}

}  // namespace marin

using namespace marin;

extern "C" {

marin_status marin_upload_matrix(marin_gpu *g, size_t rows, size_t cols, const uint16_t *bits, size_t len,
                                 marin_matrix **out) {
    return guard([&] {
        const size_t expected = mul(rows, cols, "matrix");
        check_len("matrix data", expected, len);
        auto *m = new marin_matrix();
        m->gpu = g;
        m->rows = rows;
        m->cols = cols;
        try {
            m->data = (uint16_t *)g->alloc(mul(expected, 2, "matrix") + 16, false);
            g->upload(m->data, bits, expected * 2);
        } catch (...) {
            if (m->data) g->release(m->data);
            delete m;
            throw;
        }
        *out = m;
    });
}

void marin_matrix_free(marin_matrix *m) {
    if (!m) return;
    (void)hipStreamSynchronize(m->gpu->stream);
    m->gpu->release(m->data);
    delete m;
}

void marin_matrix_shape(const marin_matrix *m, size_t *rows, size_t *cols) {
    if (rows) *rows = m->rows;
    if (cols) *cols = m->cols;
}

marin_status marin_embed(marin_gpu *g, const marin_matrix *table, const uint32_t *ids, size_t n,
                         marin_tokens *scratch, marin_buffer *out) {
    return guard([&] {
        check_f32(out, "embed output", mul(n, table->cols, "embed output"));
        for (size_t i = 0; i < n; ++i)
            if (ids[i] >= table->rows) shape("token id", table->rows, ids[i]);
        if (n == 0) return;
        if (n > scratch->capacity) shape("embed token capacity", scratch->capacity, n);
        void *staged = g->stage(ids, n * 4);
        HIP_CHECK(hipMemcpyAsync(scratch->data, staged, n * 4, hipMemcpyHostToDevice, g->stream));
        g->traffic.uploads++;
        g->traffic.upload_bytes += n * 4;
        if (!table->cols) return;
        dense_embed<<<to_u32(n, "token count"), 256, 0, g->stream>>>(table->data, scratch->data, (float *)out->data,
                                                                      to_u32(table->cols, "hidden size"));
        g->launched();
    });
}

static marin_status matmul_entry(marin_gpu *g, const marin_matrix *w, const marin_buffer *x, size_t tokens,
                                 marin_buffer *out, bool mma) {
    return guard([&] {
        check_f32(x, "matmul input", mul(tokens, w->cols, "matmul input"));
        check_f32(out, "matmul output", mul(tokens, w->rows, "matmul output"));
        if (!tokens || !w->rows || !w->cols) return;
        launch_one(g, w, (const float *)x->data, tokens, (float *)out->data, mma);
    });
}

marin_status marin_matmul(marin_gpu *g, const marin_matrix *w, const marin_buffer *x, size_t tokens,
                          marin_buffer *out) {
    return matmul_entry(g, w, x, tokens, out, true);
}

marin_status marin_matmul_precise(marin_gpu *g, const marin_matrix *w, const marin_buffer *x, size_t tokens,
                                  marin_buffer *out) {
    return matmul_entry(g, w, x, tokens, out, false);
}

marin_status marin_matmul_pair(marin_gpu *g, const marin_matrix *w0, const marin_matrix *w1, const marin_buffer *x,
                               size_t tokens, marin_buffer *y0, marin_buffer *y1) {
    return guard([&] {
        const marin_matrix *ws[2] = {w0, w1};
        marin_buffer *ys[2] = {y0, y1};
        grouped(g, ws, ys, 2, x, tokens);
    });
}

marin_status marin_matmul_triple(marin_gpu *g, const marin_matrix *w0, const marin_matrix *w1,
                                 const marin_matrix *w2, const marin_buffer *x, size_t tokens, marin_buffer *y0,
                                 marin_buffer *y1, marin_buffer *y2) {
    return guard([&] {
        const marin_matrix *ws[3] = {w0, w1, w2};
        marin_buffer *ys[3] = {y0, y1, y2};
        grouped(g, ws, ys, 3, x, tokens);
    });
}

}  // extern "C"
