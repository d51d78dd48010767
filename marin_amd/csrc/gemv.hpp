// The matrix-core quantized product (gemv.hip): inputs, outputs and the launcher.
#pragma once

#include "quant.hpp"

namespace marin {

constexpr int GEMV_TOKENS = 4;  // tokens per launch (four 8-bit limbs each fill the 16 B columns)

enum GemvInMode : int {
    IN_F32 = 0,   // x f32 [tokens][x_stride]
    IN_NORM = 1,  // RMSNorm(x) * norm, x f32 [tokens][x_stride] (kernels.cu:51-60 order: x * rs * w)
    IN_BF16 = 2   // x bf16 [tokens][x_stride]
};
enum GemvOutMode : int {
    OUT_F32 = 0,   // y[t][r] = v
    OUT_ADD = 1,   // y[t][r] += v (residual)
    OUT_BF16 = 2,  // y bf16
    OUT_SILU = 3   // rows (2i, 2i+1) = (gate_i, up_i): y[t][i] = silu(gate_i) * up_i
};

struct GemvIn {
    int mode = IN_F32;
    const void *x = nullptr;
    size_t x_stride = 0;
    const float *norm = nullptr;
    float eps = 0.0f;
    // Optional (one-token product only): the product runs over the 16-row tiles of `map_count` blocks of
    // `map_tiles` tiles each, block j being block tile_map[j] of the matrix (device ids, e.g. selected experts);
    // output row r of the product is logical row r of that concatenation.
    const int32_t *tile_map = nullptr;
    int map_tiles = 0, map_count = 0;
    int map_blocks = 0;  // blocks of map_tiles tiles in the matrix: map entries are clamped below it
};

struct GemvOut {
    int mode = OUT_F32;
    void *y = nullptr;
    size_t y_stride = 0;
    unsigned long long *argmax = nullptr;  // optional: atomic max of (total-order key, ~row) of the last token
    bool argmax_each = false;              // with argmax: one word per token, argmax[t] (multi-token GEMM only)
};

bool gemv_supported(const marin_quant_matrix *w);
// The one-token product (gemv_decode.hip): the matrix-core arithmetic on a latency-first schedule.
bool gemv_decode_supported(const marin_quant_matrix *w);
// Returns the launched instantiation's name.
const char *launch_gemv_decode(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out);
void launch_gemv(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens);

}  // namespace marin
