// The matrix-core quantized product (gemv.hip): inputs, outputs and the launcher.
#pragma once

#include <hip/hip_runtime.h>

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

// The four signed 8-bit limbs of four integers below 2^30 in magnitude: x = l3 2^24 + l2 2^16 + l1 2^8 + l0 with
// l0..l2 in [-128, 127] (the balanced base-256 digits, unique), word l holding limb l of x0..x3 in bytes 0..3. With
// y = x + 0x808080 the low three bytes of y are l0..l2 + 128 and y's top byte is l3, so the digits are byte gathers
// (v_perm_b32) and one XOR of the sign bits.
__device__ __forceinline__ void limbs4(int x0, int x1, int x2, int x3, uint32_t w[4]) {
    const uint32_t y0 = (uint32_t)x0 + 0x808080u, y1 = (uint32_t)x1 + 0x808080u;
    const uint32_t y2 = (uint32_t)x2 + 0x808080u, y3 = (uint32_t)x3 + 0x808080u;
    const uint32_t a01 = __builtin_amdgcn_perm(y1, y0, 0x05010400u);  // y0.b0 y1.b0 y0.b1 y1.b1
    const uint32_t a23 = __builtin_amdgcn_perm(y3, y2, 0x05010400u);
    const uint32_t c01 = __builtin_amdgcn_perm(y1, y0, 0x07030602u);  // y0.b2 y1.b2 y0.b3 y1.b3
    const uint32_t c23 = __builtin_amdgcn_perm(y3, y2, 0x07030602u);
    w[0] = __builtin_amdgcn_perm(a23, a01, 0x05040100u) ^ 0x80808080u;
    w[1] = __builtin_amdgcn_perm(a23, a01, 0x07060302u) ^ 0x80808080u;
    w[2] = __builtin_amdgcn_perm(c23, c01, 0x05040100u) ^ 0x80808080u;
    w[3] = __builtin_amdgcn_perm(c23, c01, 0x07060302u);
}

bool gemv_supported(const marin_quant_matrix *w);
// The one-token product (gemv_decode.hip): the matrix-core arithmetic on a latency-first schedule.
bool gemv_decode_supported(const marin_quant_matrix *w);
// Returns the launched instantiation's name.
const char *launch_gemv_decode(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out);
void launch_gemv(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens);

}  // namespace marin
