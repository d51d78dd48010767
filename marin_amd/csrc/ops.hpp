// Elementwise launchers shared by the C ABI and the Qwen3 driver.
#pragma once

#include "common.hpp"

namespace marin {

void launch_rms_norm(marin_gpu *g, const float *src, float *dst, const float *w, size_t rows, size_t dim, float eps);
void launch_rope(marin_gpu *g, float *x, size_t head_count, size_t heads, size_t hd, size_t start, float theta);
// theta^(-2i/hd) for i < hd/2, computed on the host with powf and cached on the device per (gpu, hd, theta).
const float *rope_frequencies(marin_gpu *g, size_t hd, float theta);
void forget_rope_frequencies(marin_gpu *g);
// The same table in memory the caller owns (released with gpu->release).
float *make_rope_frequencies(marin_gpu *g, size_t hd, float theta);
// RoPE cos/sin table [positions][hd/2] (float2) from a frequency table, on the device.
float2 *make_rope_table(marin_gpu *g, const float *freq, size_t hd, size_t positions);

}  // namespace marin
