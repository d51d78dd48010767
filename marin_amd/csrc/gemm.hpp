// The multi-token quantized product on the int8 matrix cores (gemm.hip).
#pragma once

#include "gemv.hpp"

namespace marin {

constexpr size_t GEMM_MIN_TOKENS = 16;  // token counts from which the GEMM replaces chunks of the decode product

// int8 codes, group 64 or 128, at least GEMM_MIN_TOKENS tokens.
bool gemm_supported(const marin_quant_matrix *w, size_t tokens);
// y = the product of the quantized matrix with `tokens` activation rows (the same input and output modes as the
// decode product); uses the context's workspace for the activation limbs.
void launch_gemm(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens);
// Any token count: the GEMM when it applies, else the decode product GEMV_TOKENS tokens at a time.
void launch_product(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens);

}  // namespace marin
