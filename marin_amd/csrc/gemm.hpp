// The multi-token quantized product on the int8 matrix cores (gemm.hip).
#pragma once

#include "gemv.hpp"

namespace marin {

constexpr size_t GEMM_MIN_TOKENS = 5;  // token counts from which the GEMM replaces chunks of the decode product

// The routing plan of a decode batch's MoE layer (device int32 words, written by moe_plan): [0] the count U of
// distinct selected experts; [MOE_PLAN_EXPERTS + u] the u-th smallest of them; [MOE_PLAN_SLOTS + u * MOE_BATCH + t]
// the slot j with ids[t][j] == that expert, or -1.
constexpr int MOE_PLAN_MAX = 64;  // distinct experts of a batch: tokens x k
constexpr int MOE_BATCH = 8;      // tokens of a grouped batch
constexpr int MOE_PLAN_EXPERTS = 1;
constexpr int MOE_PLAN_SLOTS = 1 + MOE_PLAN_MAX;
constexpr int MOE_PLAN_WORDS = MOE_PLAN_SLOTS + MOE_PLAN_MAX * MOE_BATCH;
struct MoePlanView {
    const int32_t *plan = nullptr;
    int k = 0;    // slots per token
    int ffn = 0;  // activation row length
};

// int8 codes, group 64 or 128, at least GEMM_MIN_TOKENS tokens.
bool gemm_supported(const marin_quant_matrix *w, size_t tokens);
// The GEMM's layout requirement alone (int8 codes, group 64 or 128).
bool gemm_layout_ok(const marin_quant_matrix *w);
// y = the product of the quantized matrix with `tokens` (>= 1) activation rows (the same input and output modes as
// the decode product; with out.argmax_each, the greedy choice of every token into out.argmax[t]); uses the
// context's workspace for the activation limbs. Token blocks of 8 for up to 8 tokens, of 32 beyond.
void launch_gemm(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens);
// Activation limbs of `tokens` rows (quantize_act): limbs [tokens][4][cols] (or fragment order, below), the per-(token, group) factors
// 2^-s [tokens][groups] and the RMSNorm factors [tokens] (1 without a norm), placed in the context's workspace.
struct ActLimbs {
    const int8_t *limbs;
    const float *exps, *rs;
    const int32_t *lsum;  // fragment order only: each (token, group)'s four limb sums [tokens][groups][4]
};
// With `frag`, the limbs in B-operand fragment order instead ([window][token tile][64 lanes][16 bytes]).
ActLimbs launch_quantize_act(marin_gpu *g, const GemvIn &in, size_t tokens, size_t cols, size_t group, bool frag);
// Workspace bytes of launch_moe_gate_up (activation limbs of `tokens` rows of `cols`).
size_t moe_gate_up_workspace(size_t tokens, size_t cols, size_t group);
// The grouped gate_up of a decode batch (2..MOE_BATCH tokens): every distinct selected expert's [2F][H] rows read
// once for all tokens; act[t][slot][F] = SiLU(gate) * up for the tokens that selected it. `gate_up` is the stacked
// [experts * 2F][H] matrix; `plan` as above, for at most `max_experts` distinct experts.
void launch_moe_gate_up(marin_gpu *g, const marin_quant_matrix *gate_up, const GemvIn &in, size_t tokens,
                        const int32_t *plan, size_t max_experts, size_t k, size_t ffn, float *act);
// The product of a decode batch (gemv_batch.hip): 2..8 tokens, int8 codes, group 64 or 128.
bool gemv_batch_supported(const marin_quant_matrix *w, size_t tokens);
void launch_gemv_batch(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens);
// Any token count: the batch product for 2..8 tokens, the GEMM when it applies, else the decode product GEMV_TOKENS tokens at a time.
void launch_product(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens);

}  // namespace marin
