// Mixture-of-experts decode FFN (config 4: Qwen3-30B-A3B-shaped, int8 group-128 experts). The reference has no
// Qwen3-MoE; its analogue is Granite's route / expert GEMV / mix (crates/cuda/src/granite.cu:12-118: top-k first,
// then a softmax over the k, bf16 experts). Qwen3-MoE routes by a softmax over all experts, the k largest
// probabilities (lowest expert id on ties, like the sampler's argmax, sampler/src/lib.rs:40-48), renormalized to sum
// to 1 when asked (norm_topk_prob).
//
// The experts of a layer are two stacked quantized matrices: gate_up [experts * 2F][H] with expert e's rows at
// [e * 2F, (e + 1) * 2F), gate and up interleaved row by row; down [experts * H][F] with expert e's rows at
// [e * H, (e + 1) * H). One token's FFN is:
//  - gate_up: the one-token product over the selected experts' tiles only (a tile map of device expert ids), RMSNorm
//    of the hidden state in its prologue and SiLU(gate) * up in its epilogue -> act [k][F];
//  - expert_down: a workgroup per 16 output rows, a wave per selected expert with that expert's act limbs; the waves'
//    rows weighted by the routing weights and summed in slot order into the residual.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "gemm.hpp"
#include "gemv.hpp"

namespace marin {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int ROUTE_THREADS = 256;
constexpr int MOE_MAX_K = 8;

__device__ __forceinline__ unsigned total_key(float v) {
    const unsigned b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);  // ascending with the float's total order
}

}  // namespace

// One token per workgroup: probabilities p_e = exp(l_e - max) / sum over the experts; the k largest (lowest id on
// ties) in descending order; weights p_e, or p_e / sum of the k when `renorm`.
__global__ __launch_bounds__(ROUTE_THREADS) void moe_route(const float *__restrict__ logits, int experts, int k,
                                                           int renorm, int32_t *__restrict__ ids,
                                                           float *__restrict__ weights, uint32_t *__restrict__ fault) {
    __shared__ float p_s[1024];
    __shared__ unsigned long long best_s[ROUTE_THREADS / 64];
    __shared__ float red_s[ROUTE_THREADS / 64];
    __shared__ float sel_p[MOE_MAX_K];
    __shared__ int sel_i[MOE_MAX_K];
    const int b = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float *l = logits + (size_t)b * experts;
    float mx = -INFINITY;
    bool finite = true;
    for (int e = threadIdx.x; e < experts; e += ROUTE_THREADS) {
        const float v = l[e];
        finite = finite && fabsf(v) <= 3.402823466e38f;  // false for NaN and both infinities
        mx = fmaxf(mx, v);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) red_s[wave] = mx;
    // The reference refuses non-finite router logits (model/src/granite/layer.rs:42-47). Such a token is routed to
    // experts 0..k-1 with weight 0, so nothing downstream reads outside the experts, and the fault word reports it
    // at the next blocking call.
    if (__syncthreads_or(!finite)) {
        if (threadIdx.x < k) {
            ids[(size_t)b * k + threadIdx.x] = (int32_t)threadIdx.x;
            weights[(size_t)b * k + threadIdx.x] = 0.0f;
        }
        if (threadIdx.x == 0) *fault = FAULT_ROUTER_NONFINITE;
        return;
    }
    mx = red_s[0];
    for (int w = 1; w < ROUTE_THREADS / 64; ++w) mx = fmaxf(mx, red_s[w]);
    __syncthreads();
    float sum = 0.0f;
    for (int e = threadIdx.x; e < experts; e += ROUTE_THREADS) {
        const float v = expf(l[e] - mx);
        p_s[e] = v;
        sum += v;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    if (lane == 0) red_s[wave] = sum;
    __syncthreads();
    sum = 0.0f;
    for (int w = 0; w < ROUTE_THREADS / 64; ++w) sum += red_s[w];
    for (int e = threadIdx.x; e < experts; e += ROUTE_THREADS) p_s[e] = p_s[e] / sum;
    __syncthreads();
    for (int j = 0; j < k; ++j) {
        // largest remaining probability, lowest id on ties: key = (total order of p) << 32 | ~id
        unsigned long long best = 0ull;
        for (int e = threadIdx.x; e < experts; e += ROUTE_THREADS) {
            const float v = p_s[e];
            if (v != v) continue;
            bool taken = false;
            for (int i = 0; i < j; ++i) taken |= sel_i[i] == e;
            if (taken) continue;
            const unsigned long long key = (unsigned long long)total_key(v) << 32 | (0xffffffffu - (unsigned)e);
            best = key > best ? key : best;
        }
        for (int o = 32; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(best, o);
            best = other > best ? other : best;
        }
        if (lane == 0) best_s[wave] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            unsigned long long m = 0ull;
            for (int w = 0; w < ROUTE_THREADS / 64; ++w) m = best_s[w] > m ? best_s[w] : m;
            const int e = (int)(0xffffffffu - (unsigned)(m & 0xffffffffull));
            sel_i[j] = e;
            sel_p[j] = p_s[e];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int j = 0; j < k; ++j) s += sel_p[j];
        for (int j = 0; j < k; ++j) {
            ids[(size_t)b * k + j] = sel_i[j];
            weights[(size_t)b * k + j] = renorm ? sel_p[j] / s : sel_p[j];
        }
    }
}

// The routing plan of a decode batch (tokens * k <= 64 selections), one wave: the distinct selected experts in
// ascending order and, per (distinct expert, token), the slot that selected it or -1 (layout in gemm.hpp).
__global__ __launch_bounds__(64) void moe_plan(const int32_t *__restrict__ ids, int tokens, int k, int experts,
                                               int32_t *__restrict__ plan) {
    __shared__ int32_t slots[MOE_PLAN_MAX * MOE_BATCH];
    const int lane = threadIdx.x, n = tokens * k;
    const int id = min(max(ids[min(lane, n - 1)], 0), experts - 1);  // ids from outside stay inside the experts
    bool first = lane < n;  // first occurrence of its expert
    int rank = 0;           // distinct experts below it
    for (int j = 0; j < n; ++j) {
        const int v = __shfl(id, j);
        first = first && !(j < lane && v == id);
    }
    const unsigned long long firsts = __ballot(first);
    for (int j = 0; j < n; ++j) {
        const int v = __shfl(id, j);
        rank += ((firsts >> j) & 1ull) && v < id;
    }
    for (int i = lane; i < MOE_PLAN_MAX * MOE_BATCH; i += 64) slots[i] = -1;
    __syncthreads();
    if (lane < n) slots[rank * MOE_BATCH + lane / k] = lane % k;
    __syncthreads();
    for (int i = lane; i < MOE_PLAN_MAX * MOE_BATCH; i += 64) plan[MOE_PLAN_SLOTS + i] = slots[i];
    if (first) plan[MOE_PLAN_EXPERTS + rank] = id;
    if (lane == 0) plan[0] = __popcll(firsts);
}

// grid: (H / 16 output tiles, tokens); a wave per expert slot j < k. WG: 64-column windows per group; MW: windows of
// an expert's input (F / 64, at most 16) rounded up to what the template holds.

template <int WG, int MW, typename ST>
__global__ __launch_bounds__(64 * MOE_MAX_K) void expert_down(const uint8_t *__restrict__ codes,
                                                              const ST *__restrict__ scales,
                                                              const float *__restrict__ act,
                                                              const int32_t *__restrict__ ids,
                                                              const float *__restrict__ weights, int k, int experts,
                                                              int hidden, int ffn, float *__restrict__ out, int half) {
    __shared__ __align__(16) int8_t limbs[MOE_MAX_K][MW][4][64];
    __shared__ float gdown[MOE_MAX_K][MW];
    __shared__ float red[MOE_MAX_K][16];
    const int lane = threadIdx.x & 63;
    const int slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    // half tiles (half = 1): workgroup x takes rows 8 (x % 2) .. + 7 of tile x / 2; the lanes of the other 8 rows
    // load their partner's row, so the MFMA's rows 8..15 repeat rows 0..7 and are dropped
    const int b = blockIdx.y, tile = (int)blockIdx.x >> half, hb = (int)blockIdx.x & half;
    const int la = half ? (c & 7) + 8 * hb + 16 * q : lane;  // the lane whose 16 code bytes this lane loads
    const int qs = half ? (q & 1) + 2 * hb : q;               // the rows 4 qs .. + 3 whose scales it takes
    const int windows = ffn >> 6, groups = windows / WG;
    const int tiles_per_expert = hidden / 16;
    const bool on = slot < k;
    const int e = min(max(ids[(size_t)b * k + min(slot, k - 1)], 0), experts - 1);
    const size_t ptile = (size_t)e * tiles_per_expert + tile;
    // the expert's activation row first (lane L takes 16 consecutive columns), then every code window of the tile
    const float *arow = act + ((size_t)b * k + min(slot, k - 1)) * ffn;
    const int cb = min(16 * lane, ffn - 16);
    float4 xv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) xv[v] = *reinterpret_cast<const float4 *>(arow + cb + 4 * v);
    u32x4 a[MW];
    floatx4 sc[MW / WG];
#pragma unroll
    for (int w = 0; w < MW; ++w) {
        const int wc = min(w, windows - 1);
        a[w] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(codes + ptile * 16 * ffn + (size_t)wc * 1024 + 16 * la));
        if (w % WG == 0) {
            const ST *sp = scales + (ptile * groups + wc / WG) * 16 + 4 * qs;
            if constexpr (sizeof(ST) == 4) {
                sc[w / WG] = *reinterpret_cast<const floatx4 *>(sp);
            } else {
                const uint2 sv = *reinterpret_cast<const uint2 *>(sp);
                sc[w / WG] = (floatx4){__uint_as_float(sv.x << 16), __uint_as_float(sv.x & 0xffff0000u),
                                       __uint_as_float(sv.y << 16), __uint_as_float(sv.y & 0xffff0000u)};
            }
        }
    }
    // limbs of the expert's activations, per group exponent (the group's 4 * WG lanes are consecutive)
    {
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[4 * i] = xv[i].x;
            v[4 * i + 1] = xv[i].y;
            v[4 * i + 2] = xv[i].z;
            v[4 * i + 3] = xv[i].w;
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[i]));
        for (int o = 1; o < 4 * WG; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        int sh = 0;
        if (mx > 0.0f && mx < INFINITY) {
            int ex;
            (void)frexpf(mx, &ex);
            sh = 30 - ex;
            sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
        }
        const float up = ldexpf(1.0f, sh);
        u32x4 pk[4];
#pragma unroll
        for (int l = 0; l < 4; ++l) pk[l] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int xi = __float2int_rn(v[i] * up);
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const int lb = l == 3 ? xi : (int)(int8_t)(xi & 0xff);
                pk[l][i / 4] |= ((uint32_t)lb & 0xffu) << (8 * (i % 4));
                xi = (xi - lb) >> 8;
            }
        }
        const int wl = lane / 4;  // window of the lane's columns
        if (16 * lane < ffn && wl < MW) {
#pragma unroll
            for (int l = 0; l < 4; ++l) *reinterpret_cast<u32x4 *>(&limbs[slot][wl][l][16 * (lane & 3)]) = pk[l];
            if ((lane & (4 * WG - 1)) == 0) gdown[slot][wl / WG] = ldexpf(1.0f, -sh);
        }
    }
    __syncthreads();
    floatx4 total = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < MW / WG; ++g) {
        int4v acc = (int4v){0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < WG; ++w) {
            const int wi = g * WG + w;
            int4v bfrag = (int4v){0, 0, 0, 0};
            if (c < 4 && wi < windows) bfrag = *reinterpret_cast<const int4v *>(&limbs[slot][wi][c][16 * q]);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(int4v, a[wi]), bfrag, acc, 0, 0, 0);
        }
        if (g < groups) {
            const floatx4 f = (floatx4){(float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]};
            total += f * (sc[g] * gdown[slot][g]);
        }
    }
    // limbs weighted 2^(8c) and summed over c, scaled by the slot's routing weight
    const float wt = on ? weights[(size_t)b * k + slot] : 0.0f;
    float r4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float x = c < 4 ? total[i] * (c == 0 ? 1.0f : c == 1 ? 256.0f : c == 2 ? 65536.0f : 16777216.0f) : 0.0f;
        x += __shfl_xor(x, 1);
        x += __shfl_xor(x, 2);
        r4[i] = x * wt;
    }
    if (c == 0) *reinterpret_cast<float4 *>(&red[slot][4 * q]) = make_float4(r4[0], r4[1], r4[2], r4[3]);
    __syncthreads();
    if (slot == 0 && lane < (half ? 8 : 16)) {
        float s = 0.0f;
        for (int j = 0; j < k; ++j) s += red[j][lane];
        out[(size_t)b * hidden + tile * 16 + 8 * hb + lane] += s;
    }
}

template <int WG, int MW, typename ST>
static void launch_down_t(marin_gpu *g, const marin_quant_matrix *down, const float *act, const int32_t *ids,
                          const float *weights, size_t tokens, size_t k, size_t hidden, size_t ffn, float *out) {
    // half tiles while whole tiles leave compute units idle (one token: hidden / 16 workgroups)
    const int half = (hidden / 16) * tokens < (size_t)std::max(g->cu_count, 1) ? 1 : 0;
    dim3 grid((unsigned)((hidden / 16) << half), (unsigned)tokens);
    expert_down<WG, MW, ST><<<grid, dim3(64 * MOE_MAX_K), 0, g->stream>>>(
        down->codes, (const ST *)down->scales, act, ids, weights, (int)k, (int)(down->rows / hidden), (int)hidden,
        (int)ffn, out, half);
}

template <typename ST>
static void launch_down_st(marin_gpu *g, const marin_quant_matrix *down, const float *act, const int32_t *ids,
                           const float *weights, size_t tokens, size_t k, size_t hidden, size_t ffn, float *out) {
    const size_t windows = ffn / 64;
    if (down->group == 128) {
        if (windows <= 12) launch_down_t<2, 12, ST>(g, down, act, ids, weights, tokens, k, hidden, ffn, out);
        else launch_down_t<2, 16, ST>(g, down, act, ids, weights, tokens, k, hidden, ffn, out);
    } else {
        if (windows <= 12) launch_down_t<1, 12, ST>(g, down, act, ids, weights, tokens, k, hidden, ffn, out);
        else launch_down_t<1, 16, ST>(g, down, act, ids, weights, tokens, k, hidden, ffn, out);
    }
}

struct MoeArgs {
    const marin_quant_matrix *gate_up, *down;
    const float *x, *norm;
    float eps;
    const int32_t *ids;
    const float *weights;
    size_t tokens, k, experts, hidden, ffn;
    float *act, *out;
};

static void check_moe(const MoeArgs &a) {
    if (a.k == 0 || a.k > (size_t)MOE_MAX_K) unsupported("experts per token", MOE_MAX_K, a.k);
    if (a.k > a.experts) shape("experts per token (at most the experts)", a.experts, a.k);
    if (a.gate_up->bits != 8 || a.down->bits != 8) unsupported("expert code width (int8)", 8, (size_t)a.gate_up->bits);
    if (a.gate_up->rows != a.experts * 2 * a.ffn || a.gate_up->cols != a.hidden)
        shape("expert gate_up rows (experts * 2 * ffn)", a.experts * 2 * a.ffn, a.gate_up->rows);
    if (a.down->rows != a.experts * a.hidden || a.down->cols != a.ffn)
        shape("expert down rows (experts * hidden)", a.experts * a.hidden, a.down->rows);
    if ((2 * a.ffn) % 16 || a.hidden % 16) shape("expert rows (multiples of 16)", 16, a.ffn);
    // expert_down builds the limbs with one lane per 16 columns: 64 lanes, 1024 columns
    if (a.ffn % 64 || a.ffn > 1024) unsupported("expert ffn (multiple of 64, at most 1024)", 1024, a.ffn);
    if (!gemv_decode_supported(a.gate_up) || !(a.down->group == 64 || a.down->group == 128) || !a.down->windowed)
        unsupported("expert quantization group (64 or 128)", 128, a.down->group);
}

// One or more tokens' MoE FFN: out[t] += sum_j w[t][j] down_{e}(silu(gate_e x) * up_e x), x = RMSNorm(x[t]) when a
// norm is given.
// Device scratch of a grouped batch: the gate_up's activation limbs, then the plan.
static size_t moe_scratch_bytes(const MoeArgs &a) {
    return (moe_gate_up_workspace(a.tokens, a.hidden, a.gate_up->group) + 255) / 256 * 256 + MOE_PLAN_WORDS * 4;
}

static bool moe_grouped(const MoeArgs &a) { return a.tokens >= 2 && a.tokens <= (size_t)MOE_BATCH; }

static void launch_moe(marin_gpu *g, const MoeArgs &a, int part = 0) {
    check_moe(a);
    if (moe_grouped(a) && part != 2) {
        // a decode batch: every distinct selected expert's gate_up rows read once for all tokens
        uint8_t *ws = (uint8_t *)g->workspace(moe_scratch_bytes(a));
        int32_t *plan = (int32_t *)(ws + moe_scratch_bytes(a) - MOE_PLAN_WORDS * 4);
        moe_plan<<<1, 64, 0, g->stream>>>(a.ids, (int)a.tokens, (int)a.k, (int)a.experts, plan);
        g->launched();
        GemvIn in;
        in.mode = a.norm ? IN_NORM : IN_F32;
        in.x = a.x;
        in.x_stride = a.hidden;
        in.norm = a.norm;
        in.eps = a.eps;
        launch_moe_gate_up(g, a.gate_up, in, a.tokens, plan, std::min(a.tokens * a.k, a.experts), a.k, a.ffn, a.act);
        const double rows = (double)std::min(a.tokens * a.k, a.experts) * 2 * a.ffn;  // at most, once each
        g->launched(marin_gpu::GEMV, rows * a.hidden + rows * (a.hidden / a.gate_up->group) * (a.gate_up->bf16_scales ? 2 : 4),
                    "gemm_q8 (experts)");
    }
    for (size_t t = 0; t < a.tokens && part != 2 && !moe_grouped(a); ++t) {
        GemvIn in;
        in.mode = a.norm ? IN_NORM : IN_F32;
        in.x = a.x + t * a.hidden;
        in.x_stride = a.hidden;
        in.norm = a.norm;
        in.eps = a.eps;
        in.tile_map = a.ids + t * a.k;
        in.map_tiles = (int)(2 * a.ffn / 16);
        in.map_count = (int)a.k;
        in.map_blocks = (int)a.experts;
        GemvOut o;
        o.mode = OUT_SILU;
        o.y = a.act + t * a.k * a.ffn;
        o.y_stride = a.k * a.ffn;
        launch_gemv(g, a.gate_up, in, o, 1);
    }
    if (part == 1) return;
    if (a.down->bf16_scales)
        launch_down_st<uint16_t>(g, a.down, a.act, a.ids, a.weights, a.tokens, a.k, a.hidden, a.ffn, a.out);
    else
        launch_down_st<float>(g, a.down, a.act, a.ids, a.weights, a.tokens, a.k, a.hidden, a.ffn, a.out);
    const double bytes = (double)a.tokens * a.k *
                         ((double)a.hidden * a.ffn * 2 + (double)a.hidden * a.ffn +
                          (double)(2 * a.ffn * a.hidden + a.hidden * a.ffn) / a.down->group * (a.down->bf16_scales ? 2 : 4));
    g->launched(marin_gpu::GEMV, bytes, "expert_down");
}

}  // namespace marin

using namespace marin;

static const float *f32_of(const marin_buffer *b, size_t len, const char *what) {
    if (!b) shape(what, len, 0);
    if (b->dtype != MARIN_F32) shape(what, 4, 2);
    if (b->len < len) shape(what, len, b->len);
    return (const float *)b->data;
}

extern "C" {

marin_status marin_moe_route(marin_gpu *g, const marin_buffer *logits, size_t tokens, size_t experts, size_t k,
                             int renorm, marin_buffer *ids, marin_buffer *weights) {
    return guard([&] {
        if (!tokens) return;
        if (experts == 0 || experts > 1024) unsupported("experts", 1024, experts);
        if (k == 0 || k > (size_t)MOE_MAX_K || k > experts) unsupported("experts per token", MOE_MAX_K, k);
        f32_of(logits, tokens * experts, "router logits");
        if (!ids || ids->dtype != MARIN_U32 || ids->len < tokens * k) shape("expert ids (u32)", tokens * k, ids ? ids->len : 0);
        f32_of(weights, tokens * k, "expert weights");
        moe_route<<<(unsigned)tokens, ROUTE_THREADS, 0, g->stream>>>((const float *)logits->data, (int)experts, (int)k,
                                                                     renorm, (int32_t *)ids->data, (float *)weights->data,
                                                                     g->fault);
        g->launched();
    });
}

marin_status marin_moe_ffn(marin_gpu *g, const marin_quant_matrix *gate_up, const marin_quant_matrix *down,
                           const marin_buffer *x, const marin_buffer *norm, float eps, const marin_buffer *ids,
                           const marin_buffer *weights, size_t tokens, size_t experts, size_t k, marin_buffer *act,
                           marin_buffer *out) {
    return guard([&] {
        if (!tokens) return;
        MoeArgs a{};
        a.gate_up = gate_up;
        a.down = down;
        a.hidden = gate_up->cols;
        a.ffn = down->cols;
        a.tokens = tokens;
        a.k = k;
        a.experts = experts;
        a.x = f32_of(x, tokens * a.hidden, "hidden states");
        a.norm = norm ? f32_of(norm, a.hidden, "norm weights") : nullptr;
        a.eps = eps;
        if (!ids || ids->dtype != MARIN_U32 || ids->len < tokens * k) shape("expert ids (u32)", tokens * k, ids ? ids->len : 0);
        a.ids = (const int32_t *)ids->data;
        a.weights = f32_of(weights, tokens * k, "expert weights");
        a.act = (float *)f32_of(act, tokens * k * a.ffn, "expert activations");
        a.out = (float *)f32_of(out, tokens * a.hidden, "output");
        launch_moe(g, a);
    });
}

marin_status marin_moe_stack_time(marin_gpu *g, size_t layers, const marin_quant_matrix *const *gate_ups,
                                  const marin_quant_matrix *const *downs, const marin_buffer *x,
                                  const marin_buffer *norm, float eps, const marin_buffer *ids,
                                  const marin_buffer *weights, size_t tokens, size_t experts, size_t k,
                                  marin_buffer *act, marin_buffer *out, int part, int reps, double *seconds) {
    return guard([&] {
        if (!layers || !tokens) shape("layers and tokens", 1, 0);
        if (reps < 1) shape("timing repetitions", 1, (size_t)reps);
        if (part < 0 || part > 2) shape("stack part (0 all, 1 gate_up, 2 down)", 2, (size_t)part);
        std::vector<MoeArgs> per(layers);
        for (size_t l = 0; l < layers; ++l) {
            MoeArgs &a = per[l];
            a.gate_up = gate_ups[l];
            a.down = downs[l];
            a.hidden = a.gate_up->cols;
            a.ffn = a.down->cols;
            a.tokens = tokens;
            a.k = k;
            a.experts = experts;
            a.x = f32_of(x, tokens * a.hidden, "hidden states");
            a.norm = norm ? f32_of(norm, a.hidden, "norm weights") : nullptr;
            a.eps = eps;
            if (!ids || ids->dtype != MARIN_U32 || ids->len < layers * tokens * k)
                shape("expert ids (u32, per layer)", layers * tokens * k, ids ? ids->len : 0);
            a.ids = (const int32_t *)ids->data + l * tokens * k;
            a.weights = f32_of(weights, layers * tokens * k, "expert weights (per layer)") + l * tokens * k;
            a.act = (float *)f32_of(act, tokens * k * a.ffn, "expert activations");
            a.out = (float *)f32_of(out, tokens * a.hidden, "output");
            check_moe(a);
        }
        // scratch grown before capture (a capture may not allocate)
        size_t scratch = 0;
        for (auto &a : per) scratch = std::max(scratch, moe_grouped(a) ? moe_scratch_bytes(a) : 0);
        if (scratch) g->workspace(scratch);
        const char *ng = getenv("MARIN_NO_GRAPH");
        if (ng && *ng && *ng != '0') {
            // eager launches (for tracers that do not follow graph replays)
            for (auto &a : per) launch_moe(g, a, part);
            hipEvent_t t0 = g->next_event(), t1 = g->next_event();
            HIP_CHECK(hipEventRecord(t0, g->stream));
            for (int r = 0; r < reps; ++r)
                for (auto &a : per) launch_moe(g, a, part);
            HIP_CHECK(hipEventRecord(t1, g->stream));
            HIP_CHECK(hipEventSynchronize(t1));
            float ms = 0.0f;
            HIP_CHECK(hipEventElapsedTime(&ms, t0, t1));
            *seconds = ms * 1e-3 / reps;
            return;
        }
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        HIP_CHECK(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal));
        try {
            for (auto &a : per) launch_moe(g, a, part);
        } catch (...) {
            hipGraph_t junk = nullptr;
            (void)hipStreamEndCapture(g->stream, &junk);
            if (junk) (void)hipGraphDestroy(junk);
            throw;
        }
        HIP_CHECK(hipStreamEndCapture(g->stream, &graph));
        hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        hip_check(e, "hipGraphInstantiate");
        hipEvent_t t0 = g->next_event(), t1 = g->next_event();
        float ms = 0.0f;
        e = hipGraphLaunch(exec, g->stream);
        if (e == hipSuccess) e = hipEventRecord(t0, g->stream);
        for (int r = 0; r < reps && e == hipSuccess; ++r) e = hipGraphLaunch(exec, g->stream);
        if (e == hipSuccess) e = hipEventRecord(t1, g->stream);
        if (e == hipSuccess) e = hipEventSynchronize(t1);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, t0, t1);
        (void)hipGraphExecDestroy(exec);
        hip_check(e, "timed expert graph");
        *seconds = ms * 1e-3 / reps;
    });
}

}  // extern "C"
