// The quantized product of a decode batch (2..8 tokens, int8 or int4 codes): the one-token product's schedule with
// the tokens' limbs read from L2.
//
// Same exact arithmetic as the other products: codes are the A operand of v_mfma_i32_16x16x64_i8, the activations
// are four signed 8-bit limbs per (token, group) (quantize_act), four tokens x four limbs fill the 16 B columns, so
// a batch of up to 8 tokens takes two MFMAs per 64-column window of codes. Sums are exact int32 per group, scaled
// once by weight scale x the token's 2^-s.
//
// Schedule (a batch must read the weights once and at the speed of the one-token product):
//  - a persistent grid over 16-row tiles, 8 waves per block; wave w owns the fixed column slice [w S, (w + 1) S)
//    windows of every row, so a tile's K is split over the waves and their sums meet in LDS once per tile;
//  - a ring of RING items (tile, window) per wave runs across tile ends: the code window (HBM) and the B fragments
//    of the window for each token tile (L2: every block reads the same few KiB of limbs) travel together;
//  - every load is unconditional (clamped), so the waits are exact and never drain the ring;
//  - the loop touches global memory only through the ring: a tile's finished rows go to an LDS buffer and are
//    written out (f32, residual add, SiLU(gate) * up, bf16, the greedy choice of every token) after the loop.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>
#include <type_traits>

#include "gemm.hpp"

namespace marin {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int BW = 8;      // waves per block
// items in flight per wave: 8 for one token tile; 4 for two, so two blocks stay resident per compute unit
constexpr int BATCH_RING2 = 4;
// 8-window slices keep the wave's B fragments (all its windows, every token tile) in registers for the whole launch,
// so only the codes stream; the registers leave one block per compute unit, and the ring is one slice deep
template <int SM>
constexpr bool bres() { return SM == 8; }
template <int TT, int SM>
constexpr int bring() { return bres<SM>() ? SM : (TT == 1 ? 8 : BATCH_RING2); }
template <int SM>
constexpr int batch_min_blocks() { return bres<SM>() ? 1 : 2; }
constexpr int BATCH_BLOCKS_PER_CU = 2;
constexpr int OBUF_TILES = 40;  // tiles a block holds outputs for (the grid covers the matrix in as many rounds)

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

__device__ __forceinline__ unsigned long long choice_key(float v, int row) {
    const int b = __float_as_int(v);
    const unsigned k = (unsigned)(b ^ (int)(((unsigned)(b >> 31)) >> 1)) ^ 0x80000000u;
    return (unsigned long long)k << 32 | (unsigned long long)(0xffffffffu - (unsigned)row);
}

}  // namespace

// BITS: 8 or 4 (nibbles stored as code + 8, unpacked to bytes; 8 x the group's limb sums come off the int32 sums);
// WG: windows per quantization group; TT: token tiles of 4 (1 or 2); SM: windows per wave per tile; ST: scale type.
// FUSE (int8, B fragments in registers): no separate limb pass; every wave builds the limbs of its own column slice
// from the activations (`in`) in its prologue, exactly as quantize_rows does: per (token, group) the power of two
// that puts the group's largest magnitude of x (x * norm weight with a norm) in [2^29, 2^30), four limbs of each
// value; the RMSNorm factor of each token comes from the waves' partial sums of squares and scales the outputs.
template <int BITS, int WG, int TT, int SM, typename ST, bool FUSE>
__global__ __launch_bounds__(64 * BW, batch_min_blocks<SM>()) void gemv_batch(const uint8_t *__restrict__ codes, const ST *__restrict__ scales,
                                                      const int8_t *__restrict__ limbs,
                                                      const float *__restrict__ exps, const float *__restrict__ rsv,
                                                      const int32_t *__restrict__ lsum, GemvIn in, GemvOut out,
                                                      int tokens, int rows, int cols, int tiles) {
    static_assert(!FUSE || (BITS == 8 && bres<SM>()), "fused limbs: int8 with B in registers");
    constexpr int CB = BITS == 8 ? 16 : 8;  // code bytes per lane per window
    constexpr int S = SM;
    constexpr int BRING = bring<TT, SM>();
    constexpr bool BRES = bres<SM>();
    __shared__ __align__(16) float red[2][BW][4 * TT][16];
    // the block's finished rows, written out after the main loop: a global store or load inside the loop would
    // sit in the vector memory counter with the ring and make the waits for it drain the ring
    __shared__ float obuf[OBUF_TILES][4 * TT][16];
    __shared__ unsigned long long best_s[4 * TT];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    const int windows = cols >> 6;
    const int groups = windows / WG;
    const size_t tile_bytes = (size_t)16 * (BITS == 8 ? cols : cols / 2);
    const int w0 = wave * S;
    const int my_tiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int items = my_tiles * S;
    if (threadIdx.x < 4 * TT) best_s[threadIdx.x] = 0ull;  // read after the tiles' barriers
    __shared__ float ssq_s[FUSE ? BW : 1][4 * TT];          // FUSE: the waves' partial sums of squares per token
    __shared__ __align__(16) uint32_t tr_s[FUSE ? BW : 1][64][4];  // FUSE: a wave's limb transpose

    // the epilogue's token factors, loaded before the ring: a load issued after it would wait for all of it
    float rsl[TT];
#pragma unroll
    for (int pass = 0; pass < TT; ++pass) rsl[pass] = FUSE ? 1.0f : rsv[min(4 * pass + lane / 16, tokens - 1)];

    // FUSE: lane (q, t, L) (lane = 16 q + 4 t + L) loads values 16 q + 4 L .. + 3 of window w of token 4 j + t, for
    // every window of the slice and token tile j; all loads unconditional (clamped) and issued before the ring
    constexpr int FS = FUSE ? SM : 1, FT = FUSE ? TT : 1;
    float fx[FS][FT][4], fw[FS][4];
    if constexpr (FUSE) {
        const bool bf = in.mode == IN_BF16, nrm = in.mode == IN_NORM;
        const int ft = (lane & 15) >> 2, fl = lane & 3;
#pragma unroll
        for (int wl = 0; wl < SM; ++wl) {
            const int col = 64 * min(wave * SM + wl, (cols >> 6) - 1) + 16 * q + 4 * fl;
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                const size_t at = (size_t)min(4 * j + ft, tokens - 1) * in.x_stride + col;
                if (bf) {
                    const uint2 u = *reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(in.x) + at);
                    fx[wl][j][0] = __uint_as_float(u.x << 16);
                    fx[wl][j][1] = __uint_as_float(u.x & 0xffff0000u);
                    fx[wl][j][2] = __uint_as_float(u.y << 16);
                    fx[wl][j][3] = __uint_as_float(u.y & 0xffff0000u);
                } else {
                    const float4 f = *reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(in.x) + at);
                    fx[wl][j][0] = f.x;
                    fx[wl][j][1] = f.y;
                    fx[wl][j][2] = f.z;
                    fx[wl][j][3] = f.w;
                }
            }
            const float4 nw = *reinterpret_cast<const float4 *>(nrm ? in.norm + col : reinterpret_cast<const float *>(in.x) + col);
            fw[wl][0] = nw.x;
            fw[wl][1] = nw.y;
            fw[wl][2] = nw.z;
            fw[wl][3] = nw.w;
        }
    }
    // the limbs are in B-fragment order ([window][token tile][lane][16 bytes]); this lane's token in token tile j is
    // 4 j + c / 4, and a lane of a token past the batch reads the batch's last token (its sums are never written)
    const int ttiles = (tokens + 3) / 4;
    const int8_t *brow[TT];
    const float *erow[TT];
    const int32_t *orow[TT];
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        const int tok = min(4 * j + c / 4, tokens - 1);
        const int ln = tok == 4 * j + c / 4 ? lane : 16 * q + 4 * (tok & 3) + (c & 3);
        brow[j] = limbs + ((size_t)(tok >> 2) * 64 + ln) * 16;
        erow[j] = exps + (size_t)tok * groups;
        orow[j] = BITS == 4 ? lsum + (size_t)tok * groups * 4 + (c & 3) : nullptr;
    }

    typedef typename std::conditional<BITS == 8, u32x4, u32x2>::type Raw;
    Raw ra[BRING];
    u32x4 rb[BRING][TT];
    // BRES: the wave's B fragments, window wl of the slice, token tile j; loaded before the ring, so the waits for
    // them come first in the counter and never drain it
    u32x4 bq[BRES ? S : 1][TT];
    if constexpr (BRES && !FUSE) {
#pragma unroll
        for (int wl = 0; wl < S; ++wl) {
            const int w = min(w0 + wl, windows - 1);
#pragma unroll
            for (int j = 0; j < TT; ++j) bq[wl][j] = *reinterpret_cast<const u32x4 *>(brow[j] + (size_t)w * ttiles * 1024);
        }
    }
    floatx4 rs_[BRING / WG];
    float re[BRING / WG][TT];
    int ro[BRING / WG][TT];
    auto load_at = [&](int t, int w, int slot) {  // window w (clamped to the row) of tile t into ring slot `slot`
        ra[slot] = __builtin_nontemporal_load(
            reinterpret_cast<const Raw *>(codes + (size_t)t * tile_bytes + (size_t)w * 64 * CB + CB * lane));
        if constexpr (!BRES) {
#pragma unroll
            for (int j = 0; j < TT; ++j) rb[slot][j] = *reinterpret_cast<const u32x4 *>(brow[j] + (size_t)w * ttiles * 1024);
        }
        if (slot % WG == WG - 1) {  // the group's factors travel with its last window, read at the group's end
            const ST *sp = scales + ((size_t)t * groups + w / WG) * 16 + 4 * q;
            if constexpr (sizeof(ST) == 4) {
                rs_[slot / WG] = *reinterpret_cast<const floatx4 *>(sp);
            } else {
                const uint2 sv = *reinterpret_cast<const uint2 *>(sp);
                rs_[slot / WG] = (floatx4){__uint_as_float(sv.x << 16), __uint_as_float(sv.x & 0xffff0000u),
                                           __uint_as_float(sv.y << 16), __uint_as_float(sv.y & 0xffff0000u)};
            }
            if constexpr (!FUSE) {
#pragma unroll
                for (int j = 0; j < TT; ++j) re[slot / WG][j] = erow[j][w / WG];
            }
            if constexpr (BITS == 4) {
#pragma unroll
                for (int j = 0; j < TT; ++j) ro[slot / WG][j] = 8 * orow[j][(w / WG) * 4];
            }
        }
    };
    auto load_item = [&](int i, int slot) {
        load_at((int)blockIdx.x + (i / S) * (int)gridDim.x, min(w0 + i % S, windows - 1), slot);
    };
    // Slices a whole number of ring rounds long (ALIGNED): a round's refills are windows of one tile, worked out once
    // per round; past the last item every refill loads this round's last window again.
    constexpr bool ALIGNED = S % BRING == 0;
    const int last = items > 0 ? items - 1 : 0;
#pragma unroll
    for (int j = 0; j < BRING; ++j) load_item(min(j, last), j);

    // FUSE: the slice's limbs (B fragments), group factors and the RMSNorm partial sums, while the ring is in flight
    float egrp[FUSE ? SM / WG : 1][FT];
    if constexpr (FUSE) {
        const bool nrm = in.mode == IN_NORM;
        const int ft = (lane & 15) >> 2, fl = lane & 3;
        const int windows_ = cols >> 6;
#pragma unroll
        for (int j = 0; j < TT; ++j) {
            float ss = 0.0f;
#pragma unroll
            for (int gl = 0; gl < SM / WG; ++gl) {
                float v[WG][4];
                float mx = 0.0f;
#pragma unroll
                for (int ww = 0; ww < WG; ++ww) {
                    const int wl = gl * WG + ww;
                    const bool inrow = wave * SM + wl < windows_;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float x = inrow ? fx[wl][j][e] : 0.0f;
                        ss += x * x;
                        v[ww][e] = nrm ? x * fw[wl][e] : x;
                        mx = fmaxf(mx, fabsf(v[ww][e]));
                    }
                }
                // the group's largest magnitude: the 16 lanes of token t (L and q vary)
                mx = fmaxf(mx, __shfl_xor(mx, 1));
                mx = fmaxf(mx, __shfl_xor(mx, 2));
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                int sh = 0;
                if (mx > 0.0f && mx < INFINITY) {
                    int e;
                    (void)frexpf(mx, &e);
                    sh = 30 - e;
                    sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
                }
                const float up = ldexpf(1.0f, sh);
                egrp[gl][j] = ldexpf(1.0f, -sh);
#pragma unroll
                for (int ww = 0; ww < WG; ++ww) {
                    const int wl = gl * WG + ww;
                    uint32_t wd[4];
                    limbs4(__float2int_rn(v[ww][0] * up), __float2int_rn(v[ww][1] * up), __float2int_rn(v[ww][2] * up),
                           __float2int_rn(v[ww][3] * up), wd);
                    // quad transpose through LDS: lane L of the quad takes limb L of the quad's 16 values, in
                    // column order (lane b + k holds values 4 k .. 4 k + 3)
#pragma unroll
                    for (int m = 0; m < 4; ++m) tr_s[wave][(lane & ~3) + m][fl] = wd[m];
                    __builtin_amdgcn_wave_barrier();
                    bq[wl][j] = *reinterpret_cast<const u32x4 *>(&tr_s[wave][lane][0]);
                    __builtin_amdgcn_wave_barrier();
                }
            }
            // the wave's sum of squares of token 4 j + t: its 16 lanes
            ss += __shfl_xor(ss, 1);
            ss += __shfl_xor(ss, 2);
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if ((lane & 0x33) == 0) ssq_s[wave][4 * j + ft] = ss;
        }
    }

    floatx4 total[TT];
    int4v acc[TT];
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        total[j] = (floatx4){0.f, 0.f, 0.f, 0.f};
        acc[j] = (int4v){0, 0, 0, 0};
    }
    int tile_n = 0;
    const float lw = (c & 3) == 0 ? 1.0f : (c & 3) == 1 ? 256.0f : (c & 3) == 2 ? 65536.0f : 16777216.0f;
    for (int base = 0; base < items; base += BRING) {
        int nt = 0, nw = 0, ns = 1;
        if constexpr (ALIGNED) {
            const bool past = base + BRING > last;
            const int nb = past ? base : base + BRING;
            nt = (int)blockIdx.x + (nb / S) * (int)gridDim.x;
            nw = w0 + nb % S + (past ? BRING - 1 : 0);
            ns = past ? 0 : 1;
        }
#pragma unroll
        for (int s = 0; s < BRING; ++s) {
            const int i = base + s;
            int4v a;
            if constexpr (BITS == 8) {
                a = __builtin_bit_cast(int4v, ra[s]);
            } else {
                const Raw cur = ra[s];
                a = (int4v){(int)(cur.x & 0x0f0f0f0fu), (int)((cur.x >> 4) & 0x0f0f0f0fu), (int)(cur.y & 0x0f0f0f0fu),
                            (int)((cur.y >> 4) & 0x0f0f0f0fu)};
            }
            int4v b[TT];
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                if constexpr (BRES) b[j] = __builtin_bit_cast(int4v, bq[s][j]);  // a round is the whole slice
                else b[j] = __builtin_bit_cast(int4v, rb[s][j]);
            }
            // items past the block's last one (the ring's tail) contribute zeros and end no tile; with ALIGNED slices
            // items is a multiple of the ring, so there are none
            const bool valid = ALIGNED || i < items;
            const int wl = ALIGNED ? base % S + s : i % S;
            const int w = w0 + wl;
            const bool on = valid && w < windows;
#pragma unroll
            for (int j = 0; j < TT; ++j) acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, on ? b[j] : (int4v){0, 0, 0, 0}, acc[j], 0, 0, 0);
            if (s % WG == WG - 1) {
                // end of a group: one conversion, scaled by weight scale x the token's 2^-s
                const floatx4 gsc = rs_[s / WG];
#pragma unroll
                for (int j = 0; j < TT; ++j) {
                    float gex;
                    if constexpr (FUSE) gex = egrp[s / WG][j];  // a round is the whole slice: s is the window in it
                    else gex = re[s / WG][j];
                    if constexpr (BITS == 4) {
                        const int off = ro[s / WG][j];
                        acc[j] -= (int4v){off, off, off, off};
                    }
                    if (on) {
                        const floatx4 f = (floatx4){(float)acc[j][0], (float)acc[j][1], (float)acc[j][2], (float)acc[j][3]};
                        total[j] += f * (gsc * gex);
                    }
                    acc[j] = (int4v){0, 0, 0, 0};
                }
            }
            if (valid && wl == S - 1) {
                // ---- end of a tile: limbs weighted 2^(8 l) and summed over a token's four lanes, then over the waves
                float *rb_ = &red[tile_n & 1][0][0][0];
#pragma unroll
                for (int j = 0; j < TT; ++j) {
                    float r4[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        float v = total[j][k] * lw;
                        v += __shfl_xor(v, 1);
                        v += __shfl_xor(v, 2);
                        r4[k] = v;
                    }
                    if ((c & 3) == 0)
                        *reinterpret_cast<float4 *>(rb_ + ((wave * 4 * TT) + 4 * j + c / 4) * 16 + 4 * q) =
                            make_float4(r4[0], r4[1], r4[2], r4[3]);
                    total[j] = (floatx4){0.f, 0.f, 0.f, 0.f};
                }
                __syncthreads();
                if (wave == 0) {
                    // lane = (token tt, row r): 4 TT tokens x 16 rows over the wave's 64 lanes (a second pass for
                    // TT = 2); the tile's sums times the token's norm factor into the output buffer
#pragma unroll
                    for (int pass = 0; pass < TT; ++pass) {
                        const int tt = 4 * pass + lane / 16, r = lane % 16;
                        float v = 0.0f;
#pragma unroll
                        for (int ww = 0; ww < BW; ++ww) v += rb_[(ww * 4 * TT + tt) * 16 + r];
                        obuf[tile_n][tt][r] = v * rsl[pass];
                    }
                }
                ++tile_n;
            }
            // the slot is refilled once everything in it is consumed, so its registers carry straight over to the
            // next round
            if constexpr (ALIGNED) load_at(nt, min(nw + ns * s, windows - 1), s);
            else load_item(min(i + BRING, last), s);
        }
    }
    __syncthreads();
    // ---- outputs: thread per (tile, token, row pair)
    const int pairs = my_tiles * 4 * TT * 8;
    for (int p = (int)threadIdx.x; p < pairs; p += 64 * BW) {
        const int tn = p / (4 * TT * 8), tt = (p / 8) % (4 * TT), r = 2 * (p % 8);
        const int row = ((int)blockIdx.x + tn * (int)gridDim.x) * 16 + r;
        if (tt >= tokens) continue;
        float v0 = obuf[tn][tt][r], v1 = obuf[tn][tt][r + 1];
        if constexpr (FUSE) {
            if (in.mode == IN_NORM) {
                float ssum = 0.0f;
#pragma unroll
                for (int ww = 0; ww < BW; ++ww) ssum += ssq_s[ww][tt];
                const float rs = 1.0f / sqrtf(ssum / (float)cols + in.eps);
                v0 *= rs;
                v1 *= rs;
            }
        }
        if (out.mode == OUT_SILU) {
            if (row < rows) reinterpret_cast<float *>(out.y)[(size_t)tt * out.y_stride + (row >> 1)] = silu_f(v0) * v1;
            continue;
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float v = k ? v1 : v0;
            if (row + k >= rows) continue;
            const size_t at = (size_t)tt * out.y_stride + row + k;
            if (out.mode == OUT_F32) reinterpret_cast<float *>(out.y)[at] = v;
            else if (out.mode == OUT_ADD) reinterpret_cast<float *>(out.y)[at] += v;
            else {
                const unsigned uu = __float_as_uint(v);
                reinterpret_cast<uint16_t *>(out.y)[at] = (uint16_t)(
                    (uu & 0x7fffffffu) > 0x7f800000u ? (uu >> 16) | 0x40u : (uu + 0x7fffu + ((uu >> 16) & 1u)) >> 16);
            }
        }
        if (out.argmax_each) {
            unsigned long long key = row < rows ? choice_key(v0, row) : 0ull;
            if (row + 1 < rows) {
                const unsigned long long k1 = choice_key(v1, row + 1);
                key = k1 > key ? k1 : key;
            }
            if (key) atomicMax(&best_s[tt], key);
        }
    }
    if (out.argmax_each) {
        __syncthreads();
        if ((int)threadIdx.x < 4 * TT && (int)threadIdx.x < tokens && best_s[threadIdx.x])
            atomicMax(out.argmax + threadIdx.x, best_s[threadIdx.x]);
    }
}

// Windows per wave per tile: the smallest instantiated width whose BW slices cover the row, 0 when none does.
static int batch_slice(int windows) {
    for (int sm : {4, 8, 12, 24})
        if (BW * sm >= windows) return sm;
    return 0;
}

bool gemv_batch_supported(const marin_quant_matrix *w, size_t tokens) {
    return tokens >= 2 && tokens <= 8 && (w->bits == 8 || w->bits == 4) && w->windowed &&
           (w->group == 64 || w->group == 128) && w->cols % w->group == 0 && batch_slice((int)(w->cols / 64)) > 0;
}

template <int BITS, int WG, int TT, int SM, typename ST>
static void launch_t(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    const int tiles = (int)(w->rows_padded / 16);
    constexpr bool FUSE = BITS == 8 && bres<SM>();
    const ActLimbs al = FUSE ? ActLimbs{nullptr, nullptr, nullptr, nullptr}
                             : launch_quantize_act(g, in, tokens, w->cols, w->group, true);
    auto kern = gemv_batch<BITS, WG, TT, SM, ST, FUSE>;
    int resident = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, kern, 64 * BW, 0) != hipSuccess || resident < 1)
        resident = 1;
    const int blocks = std::max(std::min(tiles, std::min(resident, BATCH_BLOCKS_PER_CU) * std::max(g->cu_count, 1)),
                                (tiles + OBUF_TILES - 1) / OBUF_TILES);
    kern<<<dim3((unsigned)blocks), dim3(64 * BW), 0, g->stream>>>(w->codes, (const ST *)w->scales, al.limbs, al.exps,
                                                                   al.rs, al.lsum, in, out, (int)tokens, (int)w->rows,
                                                                   (int)w->cols, tiles);
}

template <int BITS, int WG, int TT, typename ST>
static void launch_sm(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    switch (batch_slice((int)(w->cols / 64))) {
        case 4: launch_t<BITS, WG, TT, 4, ST>(g, w, in, out, tokens); break;
        case 8: launch_t<BITS, WG, TT, 8, ST>(g, w, in, out, tokens); break;
        case 12: launch_t<BITS, WG, TT, 12, ST>(g, w, in, out, tokens); break;
        default: launch_t<BITS, WG, TT, 24, ST>(g, w, in, out, tokens); break;
    }
}

template <int BITS, typename ST>
static void launch_bits(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out,
                        size_t tokens) {
    const bool wg2 = w->group == 128;
    if (tokens <= 4) {
        if (wg2) launch_sm<BITS, 2, 1, ST>(g, w, in, out, tokens);
        else launch_sm<BITS, 1, 1, ST>(g, w, in, out, tokens);
    } else {
        if (wg2) launch_sm<BITS, 2, 2, ST>(g, w, in, out, tokens);
        else launch_sm<BITS, 1, 2, ST>(g, w, in, out, tokens);
    }
}

template <typename ST>
static void launch_st(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    if (w->bits == 8) launch_bits<8, ST>(g, w, in, out, tokens);
    else launch_bits<4, ST>(g, w, in, out, tokens);
}

void launch_gemv_batch(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out, size_t tokens) {
    if (!gemv_batch_supported(w, tokens)) unsupported("batch product (2..8 tokens, int8 or int4, group 64 or 128)", 8, tokens);
    if (out.argmax && !out.argmax_each) unsupported("batch product greedy choice (one per token only)", 1, 0);
    if (w->bf16_scales) launch_st<uint16_t>(g, w, in, out, tokens);
    else launch_st<float>(g, w, in, out, tokens);
    const double act = in.mode == IN_BF16 ? 2.0 : 4.0, res = out.mode == OUT_BF16 ? 2.0 : 4.0;
    const double outs = out.mode == OUT_SILU ? (double)w->rows / 2 : (double)w->rows;
    const double bytes = (double)w->rows * w->row_bytes() + (double)w->rows * w->groups() * (w->bf16_scales ? 2 : 4) +
                         (double)tokens * w->cols * act + (double)tokens * outs * res;
    g->launched(marin_gpu::GEMV, bytes, "gemv_batch");
}

}  // namespace marin
