// The one-token quantized product (decode), built for latency on CDNA4.
//
// Same arithmetic as the multi-token matrix-core product (codes are the A operand of v_mfma_i32_16x16x64_i8,
// activations become exact signed 8-bit limbs in the B columns, int32 sums per group scaled once per group), with a
// schedule cut down to what one token needs:
//  - the block builds the limbs of the whole row once, into LDS (each column loaded once per block); every wave owns
//    a fixed slice of the columns (whole groups) for the whole launch and reuses its limbs for every 16-row tile;
//  - the power of two that scales the activations into 30-bit integers is chosen per group of columns (from the
//    group's largest magnitude), not per row, so no block-wide maximum is needed; it is folded into the group's
//    weight scale;
//  - a register ring of code windows runs across tile ends, so the next tile's codes are in flight while a tile's
//    sums are reduced; the reduction is one LDS exchange and one barrier per tile (double-buffered);
//  - the launch is persistent: blocks take tiles b, b + grid, ... with a grid sized to what stays resident.
// The prologue (activation loads, RMSNorm statistic, limbs) runs while the first windows of codes are in flight.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <algorithm>
#include <cmath>
#include <string>

#include "gemv.hpp"

namespace marin {

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int RING = 8;                  // code windows in flight per wave
constexpr int DECODE_BLOCKS_PER_CU = 2;  // resident blocks the persistent grid aims at per compute unit
constexpr int MAP_MAX = 64;              // tile map entries (selected experts) a launch may carry: one per lane

// Lane permutations inside rows of 16 lanes (DPP): 0xB1 swaps neighbours, 0x4E swaps pairs, 0x141 mirrors each
// half row of 8 lanes.
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

__device__ __forceinline__ int total_key(float v) {
    const int b = __float_as_int(v);
    return b ^ (int)(((unsigned)(b >> 31)) >> 1);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }

template <typename ST>
__device__ __forceinline__ floatx4 scales4(const ST *p) {
    if constexpr (sizeof(ST) == 4) {
        return *reinterpret_cast<const floatx4 *>(p);
    } else {
        const uint2 s = *reinterpret_cast<const uint2 *>(p);
        return (floatx4){__uint_as_float(s.x << 16), __uint_as_float(s.x & 0xffff0000u), __uint_as_float(s.y << 16),
                         __uint_as_float(s.y & 0xffff0000u)};
    }
}

}  // namespace


// BITS 8 or 4; WG = 64-column windows per quantization group (group = 64 * WG); SM = windows per wave per tile
// (wave w owns windows [w * SM, (w + 1) * SM) of every row; waves past the last window hold no groups); ST = scale
// type (float or bf16 bits); DW = waves per block (4 for rows of at most 32 windows, where 8 waves would get only a
// few windows of each tile, else 8).
//
// Every global load is unconditional (out-of-range addresses are clamped), and the activation loads are issued
// before the code ring: the memory counter the wave waits on then lets the activations arrive without draining the
// ring, and the ring stays exactly RING windows deep through the main loop.
template <int BITS, int WG, int SM, typename ST, int DW>
__global__ __launch_bounds__(64 * DW) void gemv_decode(const uint8_t *__restrict__ codes, const ST *__restrict__ scales,
                                                       GemvIn in, GemvOut out, int rows, int cols, int tiles,
                                                       int half) {
    extern __shared__ __align__(16) unsigned char lds[];
    constexpr int S = SM;
    constexpr int CB = BITS == 8 ? 16 : 8;  // code bytes per lane per window
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = lane & 15, q = lane >> 4;
    const int windows = cols >> 6;
    const int groups = windows / WG;
    const size_t tile_bytes = (size_t)16 * (BITS == 8 ? cols : cols / 2);

    // LDS: limbs [DW][S][4][64] bytes | down-scale per group [groups] f32 | int4 offsets [groups][4] i32 |
    //      wave sums [2][DW][16] f32 | sum of squares [DW] f32
    int8_t *limbs = reinterpret_cast<int8_t *>(lds);
    float *gdown = reinterpret_cast<float *>(lds + (size_t)DW * S * 256);
    const int gpad = (groups + 3) & ~3;  // keeps the wave sums 16-byte aligned
    int *goff = reinterpret_cast<int *>(gdown + gpad);
    float *red = reinterpret_cast<float *>(goff + (BITS == 4 ? gpad * 4 : 0));
    float *ssq = red + 2 * DW * 16;

    const int w0 = wave * S;  // first window of this wave's slice
    const int my_tiles = (tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    const int items = my_tiles * S;

    // A tile map (at most MAP_MAX entries) is loaded first, one entry per lane, and each item picks its entry with
    // a wave-uniform lane read: a per-item load of the map would sit behind the code windows already in flight and
    // wait for all of them.
    // Without a map the activation row stands in: the ring's first addresses then wait for that one load, which
    // measured faster than issuing the ring at once (the activations it races with feed the prologue).
    const int *map_p = in.tile_map ? in.tile_map : reinterpret_cast<const int *>(in.x);
    const int map_v = min(max(map_p[min(lane, max(in.map_count, 1) - 1)], 0), max(in.map_blocks, 1) - 1);

    // ---- the activations, block-wide: in round r, thread T holds the 16 consecutive columns RC r + 16 T .. + 16
    // (RC = 1024 DW columns per round), i.e. quarter T % 4 of window 16 DW r + T / 4: exactly what the B operand of
    // that window needs, so the thread builds all four limbs of its columns and stores each as 16 bytes; every wave
    // then reads the limbs of its own
    // windows. Each column is loaded once per block; threads past the row's end all load the row's last 16 columns
    // (one cache line per wave). Four 16-byte loads per round (bf16 rows use the first two) and the norm weights
    // (the activation address stands in when there is no norm), all unconditional and issued before the code ring:
    // with no branch around them the waits for them are exact and never drain the ring.
    constexpr int RC = 1024 * DW;     // columns per round
    constexpr int R = (S + 15) / 16;  // rounds: DW * S windows at most, 16 DW per round
    const bool norm = in.mode == IN_NORM, bf = in.mode == IN_BF16;
    const unsigned char *xb = reinterpret_cast<const unsigned char *>(in.x);
    u32x4 xr[R][4], nr[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int cb = min(r * RC + 16 * (int)threadIdx.x, cols - 16);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const size_t xo = bf ? (size_t)cb * 2 + 16 * (v & 1) : (size_t)cb * 4 + 16 * v;
            xr[r][v] = *reinterpret_cast<const u32x4 *>(xb + xo);
            nr[r][v] = *reinterpret_cast<const u32x4 *>(norm ? reinterpret_cast<const unsigned char *>(in.norm + cb) + 16 * v
                                                              : xb + xo);
        }
    }

    // ---- the ring: item i = (tile blockIdx + (i / S) * grid, window w0 + i % S)
    typedef typename std::conditional<BITS == 8, u32x4, u32x2>::type Raw;
    Raw ring[RING];
    floatx4 sring[RING / WG];
    // Half tiles (half = 1): logical tile tl is rows 8 (tl % 2) .. + 7 of tile tl / 2 over all its columns; the lanes
    // of the other 8 rows load their partner's row (the same cache lines), so the MFMA's rows 8..15 repeat rows 0..7
    // and are dropped at the end. A tile code is (tile of the matrix << half) | half-tile bit.
    auto tile_of = [&](int tl) {  // logical tile -> tile code
        const int pl = tl >> half;
        const int t = in.tile_map ? __builtin_amdgcn_readlane(map_v, pl / in.map_tiles) * in.map_tiles + pl % in.map_tiles
                                  : pl;
        return (t << half) | (tl & half);
    };
    auto load_at = [&](int tc, int w, int slot) {  // window w (clamped to the row) of tile code tc into ring slot `slot`
        const int t = tc >> half, hb = tc & half;
        const int la = half ? (c & 7) + 8 * hb + 16 * q : lane;  // the lane whose 16 bytes this lane loads
        const int qs = half ? (q & 1) + 2 * hb : q;               // the rows 4 qs .. + 3 whose scales it takes
        const unsigned uw = (unsigned)w;  // windows are never negative: unsigned index arithmetic needs no sign fixups
        const uint8_t *p = codes + (size_t)(unsigned)t * tile_bytes + (size_t)uw * (64 * CB) + CB * la;
        if constexpr (BITS == 8) ring[slot] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
        else ring[slot] = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p));
        if (slot % WG == 0) sring[slot / WG] = scales4(scales + ((size_t)(unsigned)t * groups + uw / WG) * 16 + 4 * qs);
    };
    auto load_item = [&](int i, int slot) {
        load_at(tile_of((int)blockIdx.x + (i / S) * (int)gridDim.x), min(w0 + i % S, windows - 1), slot);
    };
    // The refills' tiles (with their map lookups) are worked out once per ring round, not per window. Slices a whole
    // number of rounds long (ALIGNED): a round's items are windows bw .. bw + RING - 1 of one tile. Otherwise a round's
    // items run over at most NQ consecutive tiles, each item's tile picked with compile-time bounds.
    constexpr bool ALIGNED = S % RING == 0;
    constexpr int NQ = (S + RING - 1) / S + 1;
    static_assert(NQ <= 3, "a ring round spans at most three tiles");
    const int last = items > 0 ? items - 1 : 0;
#pragma unroll
    for (int j = 0; j < RING; ++j) load_item(min(j, last), j);
    const int t_last = tile_of((int)blockIdx.x + (last / S) * (int)gridDim.x);  // refills past the last item
    const int w_last = min(w0 + last % S, windows - 1);

    // ---- prologue: the limbs (and the RMSNorm partial sums: the threads' columns cover the row once)
    float xv[R][16];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            if (bf) {
                const uint32_t wd = xr[r][e / 8][(e / 2) % 4];
                xv[r][e] = __uint_as_float((e & 1) ? (wd & 0xffff0000u) : (wd << 16));
            } else {
                xv[r][e] = __uint_as_float(xr[r][e / 4][e % 4]);
            }
        }
    }
    auto in_row = [&](int r) {  // this thread's columns lie in the row
        return r * RC + 16 * (int)threadIdx.x < cols;
    };
    // the RMSNorm statistic: the waves' partial sums meet at the prologue's barrier; the limbs hold x * weight, and
    // the factor 1 / sqrt(mean(x^2) + eps) multiplies each row's sum at the end, so no barrier waits for it here
    if (norm) {
        float ss = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (in_row(r))
#pragma unroll
                for (int e = 0; e < 16; ++e) ss += xv[r][e] * xv[r][e];
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
        if (lane == 0) ssq[wave] = ss;
    }
    // windows past the row's end (up to the slices' DW * S) get zero limbs, so the main loop reads every window's
    // limbs unconditionally and those windows add nothing
    const u32x4 zero4 = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int wr = r * 16 * DW + (int)threadIdx.x / 4;  // window of this thread's columns
        if (r * RC + wave * 1024 >= cols) {  // wave-uniform: nothing loaded
            if (wr < DW * S) {
#pragma unroll
                for (int l = 0; l < 4; ++l) *reinterpret_cast<u32x4 *>(limbs + ((size_t)wr * 4 + l) * 64 + 16 * (lane & 3)) = zero4;
            }
            continue;
        }
        const bool valid = in_row(r);
        float v[16];
        float mx = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            float x = xv[r][e];
            if (norm) x = x * __uint_as_float(nr[r][e / 4][e % 4]);
            v[e] = x;
            mx = fmaxf(mx, fabsf(x));
        }
        // the group's largest magnitude: its 4 WG lanes are consecutive
        mx = fmaxf(mx, dpp_f<0xB1>(mx));  // lanes xor 1
        mx = fmaxf(mx, dpp_f<0x4E>(mx));  // lanes xor 2
        if constexpr (WG == 2) mx = fmaxf(mx, dpp_f<0x141>(mx));  // the other quad of the 8 lanes
        int sh = 0;
        if (mx > 0.0f && mx < INFINITY) {
            int e;
            (void)frexpf(mx, &e);
            sh = 30 - e;  // largest magnitude lands in [2^29, 2^30)
            sh = sh > 126 ? 126 : (sh < -126 ? -126 : sh);
        }
        const float up = ldexpf(1.0f, sh);
        u32x4 pk[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t w[4];
            limbs4(__float2int_rn(v[4 * j] * up), __float2int_rn(v[4 * j + 1] * up), __float2int_rn(v[4 * j + 2] * up),
                   __float2int_rn(v[4 * j + 3] * up), w);
#pragma unroll
            for (int l = 0; l < 4; ++l) pk[l][j] = w[l];
        }
        if (wr < DW * S) {
#pragma unroll
            for (int l = 0; l < 4; ++l)
                *reinterpret_cast<u32x4 *>(limbs + ((size_t)wr * 4 + l) * 64 + 16 * (lane & 3)) = valid ? pk[l] : zero4;
        }
        const int g = wr / WG;
        if (valid && (lane & (4 * WG - 1)) == 0) gdown[g] = ldexpf(1.0f, -sh);
        if constexpr (BITS == 4) {
            // stored nibbles are code + 8: the group's sum of each limb column, times 8, comes off the sums
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                int sm = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) sm = __builtin_amdgcn_sdot4((int)pk[l][j], 0x01010101, sm, false);
                sm += dpp_i<0xB1>(sm);
                sm += dpp_i<0x4E>(sm);
                if constexpr (WG == 2) sm += dpp_i<0x141>(sm);
                if (valid && (lane & (4 * WG - 1)) == 0) goff[g * 4 + l] = 8 * sm;
            }
        }
    }
    __syncthreads();
    float rs = 1.0f;
    if (norm) {
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < DW; ++w) total += ssq[w];
        rs = 1.0f / sqrtf(total / (float)cols + in.eps);
    }

    // slices one ring round long keep their B fragments in registers for the launch
    constexpr bool BRES = S == RING;
    int4v bq[BRES ? S : 1];
    if constexpr (BRES) {
#pragma unroll
        for (int wl = 0; wl < S; ++wl) bq[wl] = *reinterpret_cast<const int4v *>(limbs + ((size_t)(wave * S + wl) * 4 + (c & 3)) * 64 + 16 * q);
    }
    floatx4 total = (floatx4){0.f, 0.f, 0.f, 0.f};
    floatx4 gsc = total;
    int4v acc = (int4v){0, 0, 0, 0};
    unsigned long long best = 0ull;
    int tile_n = 0;
    for (int base = 0; base < items; base += RING) {
        // ALIGNED: the next round's tile and first window; past the last item every refill loads this round's last
        // window again (one cache line per lane group, so the refills stay unconditional without re-reading the
        // round). items is a multiple of RING, so every item of a round is real.
        int nt = 0, nw = 0, ns = 1;
        if constexpr (ALIGNED) {
            const bool past = base + RING > last;
            const int nb = past ? base : base + RING;
            nt = tile_of((int)blockIdx.x + (nb / S) * (int)gridDim.x);
            nw = w0 + nb % S + (past ? RING - 1 : 0);
            ns = past ? 0 : 1;
        }
        const int bw = ALIGNED ? base % S : 0;
        int q0 = 0, r0 = 0, tq[3] = {0, 0, 0};
        if constexpr (!ALIGNED) {
            const int nb = base + RING;
            q0 = nb / S;
            r0 = nb % S;
#pragma unroll
            for (int d = 0; d < NQ; ++d) tq[d] = tile_of((int)blockIdx.x + (q0 + d) * (int)gridDim.x);
        }
#pragma unroll
        for (int j = 0; j < RING; ++j) {
            const int i = base + j;
            const Raw cur = ring[j];
            if (j % WG == 0) gsc = sring[j / WG];  // the slot is refilled below, before the group's last window
            if constexpr (ALIGNED) {
                load_at(nt, min(nw + ns * j, windows - 1), j);
            } else {
                const int off = r0 + j;  // window of the refill counted from tile q0's first
                const int d = off >= 2 * S ? 2 : (off >= S ? 1 : 0);
                const bool past = i + RING > last;
                load_at(past ? t_last : (d == 0 ? tq[0] : d == 1 ? tq[1] : tq[2]),
                        past ? w_last : min(w0 + off - d * S, windows - 1), j);
                if (i >= items) continue;
            }
            const int wl = ALIGNED ? bw + j : i % S;  // window inside the slice
            const int w = w0 + wl;     // window of the row
            // lanes c >= 4 (B columns 4..15, whose sums are never used) read the limbs of lane c % 4
            int4v b;
            if constexpr (BRES) b = bq[j];  // a round is the whole slice
            else b = *reinterpret_cast<const int4v *>(limbs + ((size_t)(wave * S + wl) * 4 + (c & 3)) * 64 + 16 * q);
            int4v a;
            if constexpr (BITS == 8) {
                a = __builtin_bit_cast(int4v, cur);
            } else {
                a = (int4v){(int)(cur.x & 0x0f0f0f0fu), (int)((cur.x >> 4) & 0x0f0f0f0fu), (int)(cur.y & 0x0f0f0f0fu),
                            (int)((cur.y >> 4) & 0x0f0f0f0fu)};
            }
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc, 0, 0, 0);
            if (j % WG == WG - 1) {
                // end of a group: one conversion, scaled by weight scale x 2^-shift of the group
                // past the row's end the sums are zero and any finite factor will do
                const int g = min(w / WG, groups - 1);
                if constexpr (BITS == 4) {
                    const int off = c < 4 && w < windows ? goff[g * 4 + c] : 0;
                    acc -= (int4v){off, off, off, off};
                }
                const float d = gdown[g];
                const floatx4 f = (floatx4){(float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]};
                total += f * (gsc * d);
                acc = (int4v){0, 0, 0, 0};
            }
            if (wl == S - 1) {
                // ---- end of a tile: limbs weighted 2^(8c) and summed over c, then over the waves
                float r4[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float v = c < 4 ? total[k] * (c == 0 ? 1.0f : c == 1 ? 256.0f : c == 2 ? 65536.0f : 16777216.0f)
                                    : 0.0f;
                    v += __shfl_xor(v, 1);
                    v += __shfl_xor(v, 2);
                    r4[k] = v;
                }
                float *rb = red + (tile_n & 1) * DW * 16;
                if (c == 0) *reinterpret_cast<float4 *>(rb + wave * 16 + 4 * q) = make_float4(r4[0], r4[1], r4[2], r4[3]);
                total = (floatx4){0.f, 0.f, 0.f, 0.f};
                __syncthreads();
                if (wave == 0 && lane < 16) {
                    float v = 0.0f;
#pragma unroll
                    for (int ww = 0; ww < DW; ++ww) v += rb[ww * 16 + lane];
                    v *= rs;
                    const int t = (int)blockIdx.x + tile_n * (int)gridDim.x;
                    // half tiles: lanes 0..7 hold rows 8 (t % 2) .. of tile t / 2
                    const int row = half ? (t >> 1) * 16 + 8 * (t & 1) + lane : t * 16 + lane;
                    const bool mine = row < rows && (!half || lane < 8);
                    if (out.mode == OUT_SILU) {
                        const float upv = __shfl_xor(v, 1);
                        if ((lane & 1) == 0 && mine)
                            reinterpret_cast<float *>(out.y)[row >> 1] = silu_f(v) * upv;
                    } else if (mine) {
                        if (out.mode == OUT_F32) reinterpret_cast<float *>(out.y)[row] = v;
                        else if (out.mode == OUT_ADD) reinterpret_cast<float *>(out.y)[row] += v;
                        else {
                            const unsigned uu = __float_as_uint(v);
                            reinterpret_cast<uint16_t *>(out.y)[row] = (uint16_t)(
                                (uu & 0x7fffffffu) > 0x7f800000u ? (uu >> 16) | 0x40u
                                                                 : (uu + 0x7fffu + ((uu >> 16) & 1u)) >> 16);
                        }
                        if (out.argmax) {
                            // largest under f32's total order, lowest row on ties (sampler/src/lib.rs:40-48)
                            const unsigned long long key =
                                (unsigned long long)((unsigned)total_key(v) ^ 0x80000000u) << 32 |
                                (unsigned long long)(0xffffffffu - (unsigned)row);
                            best = key > best ? key : best;
                        }
                    }
                }
                ++tile_n;
            }
        }
    }
    if (out.argmax && wave == 0) {
        for (int o = 8; o > 0; o >>= 1) {
            const unsigned long long other = __shfl_xor(best, o);
            best = other > best ? other : best;
        }
        if (lane == 0 && best) atomicMax(out.argmax, best);
    }
}

// Waves per block and windows per wave per tile for a row of `windows` 64-column windows: 4 waves for rows of at most
// 32 windows, else 8; the smallest instantiated width whose slices cover the row. 0 when none does.
static int slice_windows(int windows, int &dw) {
    dw = windows <= 32 ? 4 : 8;
    const int widths4[] = {4, 8}, widths8[] = {8, 12, 24};
    if (dw == 4) {
        for (int sm : widths4)
            if (4 * sm >= windows) return sm;
    } else {
        for (int sm : widths8)
            if (8 * sm >= windows) return sm;
    }
    return 0;
}

template <int BITS, int WG, int SM, typename ST, int DW>
static const char *launch_decode_t(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out) {
    // the instantiation's name as rocprof prints it, for the launch profile
    static const std::string name = "gemv_decode<" + std::to_string(BITS) + ", " + std::to_string(WG) + ", " +
                                    std::to_string(SM) + ", " + (sizeof(ST) == 4 ? "float" : "unsigned short") + ", " +
                                    std::to_string(DW) + ">";
    const int windows = (int)(w->cols / 64);
    const int groups = windows / WG;
    // a tile map makes the product's (logical) tiles the mapped blocks of tiles
    if (in.tile_map && (in.map_count < 1 || in.map_count > MAP_MAX || in.map_tiles < 1))
        unsupported("tile map entries (1 to 64)", MAP_MAX, (size_t)in.map_count);
    const int tiles = in.tile_map ? in.map_tiles * in.map_count : (int)(w->rows_padded / 16);
    if (in.tile_map && (in.map_blocks < 1 || (size_t)in.map_blocks * in.map_tiles * 16 > w->rows_padded))
        shape("tile map blocks (within the matrix)", w->rows_padded / 16 / in.map_tiles, (size_t)in.map_blocks);
    const int rows = in.tile_map ? tiles * 16 : (int)w->rows;
    const size_t gpad = (size_t)((groups + 3) & ~3);
    const size_t lds = (size_t)DW * SM * 256 + gpad * 4 + (BITS == 4 ? gpad * 16 : 0) + (size_t)(2 * DW * 16 + DW) * 4;
    auto kern = gemv_decode<BITS, WG, SM, ST, DW>;
    if (lds > 64 * 1024) {
        if (lds > 160 * 1024) unsupported("decode product shared memory (KiB)", 160, lds / 1024);
        HIP_CHECK(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    }
    int resident = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, kern, 64 * DW, lds) != hipSuccess || resident < 1)
        resident = 1;
    const int cu = std::max(g->cu_count, 1);
    // Half tiles where whole tiles load the compute units unevenly and the busiest unit's bytes drop by a fifth or
    // more: 384 tiles on 256 units put 2 tiles on half of them, 768 half tiles put 3 halves on each. A half tile
    // costs a whole tile's instructions for half its bytes, so nowhere else.
    const int full_load = (tiles + cu - 1) / cu, half_load2 = (2 * tiles + cu - 1) / cu;  // (half tiles: x 2)
    const int half = !in.tile_map && 5 * half_load2 <= 8 * full_load ? 1 : 0;
    const int items = tiles << half;
    const int blocks = std::min(items, std::min(resident, DECODE_BLOCKS_PER_CU) * cu);
    if (g->only && name != g->only) {
        g->skipped = true;
        return name.c_str();
    }
    hipEvent_t t0, t1;
    g->kernel_events(t0, t1);
    if (t0)
        hipExtLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(64 * DW), (uint32_t)lds, g->stream, t0, t1, 0u, w->codes,
                              (const ST *)w->scales, in, out, rows, (int)w->cols, items, half);
    else
        kern<<<dim3((unsigned)blocks), dim3(64 * DW), lds, g->stream>>>(w->codes, (const ST *)w->scales, in, out,
                                                                        rows, (int)w->cols, items, half);
    return name.c_str();
}

template <int BITS, int WG, typename ST>
static const char *launch_decode_sm(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out) {
    int dw = 0;
    const int sm = slice_windows((int)(w->cols / 64), dw);
    if (dw == 4) {
        if (sm == 4) return launch_decode_t<BITS, WG, 4, ST, 4>(g, w, in, out);
        return launch_decode_t<BITS, WG, 8, ST, 4>(g, w, in, out);
    }
    if (sm == 8) return launch_decode_t<BITS, WG, 8, ST, 8>(g, w, in, out);
    if (sm == 12) return launch_decode_t<BITS, WG, 12, ST, 8>(g, w, in, out);
    return launch_decode_t<BITS, WG, 24, ST, 8>(g, w, in, out);
}

template <typename ST>
static const char *launch_decode_st(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out) {
    const bool wg2 = w->group == 128;
    if (w->bits == 8) return wg2 ? launch_decode_sm<8, 2, ST>(g, w, in, out) : launch_decode_sm<8, 1, ST>(g, w, in, out);
    return wg2 ? launch_decode_sm<4, 2, ST>(g, w, in, out) : launch_decode_sm<4, 1, ST>(g, w, in, out);
}

bool gemv_decode_supported(const marin_quant_matrix *w) {
    int dw = 0;
    return gemv_supported(w) && (w->group == 64 || w->group == 128) && slice_windows((int)(w->cols / 64), dw) > 0;
}


const char *launch_gemv_decode(marin_gpu *g, const marin_quant_matrix *w, const GemvIn &in, const GemvOut &out) {
    if (w->bf16_scales) return launch_decode_st<uint16_t>(g, w, in, out);
    return launch_decode_st<float>(g, w, in, out);
}

}  // namespace marin
