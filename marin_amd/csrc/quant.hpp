// Quantized matrices on the device and the product kernels' launch interface.
#pragma once

#include "common.hpp"

// Device layout of a quantized matrix (the reference keeps Quantized's row-major layout, crates/cuda/src/quant.rs:16-23;
// this backend keeps every code byte but places them for the matrix-core product):
//  codes, windowed (group and columns multiples of 64, the matrix-core product's matrices):
//         [rows_padded/16 tiles][cols/64 windows][64 lanes][CB bytes], CB = 16 (int8) or 8 (int4). Lane l of a
//         window holds row 16 * tile + l % 16, columns 64 * window + 16 * (l / 16) .. + 16: exactly the A operand of
//         one v_mfma_i32_16x16x64_i8, so every wave load is one contiguous 1 KiB (512 B) run of HBM.
//  codes, row-major (other groups): [rows_padded][row_bytes].
//  int4 bytes: each 4-byte word holds 8 consecutive columns, columns 0-3 in the low nibbles and 4-7 in the high
//         nibbles (stored value code + 8).
//  scales [rows_padded/16][groups][16]  f32 or bf16: the 16 rows of a tile side by side for each group, so a lane
//         reads the scales of its four output rows with one 16-byte (8-byte) load.
// Rows past `rows` up to the next multiple of 64 are zero codes with zero scales.
struct marin_quant_matrix {
    marin_gpu *gpu = nullptr;
    size_t rows = 0, cols = 0, group = 0, rows_padded = 0;
    int bits = 8;
    bool bf16_scales = false;
    bool windowed = false;
    uint8_t *codes = nullptr;
    void *scales = nullptr;
    size_t groups() const { return cols / group; }
    size_t row_bytes() const { return bits == 8 ? cols : (cols + 1) / 2; }
};

namespace marin {

// Byte offset of byte `b` of row `row` (in the row-major device row, int4 already repacked) in the codes.
__host__ __device__ inline size_t code_offset(size_t row, size_t b, size_t row_bytes, bool windowed, size_t cb) {
    if (!windowed) return row * row_bytes + b;
    const size_t j = b / cb;  // 16-column chunk of the row
    return (row >> 4) * 16 * row_bytes + (j >> 2) * 64 * cb + ((j & 3) * 16 + (row & 15)) * cb + b % cb;
}
inline size_t code_chunk(int bits) { return bits == 8 ? 16 : 8; }

constexpr size_t ROW_PAD = 64;

void launch_gemv_valu(marin_gpu *g, const marin_quant_matrix *w, const float *x, size_t tokens, float *y);
void launch_embed_q8(marin_gpu *g, const marin_quant_matrix *w, const uint32_t *ids, size_t n, float *out);
// Fills a matrix from the synthetic generator (seed, stream) and quantizes it int8 with the reference's rule.
// rows_map: optional device-side row permutation: generated row r goes to device row map(r) (for fused layouts).
void launch_synth_quantize(marin_gpu *g, marin_quant_matrix *w, uint64_t seed, uint64_t stream, double std_dev,
                           size_t src_rows, size_t dst_row0, size_t dst_row_step);

marin_quant_matrix *new_quant_matrix(marin_gpu *g, size_t rows, size_t cols, int bits, size_t group, bool bf16);
void free_quant_matrix(marin_quant_matrix *m);
// Host codes/scales (Quantized layout) -> device layout, rows placed from dst_row0 with stride dst_row_step.
void upload_rows(marin_quant_matrix *m, const uint8_t *codes, const void *scales, size_t src_rows, size_t dst_row0,
                 size_t dst_row_step);

// The product every f32 entry point takes: the matrix-core kernel when the matrix allows, the VALU kernel otherwise.
// Any token count (chunks of GEMV_TOKENS).
void matmul_f32(marin_gpu *g, const marin_quant_matrix *w, const float *x, size_t tokens, float *y, bool precise);

}  // namespace marin
