"""GPU parity of the quantized linear layers through the C ABI (mirrors crates/cuda/tests/quant.rs).

The oracle is the f64 product of the dequantized rows (quant.rs:19-37) on the same seeded inputs; the shape grid,
group sizes, token counts, extremes and rejections are the reference's own.
"""
import functools
import os

import numpy as np
import pytest

from oracle import oracle as o
from helpers import assert_close, reference_matmul, values, values_fast

pytestmark = pytest.mark.gpu


def quantize(weights, rows, cols, bits, group):
    return o.quantize(o.bf16_bits(weights), rows, cols, bits, group)


def run_case(gpu, bits, group, rows, cols, tokens, weights, tol=1e-4, precise=False):
    codes, scales = quantize(weights, rows, cols, bits, group)
    x = values(tokens * cols, 77)
    expected = reference_matmul(codes, scales, rows, cols, bits, group, x, tokens)
    w = gpu.upload_quantized(rows, cols, bits, group, codes, scales)
    out = gpu.zeros(tokens * rows)
    (gpu.matmul_quant_precise if precise else gpu.matmul_quant)(w, gpu.upload(x), tokens, out)
    assert_close(gpu.download(out), expected, tol)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("group", [32, 64, 128, 256])
@pytest.mark.parametrize("rows,cols", [(5, 256), (70, 512), (130, 256)])
def test_quantized_matmul_matches_the_dequantized_reference(gpu, bits, group, rows, cols):
    print(f"case bits={bits} group={group} {rows}x{cols}", flush=True)
    weights = values(rows * cols, 5)
    for tokens in (1, 3, 8, 9, 15, 16, 40, 65):
        run_case(gpu, bits, group, rows, cols, tokens, weights)


@pytest.mark.parametrize("group", [64, 128, 256])
@pytest.mark.parametrize("rows,cols", [(70, 512), (130, 1024)])
def test_precise_int8_matmul_is_float32_grade(gpu, group, rows, cols):  # quant.rs:184-227
    codes, scales = quantize(values(rows * cols, 5), rows, cols, 8, group)
    w = gpu.upload_quantized(rows, cols, 8, group, codes, scales)
    for tokens, magnitude in ((1, 1.0), (15, 1.0), (16, 1.0), (17, 1.0), (40, 1.0e3), (64, 1.0), (65, 1.0e-3)):
        x = values(tokens * cols, 77) * np.float32(magnitude)
        expected = reference_matmul(codes, scales, rows, cols, 8, group, x, tokens)
        out = gpu.zeros(tokens * rows)
        gpu.matmul_quant_precise(w, gpu.upload(x), tokens, out)
        got = gpu.download(out)
        scale = np.abs(expected).max()
        worst = np.abs(got.astype(np.float64) - expected).max()
        assert worst <= 1.0e-6 * scale, f"group {group} {rows}x{cols} tokens {tokens}: {worst} of {scale}"


@pytest.mark.parametrize("bits", [8, 4])
def test_model_sized_rows_zero_groups_and_extreme_weights(gpu, bits):  # quant.rs:229-243
    w = values(33 * 2048, 6)
    w[:128] = 0.0
    w[2048:2048 + 256] *= np.float32(1.0e-12)
    w[4096] = 1.0e6
    for tokens in (1, 20):
        run_case(gpu, bits, 128, 33, 2048, tokens, w)


def test_uploads_reject_codes_and_scales_that_do_not_fit(gpu):  # quant.rs:255-280
    import marin_amd as m
    gpu.upload_quantized(2, 64, 8, 32, np.zeros(128, np.uint8), np.zeros(4, np.float32))
    gpu.upload_quantized(2, 64, 4, 32, np.zeros(64, np.uint8), np.zeros(4, np.float32))
    bad = [(2, 64, 8, 32, 127, 4), (2, 64, 8, 32, 128, 5), (2, 64, 4, 32, 128, 4), (2, 48, 8, 32, 96, 3),
           (2, 64, 8, 48, 128, 4)]
    for rows, cols, bits, group, nc, ns in bad:
        with pytest.raises(m.Shape):
            gpu.upload_quantized(rows, cols, bits, group, np.zeros(nc, np.uint8), np.zeros(ns, np.float32))


def test_matmul_rejects_wrongly_sized_buffers_instead_of_launching(gpu):  # quant.rs:282-305
    import marin_amd as m
    codes, scales = quantize(values(2 * 64, 3), 2, 64, 8, 32)
    w = gpu.upload_quantized(2, 64, 8, 32, codes, scales)
    x = gpu.zeros(64)
    before = gpu.traffic().launches
    for xx, t, out in ((gpu.zeros(63), 1, gpu.zeros(2)), (x, 1, gpu.zeros(3)), (x, 2, gpu.zeros(2))):
        with pytest.raises(m.Shape):
            gpu.matmul_quant(w, xx, t, out)
    assert gpu.traffic().launches == before
    gpu.matmul_quant(w, x, 1, gpu.zeros(2))
    gpu.matmul_quant(w, gpu.zeros(0), 0, gpu.zeros(0))


def test_int8_embedding_lookup_is_bit_exact_and_refuses_what_it_cannot_do(gpu):  # quant.rs:307-362
    import marin_amd as m
    rows, cols = 50, 256
    codes, scales = quantize(values(rows * cols, 8), rows, cols, 8, 64)
    table = gpu.upload_quantized(rows, cols, 8, 64, codes, scales)
    ids = gpu.tokens(4)
    out = gpu.zeros(3 * cols)
    gpu.embed_quant(table, [7, 0, 49], ids, out)
    deq = o.dequantize(codes, scales, rows, cols, 8, 64)
    expected = np.concatenate([deq[7], deq[0], deq[49]])
    assert np.array_equal(gpu.download(out).view(np.uint32), expected.view(np.uint32))
    one = gpu.zeros(cols)
    gpu.embed_quant(table, [49], ids, one)
    assert np.array_equal(gpu.download(one), expected[2 * cols:])
    with pytest.raises(m.Shape):
        gpu.embed_quant(table, [50], ids, one)
    with pytest.raises(m.Shape):
        gpu.embed_quant(table, [0] * 5, ids, gpu.zeros(5 * cols))
    with pytest.raises(m.Shape):
        gpu.embed_quant(table, [0, 1], ids, one)
    gpu.embed_quant(table, [], ids, gpu.zeros(0))
    c4, s4 = quantize(values(rows * cols, 8), rows, cols, 4, 64)
    narrow = gpu.upload_quantized(rows, cols, 4, 64, c4, s4)
    with pytest.raises(m.Unsupported):
        gpu.embed_quant(narrow, [1], ids, one)


# one token, f32 scales and activations, the a5 tolerance, at the shapes whose tile counts select half tiles (the 8B
# qkv: 384 tiles on 256 compute units, and one row short of it; the 1.7B down: 128 tiles of 96 windows, slices that
# are not whole ring rounds) and at whole-tile shapes beside them
@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("rows,cols", [(6144, 4096), (6143, 4096), (2048, 6144), (4096, 4096), (3072, 2048)])
def test_one_token_products_at_half_and_whole_tile_shapes(gpu, bits, rows, cols):
    print(f"case bits={bits} {rows}x{cols}", flush=True)
    weights = o.bf16_bits(values_fast(rows * cols, 21) * np.float32(0.05))
    codes, scales = o.quantize(weights, rows, cols, bits, 128)
    x = values_fast(cols, 78)
    expected = reference_matmul(codes, scales, rows, cols, bits, 128, x, 1)
    w = gpu.upload_quantized(rows, cols, bits, 128, codes, scales)
    out = gpu.zeros(rows)
    gpu.matmul_quant(w, gpu.upload(x), 1, out)
    assert_close(gpu.download(out), expected, 1e-4)


# (2048, 1000) and (4096, 6144): half tiles at one token (63 tiles, a partial last one; the 8B qkv)
@functools.lru_cache(maxsize=1)
def config1_matrix(k, n, bits):
    """The quantized synthetic matrix of one config-1 case (kept for the next token count of the same shape)."""
    o.set_threads(min(16, os.cpu_count() or 1))
    wbits = o.synth(11, 100 + n + k, n * k)
    codes, scales = o.quantize(wbits, n, k, bits, 128)
    return codes, scales


@pytest.mark.parametrize("m_tokens", [1, 4, 8])
@pytest.mark.parametrize("k,n", [(4096, 4096), (4096, 12288), (12288, 4096), (4096, 151936), (2048, 1000),
                                 (4096, 6144)])
@pytest.mark.parametrize("bits", [8, 4])
def test_decode_shapes_bf16_layout_within_the_north_star_tolerance(gpu, k, n, m_tokens, bits):
    """Config 1: bf16 activations N(0,1)-like, int8 (or int4) g128, bf16 scales, bf16 out; max relative error 1e-2
    (relative to the largest output) against the f64 product. Weights N(0, 0.02) from the synthetic generator."""
    print(f"case bits={bits} k={k} n={n} m={m_tokens}", flush=True)
    codes, scales = config1_matrix(k, n, bits)
    sbf = o.f32_to_bf16_rne(scales)
    s32 = o.bf16_to_f32(sbf)
    x = o.f32_to_bf16_rne(values_fast(m_tokens * k, 99) * np.float32(1.7))
    xf = o.bf16_to_f32(x).astype(np.float64).reshape(m_tokens, k)
    w = gpu.upload_quantized(n, k, bits, 128, codes, sbf, bf16_scales=True)
    xb = gpu.typed(1, host=x)
    out = gpu.typed(1, m_tokens * n)
    gpu.matmul_quant_bf16(w, xb, m_tokens, out)
    got = o.bf16_to_f32(gpu.download_typed(out)).astype(np.float64).reshape(m_tokens, n)
    # f64 reference in row blocks to bound host memory; int4: the even column in the low nibble, stored + 8
    # (tensor/src/quant.rs:218-229)
    exp = np.zeros((m_tokens, n))
    sv = s32.reshape(n, k // 128)
    if bits == 8:
        cview = codes.reshape(n, k).view(np.int8)
    else:
        cview = codes.reshape(n, k // 2)
    for r0 in range(0, n, 8192):
        r1 = min(n, r0 + 8192)
        if bits == 8:
            c = cview[r0:r1].astype(np.float64)
        else:
            packed = cview[r0:r1]
            c = np.empty((r1 - r0, k), np.float64)
            c[:, 0::2] = (packed & 0x0F).astype(np.float64) - 8.0
            c[:, 1::2] = (packed >> 4).astype(np.float64) - 8.0
        deq = c.reshape(r1 - r0, k // 128, 128) * sv[r0:r1, :, None]
        exp[:, r0:r1] = xf @ deq.reshape(r1 - r0, k).T
    rel = np.abs(got - exp).max() / np.abs(exp).max()
    assert rel <= 1e-2, rel
    # bf16 output rounding bounds the error per element as well
    assert np.all(np.abs(got - exp) <= np.abs(exp) * 2 ** -7 + 1e-3 * np.abs(exp).max())


@pytest.mark.parametrize("k,n", [(4096, 4096), (12288, 4096), (2048, 1000), (4096, 6144)])
@pytest.mark.parametrize("tokens", [32, 100, 512])
def test_prompt_products_with_bf16_scales_are_float32_grade(gpu, k, n, tokens):
    """The prompt GEMM (32+ tokens: 22-bit activations in three limbs, workgroups of 128 or 256 rows, partial token
    blocks) with bf16 weight scales and f32 activations: within 1e-6 of the largest output of the f64 product over the
    same bf16-rounded scales, the bound of the reference's integer path (cuda/tests/quant.rs:76-118)."""
    print(f"case k={k} n={n} tokens={tokens}", flush=True)
    codes, scales = config1_matrix(k, n, 8)
    sbf = o.f32_to_bf16_rne(scales)
    s32 = o.bf16_to_f32(sbf)
    x = values_fast(tokens * k, 41)
    w = gpu.upload_quantized(n, k, 8, 128, codes, sbf, bf16_scales=True)
    out = gpu.zeros(tokens * n)
    gpu.matmul_quant(w, gpu.upload(x), tokens, out)
    got = gpu.download(out).astype(np.float64).reshape(tokens, n)
    c = codes.reshape(n, k).view(np.int8).astype(np.float64)
    deq = (c.reshape(n, k // 128, 128) * s32.reshape(n, k // 128)[:, :, None]).reshape(n, k)
    exp = x.astype(np.float64).reshape(tokens, k) @ deq.T
    worst = np.abs(got - exp).max()
    assert worst <= 1e-6 * np.abs(exp).max(), (worst, np.abs(exp).max())
