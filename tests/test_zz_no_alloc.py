"""The allocation-free product (marin_matmul_quant_bf16_noalloc) against marin_matmul_quant_bf16 through the C ABI:
bit-identical outputs on two calls in a row (the second smaller), no device allocation during them, and a product
whose scratch exceeds the fixed array refused before anything runs."""
import numpy as np
import pytest

import marin_amd as m
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def matrix(gpu, rows, cols, bits, seed):
    codes, scales = o.quantize(o.synth(seed, 7, rows * cols), rows, cols, bits, 128)
    return gpu.upload_quantized(rows, cols, bits, 128, codes, o.f32_to_bf16_rne(scales), bf16_scales=True)


def bf16_input(gpu, tokens, cols, seed):
    x = o.f32_to_bf16_rne(np.random.default_rng(seed).standard_normal(tokens * cols).astype(np.float32))
    return gpu.typed(m.Dtype.BF16, host=x)


@pytest.mark.parametrize("bits", [8, 4])
def test_the_allocation_free_product_equals_the_allocating_one(gpu, bits):
    cases = [(6144, 4096, 8), (1024, 2048, 3)]  # the second call smaller in every dimension
    mats = [matrix(gpu, r, c, bits, 3 + i) for i, (r, c, _) in enumerate(cases)]
    xs = [bf16_input(gpu, t, c, 10 + i) for i, (_, c, t) in enumerate(cases)]
    expected = []
    for w, x, (r, c, t) in zip(mats, xs, cases):
        out = gpu.typed(m.Dtype.BF16, t * r)
        gpu.matmul_quant_bf16(w, x, t, out)
        expected.append(gpu.download_typed(out))
    before = gpu.traffic().allocations
    outs = [gpu.typed(m.Dtype.BF16, t * r) for (r, c, t) in cases]
    after_outputs = gpu.traffic().allocations
    for w, x, out, (r, c, t) in zip(mats, xs, outs, cases):
        gpu.matmul_quant_bf16_noalloc(w, x, t, out)
    gpu.synchronize()
    assert gpu.traffic().allocations == after_outputs >= before
    for out, exp in zip(outs, expected):
        assert np.array_equal(gpu.download_typed(out), exp)


def test_a_product_beyond_the_fixed_scratch_is_refused_before_running(gpu):
    w = matrix(gpu, 64, 12288, 8, 5)
    tokens = 200  # about 10 MB of activation limbs, past the 4 MiB array
    x = bf16_input(gpu, tokens, 12288, 6)
    out = gpu.typed(m.Dtype.BF16, tokens * 64)
    launches = gpu.traffic().launches
    with pytest.raises(m.Unsupported, match="allocation-free"):
        gpu.matmul_quant_bf16_noalloc(w, x, tokens, out)
    assert gpu.traffic().launches == launches
    assert np.all(gpu.download_typed(out) == 0)
