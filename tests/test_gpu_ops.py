"""GPU parity of the elementwise ops (mirrors crates/cuda/tests/ops.rs) against the CPU oracle."""
import numpy as np
import pytest

from oracle import oracle as o
from helpers import assert_close, values

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim,rows", [(64, 3), (128, 32), (2048, 2), (4096, 1), (100, 5)])
def test_rms_norm_matches_the_cpu(gpu, dim, rows):
    x = values(dim * rows, 3) * np.float32(4.0)
    w = values(dim, 4) + np.float32(1.5)
    exp = o.rms_norm_rows(x, w, 1e-6)
    b = gpu.upload(x)
    out = gpu.zeros(x.size)
    gpu.rms_norm_into(b, gpu.upload(w), out, 1e-6)
    assert_close(gpu.download(out), exp, 1e-5)
    gpu.rms_norm(b, gpu.upload(w), 1e-6)
    assert_close(gpu.download(b), exp, 1e-5)


@pytest.mark.parametrize("heads,hd,start,tokens", [(4, 16, 0, 3), (32, 128, 4095, 2), (8, 128, 100, 1), (2, 2, 1, 1)])
def test_rope_matches_the_cpu(gpu, heads, hd, start, tokens):
    x = values(tokens * heads * hd, 9)
    exp = o.rope_tokens(x, heads * hd, hd, start, 1.0e6)
    b = gpu.upload(x)
    gpu.rope(b, heads, hd, start, 1.0e6)
    assert_close(gpu.download(b), exp, 2e-5 * max(1.0, start / 64))


def test_silu_mul_and_add_match_the_cpu(gpu):
    g = values(10000, 1) * np.float32(8.0)
    u = values(10000, 2) * np.float32(3.0)
    gb, ub = gpu.upload(g), gpu.upload(u)
    gpu.silu_mul(gb, ub)
    assert_close(gpu.download(gb), o.silu_mul(g, u), 1e-5)
    a = gpu.upload(g)
    gpu.add(a, ub)
    assert np.array_equal(gpu.download(a), g + u)


def test_rejects_mismatched_sizes(gpu):
    import marin_amd as m
    with pytest.raises(m.Shape):
        gpu.add(gpu.zeros(3), gpu.zeros(2))
    with pytest.raises(m.Shape):
        gpu.rms_norm(gpu.zeros(5), gpu.zeros(2), 1e-6)
    with pytest.raises(m.Shape):
        gpu.rope(gpu.zeros(6), 1, 3, 0, 1e4)
