"""Mixture-of-experts decode (config 4) on the GPU.

There is no Qwen3-MoE in the reference (its analogue is Granite's route/experts/mix, crates/cuda/src/granite.cu:12-118,
which takes the top k before a softmax over them), so parity here is pinned by closed forms: the routing is checked
on hand cases (ties go to the lowest expert id, like the sampler's argmax, sampler/src/lib.rs:40-48; renormalized
weights sum to 1) and against an f64 softmax/top-k; the expert FFN against the f64 product of the dequantized experts
(the oracle's quantizer) with the GPU's own routing, tolerance 2e-4 (1 + |e|).
"""
import os

import numpy as np
import pytest

import marin_amd as m
from helpers import assert_close
from oracle import oracle as o

pytestmark = pytest.mark.gpu


def route_reference(logits, k, renorm):
    z = np.asarray(logits, np.float64)
    p = np.exp(z - z.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    ids = np.stack([sorted(range(len(r)), key=lambda e: (-r[e], e))[:k] for r in p])
    w = np.take_along_axis(p, ids, -1)
    if renorm:
        w = w / w.sum(-1, keepdims=True)
    return ids, w


def run_route(gpu, logits, k, renorm):
    tokens, experts = logits.shape
    ids = gpu.typed(m.Dtype.U32, tokens * k)
    w = gpu.zeros(tokens * k)
    gpu.moe_route(gpu.upload(logits.ravel()), tokens, experts, k, renorm, ids, w)
    return gpu.download_typed(ids).reshape(tokens, k).astype(np.int64), gpu.download(w).reshape(tokens, k)


def test_routing_takes_the_largest_probabilities_lowest_id_on_ties(gpu):
    logits = np.zeros((2, 16), np.float32)
    logits[0, [3, 7, 11]] = 2.0  # a three-way tie: ids 3, 7, 11 in that order
    logits[0, 5] = 1.0
    logits[1] = np.arange(16, dtype=np.float32)[::-1]  # descending: experts 0, 1, 2, 3
    ids, w = run_route(gpu, logits, 4, True)
    assert ids[0].tolist() == [3, 7, 11, 5]
    assert ids[1].tolist() == [0, 1, 2, 3]
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)
    assert np.allclose(w[0, :3], w[0, 0]) and w[0, 3] < w[0, 0]
    ids2, w2 = run_route(gpu, logits, 4, False)
    assert (ids2 == ids).all() and (w2.sum(-1) < 1.0).all()


@pytest.mark.parametrize("experts,k,renorm", [(128, 8, True), (64, 4, False), (16, 1, True)])
def test_routing_matches_an_f64_softmax_top_k(gpu, experts, k, renorm):
    logits = np.random.default_rng(experts + k).standard_normal((5, experts)).astype(np.float32)
    ids, w = run_route(gpu, logits, k, renorm)
    ref_ids, ref_w = route_reference(logits, k, renorm)
    assert (ids == ref_ids).all()
    assert np.abs(w - ref_w).max() <= 1e-6


def stack_experts(experts, hidden, ffn, group, seed):
    """Host experts quantized with the oracle: the stacked gate_up (gate/up interleaved) and down codes/scales, and
    their dequantized f64 matrices per expert."""
    gate_up_c, gate_up_s, down_c, down_s, deq = [], [], [], [], []
    for e in range(experts):
        g = o.synth(seed, 3 * e, ffn * hidden)
        u = o.synth(seed, 3 * e + 1, ffn * hidden)
        d = o.synth(seed, 3 * e + 2, hidden * ffn)
        inter = np.empty((2 * ffn, hidden), np.uint16)
        inter[0::2] = g.reshape(ffn, hidden)
        inter[1::2] = u.reshape(ffn, hidden)
        c1, s1 = o.quantize(inter.ravel(), 2 * ffn, hidden, 8, group)
        c2, s2 = o.quantize(d, hidden, ffn, 8, group)
        gate_up_c.append(np.asarray(c1, np.uint8).reshape(2 * ffn, hidden))
        gate_up_s.append(np.asarray(s1, np.float32).reshape(2 * ffn, -1))
        down_c.append(np.asarray(c2, np.uint8).reshape(hidden, ffn))
        down_s.append(np.asarray(s2, np.float32).reshape(hidden, -1))
        gu = o.dequantize(c1, s1, 2 * ffn, hidden, 8, group).astype(np.float64)
        dn = o.dequantize(c2, s2, hidden, ffn, 8, group).astype(np.float64)
        deq.append((gu[0::2], gu[1::2], dn))
    return (np.concatenate(gate_up_c), np.concatenate(gate_up_s), np.concatenate(down_c), np.concatenate(down_s), deq)


# tokens 1: the one-token product with a tile map; 2..8: the grouped batch (each distinct expert read once for all
# tokens; experts 8 with k 8 makes every token share every expert); 9: one product per token
@pytest.mark.parametrize("tokens,experts,k,hidden,ffn,group", [(1, 16, 4, 512, 256, 128), (3, 8, 8, 256, 768, 128),
                                                                (2, 12, 2, 384, 128, 64), (8, 16, 4, 256, 256, 128),
                                                                (9, 6, 3, 256, 128, 128)])
def test_expert_ffn_matches_the_dequantized_experts(gpu, tokens, experts, k, hidden, ffn, group):
    gu_c, gu_s, dn_c, dn_s, deq = stack_experts(experts, hidden, ffn, group, seed=11)
    gate_up = gpu.upload_quantized(experts * 2 * ffn, hidden, 8, group, gu_c, gu_s)
    down = gpu.upload_quantized(experts * hidden, ffn, 8, group, dn_c, dn_s)
    rng = np.random.default_rng(tokens * 100 + k)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    norm = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    out0 = rng.standard_normal((tokens, hidden)).astype(np.float32)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    ids_b = gpu.typed(m.Dtype.U32, tokens * k)
    w_b = gpu.zeros(tokens * k)
    gpu.moe_route(gpu.upload(logits.ravel()), tokens, experts, k, True, ids_b, w_b)
    ids = gpu.download_typed(ids_b).reshape(tokens, k).astype(np.int64)
    wts = gpu.download(w_b).reshape(tokens, k).astype(np.float64)
    act = gpu.zeros(tokens * k * ffn)
    out = gpu.upload(out0.ravel())
    gpu.moe_ffn(gate_up, down, gpu.upload(x.ravel()), gpu.upload(norm), 1e-6, ids_b, w_b, tokens, experts, k, act,
                out)
    got = gpu.download(out).reshape(tokens, hidden)
    xs = x.astype(np.float64)
    rs = 1.0 / np.sqrt((xs * xs).mean(-1, keepdims=True) + 1e-6)
    xn = xs * rs * norm.astype(np.float64)
    exp = out0.astype(np.float64).copy()
    for t in range(tokens):
        for j in range(k):
            g, u, d = deq[ids[t, j]]
            a = g @ xn[t]
            a = a / (1.0 + np.exp(-a)) * (u @ xn[t])
            exp[t] += wts[t, j] * (d @ a)
    assert_close(got.ravel(), exp.ravel(), 2e-4)


def test_expert_ffn_rejects_shapes_it_cannot_run(gpu):
    experts, hidden, ffn = 4, 256, 128
    gate_up = gpu.quantized_synthetic(experts * 2 * ffn, hidden, 128, 1, 1)
    down = gpu.quantized_synthetic(experts * hidden, ffn, 128, 1, 2)
    ids = gpu.typed(m.Dtype.U32, 9)
    w = gpu.zeros(9)
    x = gpu.zeros(hidden)
    with pytest.raises(m.Unsupported):
        gpu.moe_ffn(gate_up, down, x, None, 1e-6, ids, w, 1, experts, 9, gpu.zeros(9 * ffn), gpu.zeros(hidden))
    with pytest.raises(m.Shape):
        gpu.moe_ffn(gate_up, down, x, None, 1e-6, ids, w, 1, experts + 1, 2, gpu.zeros(2 * ffn), gpu.zeros(hidden))


def test_nonfinite_router_logits_are_reported_and_route_nowhere_harmful(gpu):
    """model/src/granite/layer.rs:42-47 refuses non-finite router logits. The routing kernel gives such a token
    experts 0..k-1 with weight 0 (nothing downstream reads outside the experts) and the next blocking call reports
    SelfCheck; finite tokens of the same launch route normally, and the report is cleared once made."""
    experts, k = 16, 4
    logits = np.random.default_rng(3).standard_normal((4, experts)).astype(np.float32)
    logits[1, 5] = np.nan
    logits[2, 0] = np.inf
    logits[3, 9] = -np.inf
    ids = gpu.typed(m.Dtype.U32, 4 * k)
    w = gpu.zeros(4 * k)
    gpu.moe_route(gpu.upload(logits.ravel()), 4, experts, k, True, ids, w)
    with pytest.raises(m.SelfCheck, match="nonfinite router logits"):
        gpu.synchronize()
    got_ids = gpu.download_typed(ids).reshape(4, k).astype(np.int64)
    got_w = gpu.download(w).reshape(4, k)
    for t in (1, 2, 3):
        assert got_ids[t].tolist() == list(range(k)) and np.all(got_w[t] == 0.0)
    ref_ids, ref_w = route_reference(logits[:1], k, True)
    assert got_ids[0].tolist() == ref_ids[0].tolist()
    assert np.abs(got_w[0] - ref_w[0]).max() <= 1e-6
    # the expert FFN over those routes reads only real experts and adds nothing for the weight-0 tokens
    hidden, ffn = 256, 128
    gate_up = gpu.quantized_synthetic(experts * 2 * ffn, hidden, 128, 1, 1)
    down = gpu.quantized_synthetic(experts * hidden, ffn, 128, 1, 2)
    x = gpu.upload(np.ones(4 * hidden, np.float32))
    out = gpu.zeros(4 * hidden)
    gpu.moe_ffn(gate_up, down, x, None, 1e-6, ids, w, 4, experts, k, gpu.zeros(4 * k * ffn), out)
    res = gpu.download(out).reshape(4, hidden)
    assert np.all(res[1:] == 0.0) and np.any(res[0] != 0.0)
    gpu.synchronize()  # reported once, then clear


def synth_expert_rows(seed, stream, row0, rows, cols, group=128):
    """Rows row0 .. row0 + rows - 1 of a device-synthetic int8 matrix (marin_quantized_synthetic), quantized by the
    oracle: quantization is per row, so a row range quantizes exactly as inside the whole matrix. f64 dequantized."""
    w = o.synth(seed, stream, rows * cols, start=row0 * cols)
    c, s = o.quantize(w, rows, cols, 8, group)
    return (c.view(np.int8).reshape(rows, cols // group, group).astype(np.float64)
            * s.reshape(rows, cols // group, 1).astype(np.float64)).reshape(rows, cols)


@pytest.mark.parametrize("tokens", [1, 8])
def test_expert_ffn_at_the_qwen3_30b_a3b_shape(gpu, tokens):
    """Config 4 at its own size: 128 experts of FFN 768 over hidden 2048, int8 g128, top-8 with renormalized softmax
    weights, batch 1 (one-token product with the expert tile map) and 8 (grouped batch); the selected experts
    dequantized by the oracle from the same synthetic streams, f64 product, 2e-4 (1 + |e|)."""
    experts, k, hidden, ffn, seed = 128, 8, 2048, 768, 29
    print(f"case config-4 tokens={tokens}", flush=True)
    o.set_threads(min(16, os.cpu_count() or 1))
    gate_up = gpu.quantized_synthetic(experts * 2 * ffn, hidden, 128, seed, 1)
    down = gpu.quantized_synthetic(experts * hidden, ffn, 128, seed, 2)
    rng = np.random.default_rng(40 + tokens)
    x = rng.standard_normal((tokens, hidden)).astype(np.float32)
    norm = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float32)
    out0 = rng.standard_normal((tokens, hidden)).astype(np.float32)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    ids_b = gpu.typed(m.Dtype.U32, tokens * k)
    w_b = gpu.zeros(tokens * k)
    gpu.moe_route(gpu.upload(logits.ravel()), tokens, experts, k, True, ids_b, w_b)
    ids = gpu.download_typed(ids_b).reshape(tokens, k).astype(np.int64)
    wts = gpu.download(w_b).reshape(tokens, k).astype(np.float64)
    ref_ids, ref_w = route_reference(logits, k, True)
    assert (ids == ref_ids).all() and np.abs(wts - ref_w).max() <= 1e-6
    act = gpu.zeros(tokens * k * ffn)
    out = gpu.upload(out0.ravel())
    gpu.moe_ffn(gate_up, down, gpu.upload(x.ravel()), gpu.upload(norm), 1e-6, ids_b, w_b, tokens, experts, k, act,
                out)
    got = gpu.download(out).reshape(tokens, hidden)
    xs = x.astype(np.float64)
    xn = xs / np.sqrt((xs * xs).mean(-1, keepdims=True) + 1e-6) * norm.astype(np.float64)
    exp = out0.astype(np.float64).copy()
    for e in sorted(set(ids.ravel().tolist())):
        gu = synth_expert_rows(seed, 1, e * 2 * ffn, 2 * ffn, hidden)
        dn = synth_expert_rows(seed, 2, e * hidden, hidden, ffn)
        for t, j in zip(*np.nonzero(ids == e)):
            a = gu[0::2] @ xn[t]
            a = a / (1.0 + np.exp(-a)) * (gu[1::2] @ xn[t])
            exp[t] += wts[t, j] * (dn @ a)
    assert_close(got.ravel(), exp.ravel(), 2e-4)
