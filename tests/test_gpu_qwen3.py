"""End-to-end parity of the Qwen3 decode driver on the GPU against the CPU oracle.

- synthetic weights: generated and quantized on the device, bit-exact with the oracle's generator + quantizer;
- tiny-qwen3 (the reference's HF fixture) quantized int8 g64: logits against the oracle's forward on the same codes;
- synthetic Qwen3-shaped models: greedy tokens equal to the committed oracle goldens (tests/golden/qwen3_*.json),
  through the HIP-graph decode loop and the eager one, and per-step top-5 logits within tolerance;
- model/tests/quantized.rs: a one-token pass equals a prompt pass within 1e-3, runs repeat exactly, and a decode
  step allocates nothing.
"""
import json
import os

import numpy as np
import pytest

import marin_amd as m
from marin_amd.qwen3 import Qwen3
from oracle import oracle as o

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def golden(name):
    path = os.path.join(GOLDEN, f"qwen3_{name}_greedy.json")
    if not os.path.exists(path):
        pytest.skip(f"{path} not generated (tests/golden/make_qwen3_golden.py {name})")
    return json.load(open(path))


@pytest.mark.parametrize("rows,cols,group,seed,stream", [(300, 512, 128, 5, 77), (64, 4096, 64, 9, 3),
                                                         (130, 768, 256, 1, 1 << 8)])
def test_device_synthetic_weights_and_quantizer_are_bit_exact(gpu, rows, cols, group, seed, stream):
    w = gpu.quantized_synthetic(rows, cols, group, seed, stream)
    ids = gpu.tokens(rows)
    out = gpu.zeros(rows * cols)
    gpu.embed_quant(w, np.arange(rows), ids, out)
    codes, scales = o.quantize(o.synth(seed, stream, rows * cols), rows, cols, 8, group)
    expected = o.dequantize(codes, scales, rows, cols, 8, group).ravel()
    assert np.array_equal(gpu.download(out).view(np.uint32), expected.view(np.uint32))


def tiny():
    d = os.path.join(GOLDEN, "tiny-qwen3")
    cfg = json.load(open(os.path.join(d, "config.json")))
    w = o.load_safetensors_f32(os.path.join(d, "model.safetensors"))
    ref = json.load(open(os.path.join(d, "reference.json")))
    return cfg, w, ref


@pytest.mark.parametrize("fmt", [m.KvFormat.F32, m.KvFormat.F16])
def test_tiny_qwen3_int8_matches_the_oracle_on_the_same_codes(gpu, fmt):
    cfg, w, ref = tiny()
    model = Qwen3.from_hf(gpu, cfg, w, o.quantize, group=64)
    for case in ref["cases"]:
        cache = model.new_cache(128, fmt)
        oracle = o.Qwen3Oracle(cfg, w, 128, group=64, kv_f16=fmt == m.KvFormat.F16)
        got = model.forward(case["prompt_ids"], cache)
        exp = oracle.forward(case["prompt_ids"])
        # f16 storage: a last-bit difference in a key before rounding can move it by one f16 ulp (2^-11)
        tol = 1e-4 if fmt == m.KvFormat.F32 else 2.0 ** -11 * 4
        for step in case["steps"]:
            assert np.abs(got - exp).max() <= tol * (1 + np.abs(exp).max())
            assert o.argmax(got) == o.argmax(exp)
            got = model.forward([step["token"]], cache)
            exp = oracle.forward([step["token"]])


@pytest.mark.parametrize("name", ["mini", "mini_f16kv", "mini_tied"])
def test_synthetic_greedy_tokens_match_the_golden(gpu, name, monkeypatch):
    g = golden(name)
    fmt = m.KvFormat.F16 if g["kv_f16"] else m.KvFormat.F32
    model = Qwen3(gpu, g["shape"], seed=g["seed"])
    steps = len(g["tokens"])
    for graph in (True, False):
        monkeypatch.setenv("MARIN_NO_GRAPH", "0" if graph else "1")
        cache = model.new_cache(len(g["prompt"]) + steps + 1, fmt)
        toks = model.generate(g["prompt"], steps, cache)
        assert toks.tolist() == g["tokens"], f"graph={graph}"
    # step-by-step logits against the oracle's top five
    cache = model.new_cache(len(g["prompt"]) + steps + 1, fmt)
    logits = model.forward(g["prompt"], cache)
    for s in range(steps):
        ids, vals = g["top_ids"][s], np.array(g["top_vals"][s])
        assert np.abs(logits[ids] - vals).max() <= 1e-3 * (1 + np.abs(vals).max()), s
        assert o.argmax(logits) == g["tokens"][s]
        logits = model.forward([g["tokens"][s]], cache)


@pytest.mark.parametrize("fmt", [m.KvFormat.F32, m.KvFormat.F16])
def test_a_prompt_longer_than_a_chunk_matches_the_oracle(gpu, fmt):
    """A 600-token prompt runs as passes of at most the library's prompt chunk (512 tokens: 512, 88), each
    seeing the keys of the ones before; the greedy continuation and its top logits match the oracle's prompt pass.
    With f16 keys and values the chunks' attention runs on the matrix cores."""
    g = golden("mini")
    shape = g["shape"]
    prompt = o.synth_prompt(g["seed"] + 7, 600, shape["vocab"]).tolist()
    steps = 6
    toks, gaps, top_ids, top_vals = o.synth_greedy(shape, g["seed"], prompt, steps, kv_f16=fmt == m.KvFormat.F16,
                                                   with_top=True)
    model = Qwen3(gpu, shape, seed=g["seed"])
    cache = model.new_cache(len(prompt) + steps + 1, fmt)
    logits = model.forward(prompt, cache)
    for s in range(steps):
        vals = np.asarray(top_vals[s], np.float64)
        assert np.abs(logits[top_ids[s]] - vals).max() <= 1e-3 * (1 + np.abs(vals).max()), s
        if gaps[s] > 1e-3:
            assert o.argmax(logits) == toks[s], s
        logits = model.forward([int(toks[s])], cache)


@pytest.mark.parametrize("name", ["mini_f16kv", "1.7b"])
def test_prompt_attention_on_the_matrix_cores_equals_the_vector_path(gpu, name):
    """The f16-cache prompt pass with its attention on the matrix cores (q and P split into two f16 parts each)
    against the same pass on the vector-ALU attention: the logits agree to f32 accuracy. 1300 tokens: chunks of 512,
    512 and 276, the last one's rows split over two spans of 1024 positions and merged."""
    g = golden(name)
    shape = g["shape"]
    prompt = o.synth_prompt(g["seed"] + 3, 1300, shape["vocab"]).tolist()
    model = Qwen3(gpu, shape, seed=g["seed"])
    out = []
    try:
        for fast in (True, False):  # Gpu::set_fast_attention (attention.rs:81-86)
            gpu.set_fast_attention(fast)
            out.append(model.forward(prompt, model.new_cache(len(prompt) + 1, m.KvFormat.F16)))
    finally:
        gpu.set_fast_attention(True)
    assert np.abs(out[0] - out[1]).max() <= 2e-4 * (1 + np.abs(out[1]).max())


@pytest.mark.parametrize("head_dim,heads,kv_heads", [(64, 8, 8), (64, 8, 2), (64, 16, 2), (128, 4, 4), (128, 16, 2)])
def test_prompt_attention_equals_the_vector_path_at_every_group_size(gpu, head_dim, heads, kv_heads):
    """The matrix-core prompt attention at group sizes 1, 4 and 8 (q heads per kv head) and both head sizes, where
    the staging of its key/value tiles takes its other layouts: against the vector-ALU attention on the same model,
    a 1100-token prompt (two chunks of 512 and one of 76, rows past 1024 positions split over spans)."""
    shape = dict(golden("mini_f16kv")["shape"], layers=2, head_dim=head_dim, heads=heads, kv_heads=kv_heads)
    prompt = o.synth_prompt(29, 1100, shape["vocab"]).tolist()
    model = Qwen3(gpu, shape, seed=5)
    out = []
    try:
        for fast in (True, False):
            gpu.set_fast_attention(fast)
            out.append(model.forward(prompt, model.new_cache(len(prompt) + 1, m.KvFormat.F16)))
    finally:
        gpu.set_fast_attention(True)
    assert np.abs(out[0] - out[1]).max() <= 2e-4 * (1 + np.abs(out[1]).max())


def agree_until_a_near_tie(got, exp, gaps, tie=1e-3):
    """Greedy sequences agree, or first differ at a step whose oracle top-1/top-2 gap is below `tie`."""
    for i, (a, b) in enumerate(zip(got, exp)):
        if a != b:
            assert gaps[i] < tie, (i, a, b, gaps[i])
            return i
    return len(exp)


@pytest.mark.parametrize("batch", [3, 8])
def test_batch_decode_matches_each_sequence_on_the_oracle(gpu, batch, monkeypatch):
    """Sequences of different prompt lengths decoded together (every product over the batch, one attention launch
    over all sequences) give each sequence the oracle's greedy tokens; graph replay and eager launches agree."""
    g = golden("mini")
    shape = g["shape"]
    steps = 8
    prompts = [o.synth_prompt(g["seed"] + 11 + i, 17 + 9 * i, shape["vocab"]).tolist() for i in range(batch)]
    model = Qwen3(gpu, shape, seed=g["seed"])
    runs = []
    for graph in (True, False):
        monkeypatch.setenv("MARIN_NO_GRAPH", "0" if graph else "1")
        b = model.new_batch(batch, max(len(p) for p in prompts) + 2 * steps + 1)
        for i, p in enumerate(prompts):
            b.prefill(i, p)
        first = b.decode(steps // 2)
        runs.append(np.concatenate([first, b.decode(steps - steps // 2)], axis=1))
        assert [b.length(i) for i in range(batch)] == [len(p) + steps for p in prompts]
    assert (runs[0] == runs[1]).all()
    compared = 0
    for i, p in enumerate(prompts):
        toks, gaps = o.synth_greedy(shape, g["seed"], p, steps)
        compared += agree_until_a_near_tie(runs[0][i].tolist(), toks.tolist(), gaps)
    assert compared >= batch * steps // 2


def test_one_token_pass_equals_a_prompt_pass_and_runs_repeat(gpu):  # model/tests/quantized.rs:74-97
    g = golden("mini")
    model = Qwen3(gpu, g["shape"], seed=g["seed"])
    prompt = g["prompt"][:20]
    whole = model.forward(prompt + [3, 5], model.new_cache(64))
    c = model.new_cache(64)
    model.forward(prompt, c)
    model.forward([3], c)
    step = model.forward([5], c)
    assert np.abs(whole - step).max() < 1e-3
    again = model.forward(prompt + [3, 5], model.new_cache(64))
    assert np.array_equal(whole, again)


def test_a_decode_step_allocates_nothing(gpu):  # model/tests/quantized.rs:98-118
    g = golden("mini")
    model = Qwen3(gpu, g["shape"], seed=g["seed"])
    c = model.new_cache(128)
    model.forward(g["prompt"], c)
    model.decode(2, c)
    before = gpu.traffic().allocations
    model.forward([7], c)
    model.decode(8, c)
    assert gpu.traffic().allocations == before


@pytest.mark.parametrize("name", ["1.7b", "8b"])
def test_model_shaped_greedy_tokens_match_the_golden(gpu, name):
    g = golden(name)
    model = Qwen3(gpu, g["shape"], seed=g["seed"])
    steps = len(g["tokens"])
    cache = model.new_cache(len(g["prompt"]) + steps + 1)
    toks = model.generate(g["prompt"], steps, cache)
    assert toks.tolist() == g["tokens"]
    cache = model.new_cache(len(g["prompt"]) + 2)
    logits = model.forward(g["prompt"], cache)
    ids, vals = g["top_ids"][0], np.array(g["top_vals"][0])
    assert np.abs(logits[ids] - vals).max() <= 1e-3 * (1 + np.abs(vals).max())


def test_profiled_step_accounts_every_launch(gpu):
    g = golden("mini")
    model = Qwen3(gpu, g["shape"], seed=g["seed"])
    c = model.new_cache(128)
    model.forward(g["prompt"], c)
    p = model.profile_step(c)
    L = g["shape"]["layers"]
    assert p["gemv_launches"] == 4 * L + 1
    # one attention launch per layer: q/k norm, RoPE, the cache store and the chunk merge happen inside it
    assert p["attention_launches"] == L
    assert p["gemv_bytes"] > 0 and p["gemv_seconds"] > 0 and p["step_seconds"] >= p["gemv_seconds"]


def test_a_packed_artifact_loads_the_same_model_as_quantizing_on_load(gpu, tmp_path):
    """marin-q8-v1 (loader/src/packed.rs, GpuStore::packed gpu.rs:47-50): the reference's own codes and scales,
    uploaded as they are, give exactly the logits of quantizing the same bf16 weights on load."""
    import shutil

    from packed_bundle import write_packed

    cfg, w, ref = tiny()
    src = tmp_path / "src"
    src.mkdir()
    shutil.copyfile(os.path.join(GOLDEN, "tiny-qwen3", "config.json"), src / "config.json")
    (src / "tokenizer.json").write_text('{"version": "1.0"}')
    write_packed(str(src), w, str(tmp_path / "packed"), 64)
    packed = Qwen3.from_packed(gpu, str(tmp_path / "packed"))
    direct = Qwen3.from_hf(gpu, cfg, w, o.quantize, group=64)
    prompt = ref["cases"][0]["prompt_ids"]
    a = packed.forward(prompt, packed.new_cache(64))
    b = direct.forward(prompt, direct.new_cache(64))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_a_4096_token_prompt_at_8b_widths_matches_the_golden(gpu):
    """Config 3's prompt at its own length on an 8B-width model of reduced depth (2 layers): the 4096-token prefill
    with an f16 cache runs in 512-token passes on the matrix cores (rows past 1024 positions split over spans and
    merged), then 64 greedy tokens on the decode path. Tokens equal the oracle's until a step whose top-1/top-2 gap
    is a near tie; the first step's top-5 logits agree within f16-cache accuracy."""
    g = golden("8b_long")
    shape = g["shape"]
    model = Qwen3(gpu, shape, seed=g["seed"])
    steps = len(g["tokens"])
    cache = model.new_cache(len(g["prompt"]) + steps + 1, m.KvFormat.F16)
    toks = model.generate(g["prompt"], steps, cache)
    assert agree_until_a_near_tie(toks.tolist(), g["tokens"], g["gaps"]) >= steps // 2
    cache = model.new_cache(len(g["prompt"]) + 2, m.KvFormat.F16)
    logits = model.forward(g["prompt"], cache)
    ids, vals = g["top_ids"][0], np.array(g["top_vals"][0])
    assert np.abs(logits[ids] - vals).max() <= 1e-3 * (1 + np.abs(vals).max())


def test_batch_8_decode_at_8b_widths_matches_the_golden(gpu):
    """Config 3's batch 8 at 8B widths (3 layers): eight prompts of different lengths decoded together, every
    product over the batch on the batch kernels of the 8B shapes; each sequence gets the oracle's greedy tokens
    (tests/golden/qwen3_8b_batch_greedy.json), or first differs at a near tie."""
    g = golden("8b_batch")
    shape, seqs, steps = g["shape"], g["sequences"], g["steps"]
    model = Qwen3(gpu, shape, seed=g["seed"])
    b = model.new_batch(len(seqs), max(len(s["prompt"]) for s in seqs) + steps + 1)
    for i, s in enumerate(seqs):
        b.prefill(i, s["prompt"])
    got = b.decode(steps)
    compared = 0
    for i, s in enumerate(seqs):
        compared += agree_until_a_near_tie(got[i].tolist(), s["tokens"], s["gaps"])
    assert compared >= len(seqs) * steps // 2


@pytest.mark.parametrize("count", [2, 5, 8])
def test_forward_rows_gives_every_rows_logits(gpu, count):
    """CausalLm::forward_rows (runtime/src/lib.rs:86-99, model/src/qwen3/gpu.rs:212-236): one pass over the guessed
    tokens returns the logits after each of them. Every row matches the oracle fed the same tokens one at a time
    (the reference's default forward_rows) and the GPU's own one-token passes; the greedy continuation after it is
    the one after feeding the tokens one by one; more than 8 tokens are refused and change nothing."""
    g = golden("mini")
    shape = g["shape"]
    model = Qwen3(gpu, shape, seed=g["seed"])
    prompt = g["prompt"][:24]
    guesses = g["tokens"][:count]
    cache = model.new_cache(64)
    model.forward(prompt, cache)
    rows = model.forward_rows(guesses, cache)
    assert rows.shape == (count, shape["vocab"]) and len(cache) == len(prompt) + count
    exp = o.synth_rows(shape, g["seed"], prompt, guesses)
    for i in range(count):
        assert np.abs(rows[i] - exp[i]).max() <= 1e-3 * (1 + np.abs(exp[i]).max()), i
    one = model.new_cache(64)
    model.forward(prompt, one)
    singles = np.stack([model.forward([t], one) for t in guesses])
    assert np.abs(rows - singles).max() < 1e-3
    assert model.decode(4, cache).tolist() == model.decode(4, one).tolist()
    with pytest.raises(m.Unsupported):
        model.forward_rows(g["tokens"][:9], cache)
    assert len(cache) == len(prompt) + count + 4
