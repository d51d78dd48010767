"""Writes the greedy-decode goldens of the synthetic Qwen3 models with the CPU oracle.

    python tests/golden/make_qwen3_golden.py [mini|1.7b|all]

Each fixture holds the model shape, the weight seed, the prompt (from or_synth_prompt) and the greedy tokens with the
top-1/top-2 logit gap of every step. The GPU tests rebuild the same weights on the device from the seed and must
choose the same tokens.
"""
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as o  # noqa: E402

MINI = dict(layers=4, hidden=512, heads=8, kv_heads=4, head_dim=64, ffn=1024, vocab=4096, eps=1e-6, theta=1.0e6,
            tied=False, group=128)
CASES = {
    "mini": dict(shape=MINI, seed=7, prompt_len=40, steps=64, kv_f16=False),
    "mini_f16kv": dict(shape=MINI, seed=7, prompt_len=40, steps=64, kv_f16=True),
    "mini_tied": dict(shape=dict(MINI, tied=True), seed=7, prompt_len=40, steps=16, kv_f16=False),
    "1.7b": dict(shape=dict(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, ffn=6144, vocab=151936,
                            eps=1e-6, theta=1.0e6, tied=True, group=128),
                 seed=1, prompt_len=128, steps=64, kv_f16=False),
    "8b": dict(shape=dict(layers=36, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=151936,
                          eps=1e-6, theta=1.0e6, tied=False, group=128),
               seed=3, prompt_len=16, steps=32, kv_f16=False),
    # 8B widths at reduced depth: a 4096-token prompt (prefill on the matrix cores with an f16 cache, rows past 1024
    # positions split over spans), then 64 greedy tokens
    "8b_long": dict(shape=dict(layers=2, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=151936,
                               eps=1e-6, theta=1.0e6, tied=False, group=128),
                    seed=5, prompt_len=4096, steps=64, kv_f16=True),
}
# decode batches: `batch` prompts of lengths 17 + 9 i (seeds seed + 11 + i), each decoded greedily on its own
BATCHES = {
    "8b_batch": dict(shape=dict(CASES["8b_long"]["shape"], layers=3), seed=6, batch=8, steps=16, kv_f16=False),
}


def make_batch(name):
    c = BATCHES[name]
    o.set_threads(os.cpu_count() or 1)
    t = time.time()
    seqs = []
    for i in range(c["batch"]):
        prompt = o.synth_prompt(c["seed"] + 11 + i, 17 + 9 * i, c["shape"]["vocab"])
        toks, gaps = o.synth_greedy(c["shape"], c["seed"], prompt, c["steps"], kv_f16=c["kv_f16"])
        seqs.append(dict(prompt=[int(v) for v in prompt], tokens=[int(v) for v in toks],
                         gaps=[float(g) for g in gaps]))
    out = dict(name=name, shape=c["shape"], seed=c["seed"], kv_f16=c["kv_f16"], steps=c["steps"], sequences=seqs,
               note="or_qwen3_greedy per sequence: int8 group-128 weights from or_synth_bf16, f32 math")
    with open(os.path.join(HERE, f"qwen3_{name}_greedy.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(f"{name}: {time.time() - t:.1f}s, min gap {min(min(s['gaps']) for s in seqs):.4g}")


def make(name):
    c = CASES[name]
    o.set_threads(os.cpu_count() or 1)
    prompt = o.synth_prompt(c["seed"], c["prompt_len"], c["shape"]["vocab"])
    t = time.time()
    toks, gaps, top_ids, top_vals = o.synth_greedy(c["shape"], c["seed"], prompt, c["steps"], kv_f16=c["kv_f16"],
                                                   with_top=True)
    out = dict(name=name, shape=c["shape"], seed=c["seed"], kv_f16=c["kv_f16"], prompt=[int(v) for v in prompt],
               tokens=[int(v) for v in toks], gaps=[float(g) for g in gaps],
               top_ids=top_ids.tolist(), top_vals=[[float(v) for v in r] for r in top_vals],
               note="or_qwen3_greedy: int8 group-128 weights from or_synth_bf16, f32 math, lowest-index argmax")
    path = os.path.join(HERE, f"qwen3_{name}_greedy.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(f"{name}: {time.time() - t:.1f}s, min gap {min(gaps):.4g}, tokens {out['tokens'][:12]}...")


if __name__ == "__main__":
    which = sys.argv[1] if len(sys.argv) > 1 else "all"
    for n in (list(CASES) + list(BATCHES) if which == "all" else [which]):
        make_batch(n) if n in BATCHES else make(n)
