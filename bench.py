"""Decode throughput of the Qwen3-8B-shaped int8 model on one MI355X (batch 1).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--prompt 4096] [--kv f16] [--no-cpu]

A step is one greedy decode token: argmax of the last logits, then one pass of the token through 36 layers and the
output head (int8 group-128 weights, f32 scales, f32 activations split to f16 hi/lo on the matrix cores, f32
accumulation). Weights are random-init N(0, 0.02) generated and quantized on the device (no checkpoint); the prompt
is 4096 uniform random ids, prefilled before timing. The timed region is exactly K steps between two stream
synchronizations, with every input already resident in HBM.

One JSON line goes to stdout. `roofline` comes from event-profiled decode steps run right after the timed region
(an event after every launch; the quantized products' algorithmic bytes over their summed durations). `cpu_baseline`
times the CPU oracle (oracle/marin_oracle.c, a C restatement of Marin's single-threaded int8 decode GEMV and
attention) on one core over a bounded sample of the same token's work.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0


def cpu_baseline(shape: dict, ctx: int, budget_s: float = 12.0) -> dict:
    """Seconds per 8B decode token on one host core: every projection shape of one layer (x36), the output head,
    and attention over `ctx` f32 cached positions for every layer, with the oracle's Q8Gemv and AttendOne."""
    from oracle import oracle as o
    o.set_threads(1)
    rng = np.random.default_rng(0)
    H, F, V, L = shape["hidden"], shape["ffn"], shape["vocab"], shape["layers"]
    qd, kvd, g = shape["heads"] * shape["head_dim"], shape["kv_heads"] * shape["head_dim"], shape["group"]
    mats = [(qd, H), (kvd, H), (kvd, H), (H, qd), (F, H), (F, H), (H, F)]

    def gemv_time(rows, cols, reps=1):
        codes = rng.integers(0, 256, rows * cols, dtype=np.uint8)
        codes[codes == 128] = 127
        scales = rng.random(rows * cols // g, dtype=np.float32) * np.float32(1e-3)
        x = rng.standard_normal(cols).astype(np.float32)
        out = np.zeros(rows, np.float32)
        t = time.perf_counter()
        for _ in range(reps):
            o.lib.or_q8_gemv(codes.ctypes.data, scales.ctypes.data, x.ctypes.data, out.ctypes.data, rows, cols, g)
        return (time.perf_counter() - t) / reps

    t0 = time.perf_counter()
    layer = sum(gemv_time(r, c) for r, c in mats)
    head = gemv_time(V, H)
    hd = shape["head_dim"]
    q = rng.standard_normal(qd).astype(np.float32)
    kv = rng.standard_normal(2 * ctx * kvd).astype(np.float32)
    out = np.zeros(qd, np.float32)
    t = time.perf_counter()
    o.lib.or_attention(q.ctypes.data, kv.ctypes.data, kv.ctypes.data + ctx * kvd * 4, out.ctypes.data,
                       shape["heads"], shape["kv_heads"], hd, ctx - 1, 1)
    attn = time.perf_counter() - t
    per_token = L * (layer + attn) + head
    reps = 1
    while time.perf_counter() - t0 < budget_s and reps < 4:  # a second pass steadies the estimate
        layer2 = sum(gemv_time(r, c) for r, c in mats)
        per_token = min(per_token, L * (layer2 + attn) + head)
        reps += 1
    return {"value": round(1.0 / per_token, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"one {L}-layer token: each projection shape of one layer x{L}, output head once, attention "
                      f"over {ctx} f32 positions x{L}; oracle Q8Gemv/AttendOne on 1 core, best of {reps}",
            "seconds_per_token": round(per_token, 4)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=4096)
    ap.add_argument("--kv", choices=["f32", "f16", "bf16"], default="f16")
    ap.add_argument("--profile-steps", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the decode step's kernels one by one instead of replaying a HIP graph (for tracers)")
    args = ap.parse_args()
    if args.no_graph:
        os.environ["MARIN_NO_GRAPH"] = "1"
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the one-GPU throughput is the reported value", file=sys.stderr)
        return 2

    import marin_amd as m
    from marin_amd.qwen3 import SHAPES, Qwen3, weight_bytes

    shape = SHAPES["qwen3-8b"]
    fmt = {"f32": m.KvFormat.F32, "f16": m.KvFormat.F16, "bf16": m.KvFormat.BF16}[args.kv]
    print(f"[bench] qwen3-8b int8 g128, prompt {args.prompt}, kv {args.kv}, warmup {args.warmup}, steps "
          f"{args.steps}", file=sys.stderr, flush=True)
    gpu = m.Gpu()
    info = gpu.info()
    t = time.perf_counter()
    model = Qwen3(gpu, shape, seed=args.seed)
    build_s = time.perf_counter() - t
    capacity = args.prompt + args.warmup + args.steps + args.profile_steps + 8
    cache = model.new_cache(capacity, fmt)
    prompt = np.random.default_rng(args.seed).integers(0, shape["vocab"], args.prompt, dtype=np.uint32)
    gpu.synchronize()
    t = time.perf_counter()
    model.forward(prompt, cache)
    gpu.synchronize()
    prefill_s = time.perf_counter() - t
    print(f"[bench] weights {build_s:.1f}s, prefill {prefill_s:.2f}s", file=sys.stderr, flush=True)

    model.decode(args.warmup, cache)
    gpu.synchronize()
    m0 = gpu.mark()
    t = time.perf_counter()
    tokens = model.decode(args.steps, cache)  # ends with a blocking download of the chosen ids
    gpu.synchronize()
    wall = time.perf_counter() - t
    gpu_s = gpu.mark().since(m0)
    tok_s = args.steps / wall
    print(f"[bench] {args.steps} steps in {wall * 1e3:.1f} ms (events {gpu_s * 1e3:.1f} ms): {tok_s:.1f} tok/s",
          file=sys.stderr, flush=True)

    profs = [model.profile_step(cache) for _ in range(args.profile_steps)]
    gemv_s = sum(p["gemv_seconds"] for p in profs)
    gemv_b = sum(p["gemv_bytes"] for p in profs)
    attn_s = sum(p["attention_seconds"] for p in profs)
    attn_b = sum(p["attention_bytes"] for p in profs)
    step_s = sum(p["step_seconds"] for p in profs) / len(profs)
    gemv_gbps = gemv_b / gemv_s / 1e9
    attn_gbps = attn_b / attn_s / 1e9 if attn_s else 0.0
    launches = profs[0]["gemv_launches"]
    print(f"[bench] profiled step {step_s * 1e3:.3f} ms: gemv {gemv_s / len(profs) * 1e3:.3f} ms "
          f"({gemv_gbps:.0f} GB/s over {launches} launches), attention {attn_s / len(profs) * 1e3:.3f} ms "
          f"({attn_gbps:.0f} GB/s), other {sum(p['other_seconds'] for p in profs) / len(profs) * 1e3:.3f} ms",
          file=sys.stderr, flush=True)

    line = {
        "metric": "decode tok/s Qwen3-8B-shape int8 bs=1; GEMV+attn HBM GB/s vs 8 TB/s peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (random-init N(0,0.02) weights quantized int8 g128 on device; uniform random prompt ids)",
        "config": {"workload": "qwen3-8b int8-g128 greedy decode, batch 1, after a 4096-token prompt",
                   "prompt": args.prompt, "batch": 1, "kv_format": args.kv, "layers": shape["layers"],
                   "hidden": shape["hidden"], "heads": shape["heads"], "kv_heads": shape["kv_heads"],
                   "ffn": shape["ffn"], "vocab": shape["vocab"], "group": shape["group"]},
        "roofline": {"bound": "hbm", "kernel": "gemv_i8_mfma (all decode launches, byte-weighted)",
                     "achieved": round(gemv_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gemv_gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "bytes_per_step": gemv_b / len(profs), "launches_per_step": launches},
        "attention": {"achieved_GBps": round(attn_gbps, 1), "frac": round(attn_gbps / HBM_PEAK_GBPS, 4),
                      "seconds_per_step": attn_s / len(profs)},
        "weight_bytes_per_token": weight_bytes(shape),
        "prefill_tok_s": round(args.prompt / prefill_s, 1),
        "gpu": info["name"],
        "first_tokens": tokens[:8].tolist(),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(shape, args.prompt)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
