"""Decode throughput of the Qwen3-8B-shaped int8 model on one MI355X (batch 1).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--prompt 4096] [--kv f16] [--no-cpu]

A step is one greedy decode token: argmax of the last logits, then one pass of the token through 36 layers and the
output head (int8 group-128 weights, f32 scales, f32 activations split to f16 hi/lo on the matrix cores, f32
accumulation). Weights are random-init N(0, 0.02) generated and quantized on the device (no checkpoint); the prompt
is 4096 uniform random ids, prefilled before timing (`prefill_tok_s` times that prefill, after an untimed
1100-token prompt on another cache has loaded every prompt kernel). The timed region is exactly K steps between two stream
synchronizations, with every input already resident in HBM.

One JSON line goes to stdout. `roofline` comes from measurements right after the timed region: profiled decode
steps tag every product and attention launch with its kernel instantiation and algorithmic bytes; then, per kernel,
one decode pass's launches of that kernel alone are captured into a HIP graph and replayed between two events on the
stream they run on, which gives its mean launch duration (kernel time plus the graph's gap to the next launch). The
dominant kernel is the product instantiation with the most time per step; `achieved` is its algorithmic bytes per
launch over its mean launch duration (`kernels` lists every instantiation the same way). `traffic` is that kernel's HBM bytes per launch
from the committed rocprofv3 counter runs (profiles/traffic.json), when present. `cpu_baseline`
times one real decode token of the CPU oracle (oracle/marin_oracle.c, a C restatement of Marin's single-threaded int8
decode) on one core with the same cache format and context, and states the host's core count.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBPS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
TRAFFIC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")


def traffic_of(mode: str, key: str):
    """HBM bytes per launch of `key` in `mode` from the committed rocprofv3 counter runs (profiles/traffic.json:
    FETCH_SIZE and WRITE_SIZE per dispatch, scaled by the copy probe's calibration), or None."""
    if not os.path.exists(TRAFFIC):
        return None
    t = json.load(open(TRAFFIC))
    entry = t.get("modes", {}).get(mode, {}).get(key)
    if entry is None and mode == "decode":
        entry = t.get("kernels", {}).get(key)
    return entry["hbm_bytes_per_launch"] if entry else None


def counter_marker(gpu) -> None:
    """Brackets the dispatches of a `--counters` run: two launches of the copy probe on 1 MiB, which the counter
    summaries (profiles/traffic.json) use to find the region between them."""
    gpu.synchronize()
    gpu.probe_copy(1 << 20, 1)
    gpu.synchronize()


def layer_params(shape: dict) -> int:
    """Weights of the decoder layers' projections (q, k, v, o, gate, up, down)."""
    H, F = shape["hidden"], shape["ffn"]
    qd, kvd = shape["heads"] * shape["head_dim"], shape["kv_heads"] * shape["head_dim"]
    return shape["layers"] * (H * (qd + 2 * kvd) + qd * H + 3 * F * H)


def cpu_baseline(shape: dict, ctx: int, kv_f16: bool) -> dict:
    """One real decode token on the host: the CPU oracle's Qwen3 forward (oracle/marin_oracle.c, a C restatement of
    Marin's int8 decode: Q8Gemv products, AttendOne attention) through every layer and the output head after `ctx`
    cached positions in the GPU line's KV format, on one thread, as Marin decodes one token
    (crates/tensor/src/q8.rs:67-74). Weight values do not change the time, so the model is a constant code pattern
    and a filled cache rather than generated weights and a CPU prompt pass."""
    import ctypes as C

    from oracle import oracle as o
    lib = o.lib
    lib.or_qwen3_time_token.restype = C.c_double
    lib.or_qwen3_time_token.argtypes = [C.c_void_p, C.c_size_t]
    cfg = o._SynthConfig(layers=shape["layers"], hidden=shape["hidden"], heads=shape["heads"],
                         kv_heads=shape["kv_heads"], head_dim=shape["head_dim"], ffn=shape["ffn"],
                         vocab=shape["vocab"], group=shape["group"], capacity=0, eps=shape["eps"],
                         theta=shape["theta"], tied=int(shape["tied"]), kv_f16=int(kv_f16), seed=1)
    t = time.perf_counter()
    sec = lib.or_qwen3_time_token(C.byref(cfg), ctx)
    wall = time.perf_counter() - t
    if sec <= 0:
        return {"value": None, "unit": "tok/s", "cores": 1, "kind": "port",
                "sample": f"oracle token failed ({sec})", "host_cores": os.cpu_count()}
    return {"value": round(1.0 / sec, 4), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"one real {shape['layers']}-layer decode token after {ctx} cached positions "
                      f"({'f16' if kv_f16 else 'f32'} cache), oracle or_qwen3_forward on 1 thread "
                      f"({wall:.1f}s with setup)",
            "seconds_per_token": round(sec, 4), "host_cores": os.cpu_count()}


MOE = {"layers": 48, "hidden": 2048, "experts": 128, "ffn": 768, "k": 8, "group": 128, "heads": 32, "kv_heads": 4,
       "head_dim": 128, "context": 2048}


def moe_attention_us(m, gpu, c, batch, rng, reps) -> float:
    """Per-layer decode attention of the MoE stack: `batch` sequences at `context` positions each, 32 q / 4 kv heads,
    head_dim 128, bf16 pages of 16 positions; one pool per layer (every layer's keys and values distinct, 48 layers
    streamed in turn). Mean microseconds per layer over `reps` passes of the 48 layers."""
    L, kvh, hd, heads, ctx, pt = c["layers"], c["kv_heads"], c["head_dim"], c["heads"], c["context"], 16
    per_seq = -(-ctx // pt)
    block = _bf16(rng.standard_normal((64, 2 * pt * kvh * hd)))
    tables = np.arange(batch * per_seq, dtype=np.uint32).reshape(batch, per_seq)
    ctxs = np.full(batch, ctx, np.uint32)
    pools = []
    for l in range(L):
        pool = m.PagePool(gpu, batch * per_seq, pt, kvh, hd, m.KvFormat.BF16)
        for pid in range(batch * per_seq):
            pool.write_page(pid, block[(pid + l) % 64])
        pools.append(pool)
    q = gpu.typed(m.Dtype.BF16, host=_bf16(rng.standard_normal((batch, heads, hd))))
    out = gpu.typed(m.Dtype.BF16, batch * heads * hd)
    for pool in pools:
        pool.attention(q, tables, ctxs, heads, out)
    gpu.synchronize()
    a = gpu.mark()
    for _ in range(reps):
        for pool in pools:
            pool.attention(q, tables, ctxs, heads, out)
    b = gpu.mark()
    return b.since(a) / (reps * L) * 1e6


def bench_moe(m, args) -> int:
    """Config 4: per layer, router logits from random-init N(0, 0.02) router weights and N(0, 1) hidden states
    (host), softmax top-8 routing on the GPU, then the timed region: the 48 layers' expert FFNs (RMSNorm, stacked
    gate_up product over the selected experts' tiles with SiLU(gate) * up, grouped down product weighted into the
    residual) captured as one HIP graph and replayed. Algorithmic bytes per layer: codes and f32 scales of the
    union of the experts the batch selects (each read once by an ideal kernel)."""
    c = MOE
    gpu = m.Gpu()
    H, E, F, K, L, G = c["hidden"], c["experts"], c["ffn"], c["k"], c["layers"], c["group"]
    print(f"[bench] moe: {L} layers, {E} experts x ffn {F}, top-{K}, hidden {H}, int8 g{G}", file=sys.stderr,
          flush=True)
    t = time.perf_counter()
    gate_ups = [gpu.quantized_synthetic(E * 2 * F, H, G, args.seed, 2 * l) for l in range(L)]
    downs = [gpu.quantized_synthetic(E * H, F, G, args.seed, 2 * l + 1) for l in range(L)]
    gpu.synchronize()
    print(f"[bench] experts built in {time.perf_counter() - t:.1f}s", file=sys.stderr, flush=True)
    expert_bytes = 3 * F * H * (1 + 4 / G)
    rng = np.random.default_rng(args.seed)
    norm = gpu.upload((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    results = {}
    for batch in (1, 8):
        x = rng.standard_normal((batch, H)).astype(np.float32)
        router = (0.02 * rng.standard_normal((L, E, H))).astype(np.float32)
        logits = np.einsum("leh,bh->lbe", router, x).astype(np.float32)
        ids = gpu.typed(m.Dtype.U32, L * batch * K)
        wts = gpu.zeros(L * batch * K)
        for l in range(L):
            li, lw = gpu.typed(m.Dtype.U32, batch * K), gpu.zeros(batch * K)
            gpu.moe_route(gpu.upload(logits[l].ravel()), batch, E, K, True, li, lw)
            gpu.copy_into_range(lw, wts, l * batch * K)
            host_ids = gpu.download_typed(li)
            results.setdefault(batch, {"ids": []})["ids"].append(host_ids)
        ids = gpu.typed(m.Dtype.U32, host=np.concatenate(results[batch]["ids"]))
        act = gpu.zeros(batch * K * F)
        out = gpu.zeros(batch * H)
        xb = gpu.upload(x.ravel())
        if args.counters:
            # eager (MARIN_NO_GRAPH): one untimed stack then one timed stack of the L layers between the markers
            counter_marker(gpu)
            gpu.moe_stack_time(gate_ups, downs, xb, norm, 1e-6, ids, wts, batch, E, K, act, out, reps=1)
            counter_marker(gpu)
            print(json.dumps({"counters": "moe", "batch": batch, "stacks": 2, "layers": L,
                              "experts_read_per_layer": sum(len(np.unique(i)) for i in results[batch]["ids"]) / L}))
            return 0
        sec = gpu.moe_stack_time(gate_ups, downs, xb, norm, 1e-6, ids, wts, batch, E, K, act, out,
                                 reps=max(args.steps // 16, 5))
        reps = max(args.steps // 16, 5)
        parts = [gpu.moe_stack_time(gate_ups, downs, xb, norm, 1e-6, ids, wts, batch, E, K, act, out, reps=reps,
                                    part=p) for p in (1, 2)]
        union = sum(len(np.unique(i)) for i in results[batch]["ids"])
        selected = L * batch * K
        algo = union * expert_bytes
        results[batch] = {"us_per_stack": round(sec * 1e6, 1), "us_per_layer": round(sec * 1e6 / L, 2),
                          "experts_read_per_layer": round(union / L, 2), "selections_per_layer": selected // L,
                          "algorithmic_bytes_per_stack": round(algo), "GBps": round(algo / sec / 1e9, 1),
                          "GBps_per_selection": round(selected * expert_bytes / sec / 1e9, 1),
                          "tok_s_expert_stack": round(batch / sec, 1),
                          "gate_up_us_per_layer": round(parts[0] * 1e6 / L, 2),
                          "down_us_per_layer": round(parts[1] * 1e6 / L, 2),
                          "gate_up_GBps": round(union * 2 * F * H * (1 + 4 / G) / parts[0] / 1e9, 1),
                          "down_GBps": round(union * F * H * (1 + 4 / G) / parts[1] / 1e9, 1)}
        att_us = moe_attention_us(m, gpu, c, batch, rng, reps)
        results[batch]["attention_us_per_layer"] = round(att_us, 2)
        results[batch]["layer_us"] = round(sec * 1e6 / L + att_us, 2)
        print(f"[bench] moe batch {batch}: attention at ctx {c['context']}: {att_us:.1f} us/layer", file=sys.stderr,
              flush=True)
        print(f"[bench] moe batch {batch}: {sec * 1e6:.1f} us per {L}-layer stack, {union / L:.1f} experts/layer, "
              f"{algo / sec / 1e9:.0f} GB/s (gate_up {parts[0] * 1e6 / L:.1f} us/layer, down "
              f"{parts[1] * 1e6 / L:.1f} us/layer)", file=sys.stderr, flush=True)
    r1 = results[1]
    line = {
        "metric": "grouped-expert GEMV GB/s, Qwen3-30B-A3B-shape int8 MoE layer stack",
        "value": r1["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": max(args.steps // 16, 5), "warmup": 1,
        "ms_per_step": round(r1["us_per_stack"] / 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (random-init N(0,0.02) experts quantized int8 g128 on device; N(0,1) hidden states; "
                "random-init router weights)",
        "config": {"workload": "qwen3-30b-a3b expert FFN stack (48 layers, 128 experts x ffn 768, top-8, hidden "
                               "2048), batch 1; batch 8 under batches; each layer's decode attention at 2048 "
                               "positions (32 q / 4 kv heads) timed beside it (attention_us_per_layer)", **c},
        "roofline": {"bound": "hbm", "kernel": "gemv_decode (tile-mapped) + expert_down, per layer",
                     "achieved": r1["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(r1["GBps"] / HBM_PEAK_GBPS, 4), "traffic": traffic_of("moe", "expert layer"),
                     "bytes_per_launch": round(r1["algorithmic_bytes_per_stack"] / L)},
        "batches": results,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_batch(m, args) -> int:
    """Config 3 at batch N: N sequences, each with its own `--prompt`-token prompt of uniform random ids prefilled
    through its own cache, then decoded together (one greedy token per sequence per step: every product over the N
    tokens, one attention launch over all sequences, the step replayed as a HIP graph). value = N x K / wall seconds
    of K timed steps."""
    from marin_amd.qwen3 import SHAPES, Qwen3, weight_bytes

    shape = SHAPES["qwen3-8b"]
    fmt = {"f32": m.KvFormat.F32, "f16": m.KvFormat.F16, "bf16": m.KvFormat.BF16}[args.kv]
    B = args.batch
    print(f"[bench] qwen3-8b int8 g128 batch {B}, prompt {args.prompt}, kv {args.kv}, warmup {args.warmup}, steps "
          f"{args.steps}", file=sys.stderr, flush=True)
    gpu = m.Gpu()
    model = Qwen3(gpu, shape, seed=args.seed)
    batch = model.new_batch(B, args.prompt + args.warmup + args.steps + 8, fmt)
    rng = np.random.default_rng(args.seed)
    t = time.perf_counter()
    for i in range(B):
        batch.prefill(i, rng.integers(0, shape["vocab"], args.prompt, dtype=np.uint32))
    gpu.synchronize()
    prefill_s = time.perf_counter() - t
    print(f"[bench] {B} prompts in {prefill_s:.2f}s", file=sys.stderr, flush=True)
    if args.counters:
        batch.decode(1)  # one step first, so the counted step is not the one that opens new KV slabs
        counter_marker(gpu)
        batch.decode(1)
        counter_marker(gpu)
        print(json.dumps({"counters": "batch", "batch": B, "steps": 1}))
        return 0
    batch.decode(args.warmup)
    gpu.synchronize()
    t = time.perf_counter()
    toks = batch.decode(args.steps)  # ends with a blocking download of the chosen ids
    gpu.synchronize()
    wall = time.perf_counter() - t
    tok_s = B * args.steps / wall
    print(f"[bench] batch {B}: {args.steps} steps in {wall * 1e3:.1f} ms: {tok_s:.1f} tok/s aggregate, "
          f"{wall / args.steps * 1e3:.3f} ms per step", file=sys.stderr, flush=True)
    # algorithmic bytes of one step: the weights once, plus every sequence's cached keys and values at the mean context
    # of the timed steps
    kv_el = {"f32": 4, "f16": 2, "bf16": 2}[args.kv]
    mean_ctx = args.prompt + args.warmup + args.steps / 2
    step_bytes = weight_bytes(shape) + B * mean_ctx * shape["layers"] * shape["kv_heads"] * shape["head_dim"] * 2 * kv_el
    step_gbps = step_bytes / (wall / args.steps) / 1e9
    line = {
        "metric": f"decode tok/s Qwen3-8B-shape int8 bs={B} (aggregate over the batch)",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (random-init N(0,0.02) weights quantized int8 g128 on device; uniform random prompt ids)",
        "config": {"workload": f"qwen3-8b int8-g128 greedy decode, batch {B}, each sequence after a "
                               f"{args.prompt}-token prompt", "prompt": args.prompt, "batch": B, "kv_format": args.kv,
                   "layers": shape["layers"], "hidden": shape["hidden"], "ffn": shape["ffn"], "vocab": shape["vocab"]},
        "roofline": {"bound": "hbm", "kernel": "one decode step (every launch of the step)", "achieved": round(step_gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(step_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_of("batch", "decode step"), "bytes_per_launch": round(step_bytes)},
        "weight_GBps": round(weight_bytes(shape) / (wall / args.steps) / 1e9, 1),
        "prefill_tok_s": round(B * args.prompt / prefill_s, 1),
        "first_tokens": toks[:, :4].tolist(),
    }
    print(json.dumps(line), flush=True)
    return 0


def _bf16(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bench_linear(m, args) -> int:
    """Config 1: the isolated quantized linear layer at decode shapes. Weights N(0, 0.02) quantized int8 on the device
    (int4: random codes, constant scales; the timing does not depend on the values), group 128, f32 scales;
    activations bf16 N(0, 1) of M tokens, bf16 out. Each case cycles through copies of its matrix totalling more than
    the 256 MB last-level cache, so every product streams its weights from HBM; `reps` products are one HIP graph
    replayed between two events. Bytes per product: N K (1 or 1/2) + N (K / 128) 4 +
    M K 2 + M N 2. value: the int8 M = 1 cases' bytes over their time."""
    gpu = m.Gpu()
    rng = np.random.default_rng(args.seed)
    shapes = [(4096, 4096), (4096, 12288), (12288, 4096), (4096, 151936)]  # (K, N)
    if args.counters:
        # one eager product per int8 M = 1 shape, in this order, each between two markers, for rocprofv3 counter runs
        for K, N in shapes:
            w = gpu.quantized_synthetic(N, K, 128, args.seed, 0)
            x = gpu.typed(m.Dtype.BF16, host=_bf16(rng.standard_normal((1, K))))
            out = gpu.typed(m.Dtype.BF16, N)
            counter_marker(gpu)
            gpu.matmul_quant_bf16(w, x, 1, out)
            counter_marker(gpu)
            del w
        print(json.dumps({"counters": "linear", "order": [f"int8 K={K} N={N} M=1" for K, N in shapes]}))
        return 0
    cases = []
    for bits in (8, 4):
        for K, N in shapes:
            wbytes = N * K * (1 if bits == 8 else 0.5) + N * (K // 128) * 4
            copies = max(2, int(np.ceil(300e6 / wbytes)))
            if bits == 8:
                mats = [gpu.quantized_synthetic(N, K, 128, args.seed, i) for i in range(copies)]
            else:
                codes = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
                scales = np.full(N * (K // 128), 0.01, np.float32)
                mats = [gpu.upload_quantized(N, K, 4, 128, codes, scales) for _ in range(copies)]
                del codes
            for M in (1, 4, 8):
                x = gpu.typed(m.Dtype.BF16, host=_bf16(rng.standard_normal((M, K))))
                out = gpu.typed(m.Dtype.BF16, M * N)
                sec = gpu.time_matmul_bf16(mats, x, M, out, reps=max(2 * copies, 100))
                nbytes = wbytes + M * K * 2 + M * N * 2
                cases.append({"bits": bits, "K": K, "N": N, "M": M, "us": round(sec * 1e6, 2),
                              "GBps": round(nbytes / sec / 1e9, 1), "frac": round(nbytes / sec / 1e9 / HBM_PEAK_GBPS, 4)})
                print(f"[bench] linear int{bits} K={K} N={N} M={M}: {sec * 1e6:.2f} us, {nbytes / sec / 1e9:.0f} GB/s",
                      file=sys.stderr, flush=True)
            del mats
            gpu.synchronize()
    one = [c for c in cases if c["bits"] == 8 and c["M"] == 1]
    tot_b = sum(c["N"] * c["K"] + c["N"] * (c["K"] // 128) * 4 + c["K"] * 2 + c["N"] * 2 for c in one)
    tot_s = sum(c["us"] for c in one) * 1e-6
    gbps = tot_b / tot_s / 1e9
    line = {
        "metric": "isolated int8/int4 g128 linear, decode shapes, HBM GB/s", "value": round(gbps, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": 100, "warmup": 1, "ms_per_step": round(tot_s / len(one) * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (int8: N(0,0.02) weights quantized on device; int4: random codes; bf16 N(0,1) inputs)",
        "config": {"workload": "config 1: (K, N) in {(4096,4096), (4096,12288), (12288,4096), (4096,151936)}, "
                               "M in {1, 4, 8}, int8 and int4 group 128, bf16 in and out; value over int8 M=1"},
        "roofline": {"bound": "hbm", "kernel": "gemv_decode (int8, M = 1, the four shapes)", "achieved": round(gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_of("linear", "int8 M=1, four shapes"),
                     "bytes_per_launch": round(tot_b / len(one))},
        "cases": cases,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_prefill(m, args) -> int:
    """The prompt GEMM alone (prefill's products): each 8B projection shape times 512 tokens (one prompt chunk), f32
    activations N(0, 1) and f32 out, weights N(0, 0.02) quantized int8 g128 on the device; `reps` eager products
    between two events (each with its activation-limb pass). Useful work 2 N K T int8 operations per product; the
    matrix cores execute 3 limbs of it (the activations' 22-bit fixed point). value: useful int8 TOP/s over the four
    shapes."""
    gpu = m.Gpu()
    rng = np.random.default_rng(args.seed)
    T = 512
    shapes = [("qkv", 4096, 6144), ("o", 4096, 4096), ("gate_up", 4096, 24576), ("down", 12288, 4096)]
    cases, tot_ops, tot_s = [], 0.0, 0.0
    for name, K, N in shapes:
        w = gpu.quantized_synthetic(N, K, 128, args.seed, 0)
        x = gpu.upload(rng.standard_normal(T * K).astype(np.float32))
        out = gpu.zeros(T * N)
        for _ in range(3):
            gpu.matmul_quant(w, x, T, out)
        gpu.synchronize()
        if args.counters:
            counter_marker(gpu)
            gpu.matmul_quant(w, x, T, out)
            counter_marker(gpu)
            del w
            continue
        reps = 20
        a = gpu.mark()
        for _ in range(reps):
            gpu.matmul_quant(w, x, T, out)
        sec = gpu.mark().since(a) / reps
        ops = 2.0 * N * K * T
        tot_ops += ops
        tot_s += sec
        cases.append({"matrix": name, "K": K, "N": N, "tokens": T, "us": round(sec * 1e6, 1),
                      "useful_int8_TOPs": round(ops / sec / 1e12, 1),
                      "mfma_frac": round(3 * ops / sec / 1e12 / INT8_PEAK_TOPS, 4)})
        print(f"[bench] prefill product {name} {N}x{K} x {T} tokens: {sec * 1e6:.1f} us, {ops / sec / 1e12:.0f} useful "
              f"int8 TOP/s", file=sys.stderr, flush=True)
        del w
        gpu.synchronize()
    if args.counters:
        print(json.dumps({"counters": "prefill", "order": [c[0] for c in shapes]}))
        return 0
    tops = tot_ops / tot_s / 1e12
    line = {
        "metric": "prompt GEMM useful int8 TOP/s (Qwen3-8B projection shapes, 512-token chunk)", "value": round(tops, 1),
        "unit": "TOP/s", "n_gpus": 1, "steps": 20, "warmup": 3, "ms_per_step": round(tot_s / len(shapes) * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (N(0,0.02) weights quantized int8 g128 on device; N(0,1) f32 activations)",
        "config": {"workload": "prefill products: qkv, o, gate_up, down of Qwen3-8B at 512 tokens, f32 in and out"},
        "roofline": {"bound": "mfma", "kernel": "gemm_prompt (+ its quantize_act pass)", "achieved": round(3 * tops, 1),
                     "peak": INT8_PEAK_TOPS, "unit": "TOP/s", "frac": round(3 * tops / INT8_PEAK_TOPS, 4),
                     "traffic": None, "note": "achieved counts the three limbs the matrix cores execute"},
        "cases": cases,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_paged(m, args) -> int:
    """Config 2: batched paged GQA decode attention. Batch 16, 32 q / 8 kv heads, head_dim 128, bf16 q/k/v N(0,1),
    pages of 16 positions; contexts uniform in [512, 8192] (seeded); one pool of exactly the pages needed, dealt to
    the sequences in a seeded shuffled order; scale 1/sqrt(128), the query at the last position. Bytes per call:
    sum of contexts x 8 kv heads x 128 x 2 (keys and values) x 2 B, plus q and out. value: bytes / mean call time
    over `--steps` calls between two events."""
    gpu = m.Gpu()
    rng = np.random.default_rng(args.seed)
    batch, heads, kvh, hd, pt = 16, 32, 8, 128, 16
    ctx = rng.integers(512, 8193, size=batch).astype(np.uint32)
    pages_each = [-(-int(c) // pt) for c in ctx]
    total = sum(pages_each)
    perm = rng.permutation(total)
    # copies of the pool totalling at least twice the 256 MB last-level cache, used in turn, so every call streams its
    # keys and values from HBM
    page_bytes = 2 * pt * kvh * hd * 2
    npools = max(2, -(-(2 * 256 << 20) // (total * page_bytes)))
    pools = [m.PagePool(gpu, total, pt, kvh, hd, m.KvFormat.BF16) for _ in range(npools)]
    stride = max(pages_each)
    tables = np.zeros((batch, stride), np.uint32)
    block = _bf16(rng.standard_normal((64, 2 * pt * kvh * hd)))  # 64 distinct pages of random rows, dealt cyclically
    at = 0
    for b in range(batch):
        for i in range(pages_each[b]):
            pid = int(perm[at])
            tables[b, i] = pid
            for pool in pools:
                pool.write_page(pid, block[at % 64])
            at += 1
    q = gpu.typed(m.Dtype.BF16, host=_bf16(rng.standard_normal((batch, heads, hd))))
    out = gpu.typed(m.Dtype.BF16, batch * heads * hd)
    if args.counters:
        counter_marker(gpu)
        pools[0].attention(q, tables, ctx, heads, out)
        counter_marker(gpu)
        print(json.dumps({"counters": "paged", "order": ["attention_decode", "attention_decode_merge"]}))
        return 0
    for i in range(2 * npools):
        pools[i % npools].attention(q, tables, ctx, heads, out)
    gpu.synchronize()
    steps = max(args.steps, 20) // npools * npools
    a = gpu.mark()
    for i in range(steps):
        pools[i % npools].attention(q, tables, ctx, heads, out)
    b = gpu.mark()
    sec = b.since(a) / steps
    nbytes = int(ctx.sum()) * kvh * hd * 2 * 2 + 2 * batch * heads * hd * 2
    gbps = nbytes / sec / 1e9
    print(f"[bench] paged attention batch {batch}: {sec * 1e6:.1f} us per call, {nbytes / 1e6:.1f} MB, {gbps:.0f} GB/s",
          file=sys.stderr, flush=True)
    line = {
        "metric": "batched paged GQA decode attention HBM GB/s (batch 16, ragged contexts)", "value": round(gbps, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": 5, "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": f"synthetic (bf16 N(0,1) q/k/v; 64 distinct random pages dealt over the pool; {npools} copies of the "
                f"pool ({npools * total * page_bytes / 1e6:.0f} MB) used in turn)",
        "config": {"workload": "config 2: batch 16, 32 q / 8 kv heads, head_dim 128, 16-position pages, contexts "
                               "uniform in [512, 8192], shuffled page tables from one pool", "contexts": ctx.tolist()},
        "roofline": {"bound": "hbm", "kernel": "attention_decode + attention_decode_merge", "achieved": round(gbps, 1),
                     "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic_of("paged", "attention call"), "bytes_per_launch": nbytes},
        "bytes_per_call": nbytes,
    }
    print(json.dumps(line), flush=True)
    return 0


SUB_MODES = [("linear", ["--linear"]), ("paged", ["--paged"]), ("moe", ["--moe"]), ("batch8", ["--batch", "8"]),
             ("prefill", ["--prefill"])]


def run_sub_benchmarks(args) -> dict:
    """The other configurations, each in a child process of its own (before this process touches the GPU), so that
    the default run's one JSON line carries them too: per mode its metric, value, unit, time per step and roofline."""
    import subprocess
    res = {}
    for name, flags in SUB_MODES:
        cmd = [sys.executable, "-u", os.path.abspath(__file__), *flags, "--no-cpu", "--seed", str(args.seed)]
        print(f"[bench] sub-benchmark {name}: {' '.join(flags)}", file=sys.stderr, flush=True)
        try:
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
        except subprocess.TimeoutExpired:
            res[name] = {"error": "timed out"}
            continue
        lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
        if r.returncode != 0 or not lines:
            res[name] = {"error": f"exit {r.returncode}", "stderr_tail": r.stderr[-400:]}
            continue
        d = json.loads(lines[-1])
        keep = {k: d[k] for k in ("metric", "value", "unit", "ms_per_step", "dtype", "roofline", "config") if k in d}
        if name == "moe":
            keep["batches"] = {b: {k: v[k] for k in ("us_per_layer", "GBps", "attention_us_per_layer", "layer_us")}
                               for b, v in d["batches"].items()}
        if name == "linear":
            keep["cases"] = [{k: c[k] for k in ("bits", "K", "N", "M", "us", "GBps")} for c in d["cases"]]
        if name == "prefill":
            keep["cases"] = d["cases"]
        res[name] = keep
    return res


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
    ap.add_argument("--no-timing", action="store_true",
                    help="skip the per-kernel graph timing (for rocprofv3 counter runs, which only need the decode "
                         "dispatches); mean launch durations then come from the profiled steps' events")
    ap.add_argument("--probe-copy", type=float, default=0.0, metavar="MB",
                    help="only run the bandwidth probe: copies of MB megabytes (for counter calibration), then exit")
    ap.add_argument("--batch", type=int, default=1,
                    help="config 3 at batch N (2..8): N sequences of the prompt length decoded together; one JSON line "
                         "with the aggregate tok/s")
    ap.add_argument("--linear", action="store_true",
                    help="config 1 instead: the isolated quantized linear shapes at M 1, 4, 8, int8 and int4, bf16 in "
                         "and out; one JSON line")
    ap.add_argument("--paged", action="store_true",
                    help="config 2 instead: batched paged GQA decode attention, batch 16, ragged contexts; one JSON "
                         "line")
    ap.add_argument("--moe", action="store_true",
                    help="config 4 instead: the Qwen3-30B-A3B-shaped expert FFN stack at batch 1 and 8 (grouped-expert "
                         "GEMV GB/s), one JSON line")
    ap.add_argument("--prefill", action="store_true",
                    help="the prompt GEMM alone at the 8B projection shapes x 512 tokens (useful int8 TOP/s); one JSON "
                         "line")
    ap.add_argument("--counters", action="store_true",
                    help="for rocprofv3 --pmc runs: set the mode's inputs up, then launch its measured work once, "
                         "eagerly, between two copy-probe markers, and exit (no timing, no JSON result line)")
    ap.add_argument("--headline-only", action="store_true",
                    help="the default run without the other configurations' sub-benchmarks")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch the decode step's kernels one by one instead of replaying a HIP graph (for tracers)")
    args = ap.parse_args()
    if args.no_graph or args.counters:
        os.environ["MARIN_NO_GRAPH"] = "1"
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the one-GPU throughput is the reported value", file=sys.stderr)
        return 2

    headline = not (args.moe or args.linear or args.paged or args.prefill or args.batch > 1 or args.probe_copy)
    subs = None
    if headline and not (args.headline_only or args.counters or args.no_graph or args.no_timing):
        subs = run_sub_benchmarks(args)

    import marin_amd as m
    from marin_amd.qwen3 import SHAPES, Qwen3, weight_bytes

    if args.probe_copy:
        nbytes = int(args.probe_copy * 1e6) // 16 * 16
        sec = m.Gpu().probe_copy(nbytes, 50)
        print(json.dumps({"probe": "copy", "bytes": nbytes, "seconds": sec,
                          "GBps_read_plus_write": round(2 * nbytes / sec / 1e9, 1)}), flush=True)
        return 0

    if args.moe:
        return bench_moe(m, args)
    if args.linear:
        return bench_linear(m, args)
    if args.paged:
        return bench_paged(m, args)
    if args.prefill:
        return bench_prefill(m, args)
    if args.batch > 1:
        return bench_batch(m, args)

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
    # an untimed 1100-token prompt first, on a cache of its own: every prompt kernel (chunks of 512, spans past
    # 1024 positions) is loaded and the scratch is allocated before the timed prefill
    warm = min(1100, args.prompt)
    model.forward(prompt[:warm], model.new_cache(warm + 1, fmt))
    gpu.synchronize()
    t = time.perf_counter()
    model.forward(prompt, cache)
    gpu.synchronize()
    prefill_s = time.perf_counter() - t
    print(f"[bench] weights {build_s:.1f}s, prefill {prefill_s:.2f}s", file=sys.stderr, flush=True)

    if args.counters:
        model.decode(1, cache)  # one step first, so the counted step is not the one that opens a new KV slab
        counter_marker(gpu)
        model.decode(1, cache)
        counter_marker(gpu)
        print(json.dumps({"counters": "decode", "steps": 1}))
        return 0
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

    # Per-launch durations, each product and attention launch bracketed by its own two events on the stream it runs
    # on (one decode step per profiled step, launched eagerly so the events can sit between the kernels).
    recs = []
    for _ in range(args.profile_steps):
        recs += model.profile_launches(cache)
    kernels = {}
    for kind, name, nbytes, sec in recs:
        if kind == 0 and not name:
            continue
        k = kernels.setdefault(name, {"kind": ["attention merge", "product", "attention"][kind], "launches": 0,
                                      "bytes": 0.0, "seconds": 0.0})
        k["launches"] += 1
        k["bytes"] += nbytes
        k["seconds"] += sec
    steps_p = args.profile_steps
    summary = {}
    for name, k in kernels.items():
        # mean launch duration: graph replays of one pass's launches of this kernel alone, between two events
        if args.no_timing:
            sec, n = k["seconds"] / k["launches"], k["launches"] // steps_p
        else:
            sec, n = model.time_kernel(cache, name, reps=20)
        summary[name] = {"kind": k["kind"], "launches_per_step": k["launches"] // steps_p,
                         "bytes_per_launch": round(k["bytes"] / k["launches"]),
                         "mean_launch_us": round(sec * 1e6, 3),
                         "GBps": round(k["bytes"] / k["launches"] / sec / 1e9, 1),
                         "us_per_step": round(sec * n * 1e6, 1),
                         "eager_event_us": round(k["seconds"] / k["launches"] * 1e6, 3)}
    dom = max((n for n in summary if summary[n]["kind"] == "product"), key=lambda n: summary[n]["us_per_step"])
    dk = summary[dom]
    gemv_b = sum(k["bytes"] for k in kernels.values() if k["kind"] == "product") / steps_p
    attn_b = sum(k["bytes"] for k in kernels.values() if k["kind"] == "attention") / steps_p
    for name, k in sorted(summary.items(), key=lambda kv: -kv[1]["us_per_step"]):
        print(f"[bench] {name}: {k['launches_per_step']} launches/step, {k['mean_launch_us']:.2f} us each, "
              f"{k['GBps']:.0f} GB/s, {k['us_per_step']:.0f} us/step", file=sys.stderr, flush=True)
    traffic = traffic_of("decode", dom)

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
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": dk["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(dk["GBps"] / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "bytes_per_launch": dk["bytes_per_launch"], "mean_launch_us": dk["mean_launch_us"],
                     "launches_per_step": dk["launches_per_step"]},
        "kernels": summary,
        "step_algorithmic_GBps": round((gemv_b + attn_b) / (wall / args.steps) / 1e9, 1),
        "weight_bytes_per_token": weight_bytes(shape),
        "prefill_tok_s": round(args.prompt / prefill_s, 1),
        # useful int8 work of the prompt's layer products (2 x layer weights x tokens) per second
        "prefill_int8_TOPs": round(2.0 * layer_params(shape) * args.prompt / prefill_s / 1e12, 1),
        "gpu": info["name"],
        "first_tokens": tokens[:8].tolist(),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(shape, args.prompt, args.kv == "f16")
    if subs is not None:
        line["configs"] = subs
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
