"""ctypes view of the C oracle (oracle/marin_oracle.c).

TEST INFRASTRUCTURE: only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this module,
and only as the checker or as the timed host baseline. Nothing in ``marin_amd`` may import it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libmarin_oracle.so")


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    P = C.c_void_p
    sz = C.c_size_t
    sig = {
        "or_set_threads": (None, [C.c_int]),
        "or_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "or_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "or_f32_to_f16_sat": (C.c_uint16, [C.c_float]),
        "or_f16_to_f32": (C.c_float, [C.c_uint16]),
        "or_quantize": (C.c_long, [P, sz, sz, C.c_int, sz, P, P]),
        "or_dequantize_row": (None, [P, P, sz, C.c_int, sz, sz, P]),
        "or_q8_gemv": (None, [P, P, P, P, sz, sz, sz]),
        "or_matmul_dot": (None, [P, P, P, P, sz, sz, C.c_int, sz, sz]),
        "or_dot": (C.c_float, [P, P, sz]),
        "or_exp": (C.c_float, [C.c_float]),
        "or_rms_norm_rows": (None, [P, sz, P, sz, C.c_float]),
        "or_rope_tokens": (None, [P, sz, sz, sz, sz, C.c_float]),
        "or_silu_mul": (None, [P, P, sz]),
        "or_softmax": (None, [P, sz]),
        "or_attention": (None, [P, P, P, P, sz, sz, sz, sz, sz]),
        "or_attention_f64": (None, [P, P, P, P, sz, sz, sz, sz, sz]),
        "or_argmax": (C.c_uint32, [P, sz]),
        "or_synth_bf16": (C.c_uint16, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_double]),
        "or_synth_fill": (None, [C.c_uint64, C.c_uint64, C.c_double, P, sz]),
        "or_synth_fill_at": (None, [C.c_uint64, C.c_uint64, C.c_double, C.c_uint64, P, sz]),
        "or_qwen3_forward": (C.c_int, [P, P, sz, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def set_threads(n: int) -> None:
    lib.or_set_threads(n)


class QuantError(ValueError):
    pass


def quantize(bits16: np.ndarray, rows: int, cols: int, bits: int, group: int):
    """tensor::quantize. Returns (codes u8, scales f32)."""
    bits16 = np.ascontiguousarray(bits16, dtype=np.uint16)
    if bits16.size != rows * cols or bits16.size == 0:
        raise QuantError(f"matrix to quantize: expected {rows * cols}, got {bits16.size}")
    row_bytes = cols if bits == 8 else (cols + 1) // 2
    codes = np.zeros(rows * row_bytes, np.uint8)
    scales = np.zeros(rows * (cols // group if group else 0), np.float32)
    rc = lib.or_quantize(_p(bits16), rows, cols, bits, group, _p(codes), _p(scales))
    if rc == -2:
        raise QuantError(f"{cols} columns are not a multiple of the group size {group}, or a bad group")
    if rc >= 0:
        raise QuantError(f"row {rc} has a NaN or infinite weight")
    return codes, scales


def dequantize(codes, scales, rows, cols, bits, group) -> np.ndarray:
    out = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        lib.or_dequantize_row(_p(codes), _p(scales), cols, bits, group, r, _p(out[r]))
    return out


def q8_gemv(codes, scales, x, rows, cols, group) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(rows, np.float32)
    lib.or_q8_gemv(_p(codes), _p(scales), _p(x), _p(out), rows, cols, group)
    return out


def matmul_dot(codes, scales, x, rows, cols, bits, group, tokens) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(tokens * rows, np.float32)
    lib.or_matmul_dot(_p(codes), _p(scales), _p(x), _p(out), rows, cols, bits, group, tokens)
    return out


def bf16_bits(values) -> np.ndarray:
    """f32 -> bf16 by truncation, as the reference tests build their inputs (`to_bits() >> 16`)."""
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_to_f32(bits16) -> np.ndarray:
    return (np.asarray(bits16, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_rne(values) -> np.ndarray:
    u = np.asarray(values, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def values(count: int, seed: int) -> np.ndarray:
    """Deterministic values in [-1, 1): the LCG of cuda/tests/common/mod.rs:15-25 and tensor/tests/quant.rs:8-19."""
    out = np.empty(count, np.float32)
    state = seed & 0xFFFFFFFFFFFFFFFF
    a, c, m = 6364136223846793005, 1442695040888963407, (1 << 64) - 1
    # vectorised by blocks would change nothing; a plain loop is fast enough at test sizes
    for i in range(count):
        state = (state * a + c) & m
        out[i] = np.float32(np.float32(state >> 40) / np.float32(16777216.0)) * np.float32(2.0) - np.float32(1.0)
    return out


def synth(seed: int, stream: int, count: int, std: float = 0.02, start: int = 0) -> np.ndarray:
    """Values start .. start + count - 1 of a synthetic stream (bf16 bits)."""
    out = np.zeros(count, np.uint16)
    lib.or_synth_fill_at(seed, stream, std, start, _p(out), count)
    return out


def rms_norm_rows(x, weight, eps):
    x = np.array(x, np.float32, copy=True).ravel()
    w = np.ascontiguousarray(weight, np.float32)
    lib.or_rms_norm_rows(_p(x), x.size, _p(w), w.size, eps)
    return x


def rope_tokens(x, token_dim, head_size, start, theta):
    x = np.array(x, np.float32, copy=True).ravel()
    lib.or_rope_tokens(_p(x), x.size, token_dim, head_size, start, theta)
    return x


def silu_mul(gate, up):
    g = np.array(gate, np.float32, copy=True).ravel()
    u = np.ascontiguousarray(up, np.float32).ravel()
    lib.or_silu_mul(_p(g), _p(u), g.size)
    return g


def softmax(x):
    x = np.array(x, np.float32, copy=True).ravel()
    lib.or_softmax(_p(x), x.size)
    return x


def attention(q, keys, vals, heads, kv_heads, head_dim, start, tokens, f64=False):
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    vals = np.ascontiguousarray(vals, np.float32)
    out = np.zeros(tokens * heads * head_dim, np.float32)
    fn = lib.or_attention_f64 if f64 else lib.or_attention
    fn(_p(q), _p(keys), _p(vals), _p(out), heads, kv_heads, head_dim, start, tokens)
    return out


def argmax(v) -> int:
    v = np.ascontiguousarray(v, np.float32)
    return int(lib.or_argmax(_p(v), v.size))


# ---- Qwen3 forward (ctypes mirrors of or_matrix / or_layer / or_qwen3 in marin_oracle.h) ----
class _Matrix(C.Structure):
    _fields_ = [("rows", C.c_size_t), ("cols", C.c_size_t), ("group", C.c_size_t), ("bits", C.c_int),
                ("codes", C.c_void_p), ("scales", C.c_void_p), ("dense", C.c_void_p)]


class _Layer(C.Structure):
    _fields_ = [(n, _Matrix) for n in ("q", "k", "v", "o", "gate", "up", "down")] + [
        (n, C.c_void_p) for n in ("input_norm", "post_norm", "q_norm", "k_norm")]


class _Qwen3(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in ("layers", "hidden", "heads", "kv_heads", "head_dim", "ffn", "vocab",
                                          "capacity")] + [
        ("eps", C.c_float), ("theta", C.c_float), ("kv_f16", C.c_int), ("layer", C.c_void_p),
        ("embed", _Matrix), ("lm_head", _Matrix), ("final_norm", C.c_void_p),
        ("keys", C.c_void_p), ("values", C.c_void_p), ("len", C.c_size_t)]


class Qwen3Oracle:
    """Qwen3 forward on the CPU oracle. ``weights`` maps HF tensor names to f32 arrays (dense f64-dot path) unless
    ``group`` is given, in which case every matrix is quantized int8 with that group from its bf16 bits."""

    def __init__(self, cfg: dict, weights: dict, capacity: int, group: int | None = None, kv_f16: bool = False):
        self._keep = []
        self.cfg = cfg
        L = cfg["num_hidden_layers"]
        H = cfg["hidden_size"]
        hd = cfg.get("head_dim", H // cfg["num_attention_heads"])
        kvd = cfg["num_key_value_heads"] * hd

        def arr(a, dt=np.float32):
            a = np.ascontiguousarray(a, dt)
            self._keep.append(a)
            return a.ctypes.data

        def matrix(name):
            w = np.asarray(weights[name], np.float32)
            rows, cols = w.shape
            m = _Matrix(rows=rows, cols=cols, group=group or 0, bits=0)
            if group is None:
                m.dense = arr(w)
            else:
                codes, scales = quantize(f32_to_bf16_rne(w).ravel(), rows, cols, 8, group)
                m.bits = 8
                m.codes = arr(codes, np.uint8)
                m.scales = arr(scales)
            return m

        self._layers = (_Layer * L)()
        for i in range(L):
            p = f"model.layers.{i}."
            ly = self._layers[i]
            for short, name in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                                ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                                ("down", "mlp.down_proj")):
                setattr(ly, short, matrix(p + name + ".weight"))
            ly.input_norm = arr(weights[p + "input_layernorm.weight"])
            ly.post_norm = arr(weights[p + "post_attention_layernorm.weight"])
            ly.q_norm = arr(weights[p + "self_attn.q_norm.weight"])
            ly.k_norm = arr(weights[p + "self_attn.k_norm.weight"])
        m = _Qwen3()
        m.layers, m.hidden, m.heads, m.kv_heads, m.head_dim = L, H, cfg["num_attention_heads"], \
            cfg["num_key_value_heads"], hd
        m.ffn, m.vocab, m.capacity = cfg["intermediate_size"], cfg["vocab_size"], capacity
        m.eps = cfg["rms_norm_eps"]
        rp = cfg.get("rope_parameters") or {}
        m.theta = rp.get("rope_theta", cfg.get("rope_theta", 10000.0))
        m.kv_f16 = int(kv_f16)
        m.layer = C.cast(self._layers, C.c_void_p)
        m.embed = matrix("model.embed_tokens.weight")
        if "lm_head.weight" in weights and not cfg.get("tie_word_embeddings", False):
            m.lm_head = matrix("lm_head.weight")
        m.final_norm = arr(weights["model.norm.weight"])
        self._kv = np.zeros(2 * L * capacity * kvd, np.float32)
        m.keys = self._kv.ctypes.data
        m.values = self._kv.ctypes.data + L * capacity * kvd * 4
        self.m = m

    def forward(self, tokens) -> np.ndarray:
        ids = np.ascontiguousarray(tokens, np.uint32)
        logits = np.zeros(self.m.vocab, np.float32)
        rc = lib.or_qwen3_forward(C.byref(self.m), ids.ctypes.data, ids.size, logits.ctypes.data)
        if rc:
            raise ValueError(f"oracle forward failed ({rc})")
        return logits


def load_safetensors_f32(path: str) -> dict:
    """Reads a safetensors file as f32 arrays without executing anything from it (header JSON + raw little-endian
    tensors; BF16 widened by a shift)."""
    import json
    import struct
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + n])
    base = 8 + n
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        a, b = meta["data_offsets"]
        buf = raw[base + a: base + b]
        if meta["dtype"] == "BF16":
            v = bf16_to_f32(np.frombuffer(buf, np.uint16))
        elif meta["dtype"] == "F32":
            v = np.frombuffer(buf, np.float32)
        else:
            raise ValueError(meta["dtype"])
        out[name] = np.array(v, np.float32).reshape(meta["shape"])
    return out


# ---- synthetic models ----
class _SynthConfig(C.Structure):
    _fields_ = [(n, C.c_size_t) for n in ("layers", "hidden", "heads", "kv_heads", "head_dim", "ffn", "vocab",
                                          "group", "capacity")] + [
        ("eps", C.c_float), ("theta", C.c_float), ("tied", C.c_int), ("kv_f16", C.c_int), ("seed", C.c_uint64)]


lib.or_synth_stream.restype = C.c_uint64
lib.or_synth_stream.argtypes = [C.c_int, C.c_int]
lib.or_synth_prompt.restype = C.c_uint32
lib.or_synth_prompt.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32]
lib.or_qwen3_synth_new.restype = C.c_void_p
lib.or_qwen3_synth_new.argtypes = [C.c_void_p]
lib.or_qwen3_synth_free.argtypes = [C.c_void_p]
lib.or_qwen3_greedy.restype = C.c_int
lib.or_qwen3_greedy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p, C.c_size_t,
                                C.c_void_p, C.c_void_p]


def synth_prompt(seed: int, length: int, vocab: int) -> np.ndarray:
    return np.array([lib.or_synth_prompt(seed, i, vocab) for i in range(length)], np.uint32)


def synth_greedy(shape: dict, seed: int, prompt, steps: int, kv_f16: bool = False, prefill_chunk: int = 0,
                 with_top: bool = False):
    """Greedy tokens and top-1/top-2 gaps of the synthetic model ``shape`` (keys as in marin_amd.qwen3.SHAPES)."""
    prompt = np.ascontiguousarray(prompt, np.uint32)
    cfg = _SynthConfig(layers=shape["layers"], hidden=shape["hidden"], heads=shape["heads"],
                       kv_heads=shape["kv_heads"], head_dim=shape["head_dim"], ffn=shape["ffn"],
                       vocab=shape["vocab"], group=shape["group"], capacity=prompt.size + steps,
                       eps=shape["eps"], theta=shape["theta"], tied=int(shape["tied"]), kv_f16=int(kv_f16),
                       seed=seed)
    h = lib.or_qwen3_synth_new(C.byref(cfg))
    if not h:
        raise ValueError("synthetic model could not be built")
    try:
        toks = np.zeros(steps, np.uint32)
        gaps = np.zeros(steps, np.float32)
        top_ids = np.zeros(steps * 5, np.uint32)
        top_vals = np.zeros(steps * 5, np.float32)
        rc = lib.or_qwen3_greedy(h, prompt.ctypes.data, prompt.size, steps, toks.ctypes.data, gaps.ctypes.data,
                                 prefill_chunk, top_ids.ctypes.data, top_vals.ctypes.data)
        if rc:
            raise ValueError(f"oracle generation failed ({rc})")
        if with_top:
            return toks, gaps, top_ids.reshape(steps, 5), top_vals.reshape(steps, 5)
        return toks, gaps
    finally:
        lib.or_qwen3_synth_free(h)


lib.or_qwen3_synth_model.restype = C.c_void_p
lib.or_qwen3_synth_model.argtypes = [C.c_void_p]


def synth_rows(shape: dict, seed: int, prompt, tokens, kv_f16: bool = False) -> np.ndarray:
    """Logits after each of `tokens` (fed one at a time after the prompt) of the synthetic model ``shape``: the
    reference's default forward_rows (runtime/src/lib.rs:86-99). [len(tokens)][vocab] f32."""
    prompt = np.ascontiguousarray(prompt, np.uint32)
    tokens = np.ascontiguousarray(tokens, np.uint32)
    cfg = _SynthConfig(layers=shape["layers"], hidden=shape["hidden"], heads=shape["heads"],
                       kv_heads=shape["kv_heads"], head_dim=shape["head_dim"], ffn=shape["ffn"],
                       vocab=shape["vocab"], group=shape["group"], capacity=prompt.size + tokens.size + 1,
                       eps=shape["eps"], theta=shape["theta"], tied=int(shape["tied"]), kv_f16=int(kv_f16),
                       seed=seed)
    h = lib.or_qwen3_synth_new(C.byref(cfg))
    if not h:
        raise ValueError("synthetic model could not be built")
    try:
        model = lib.or_qwen3_synth_model(h)
        logits = np.zeros(shape["vocab"], np.float32)
        if lib.or_qwen3_forward(model, prompt.ctypes.data, prompt.size, logits.ctypes.data):
            raise ValueError("oracle prompt pass failed")
        rows = np.zeros((tokens.size, shape["vocab"]), np.float32)
        for i in range(tokens.size):
            if lib.or_qwen3_forward(model, tokens[i:].ctypes.data, 1, rows[i].ctypes.data):
                raise ValueError("oracle token pass failed")
        return rows
    finally:
        lib.or_qwen3_synth_free(h)
