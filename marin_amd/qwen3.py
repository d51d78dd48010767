"""The Qwen3 decode driver over the HIP backend (model/src/qwen3/gpu.rs Qwen3Gpu + runtime::CausalLm of the reference).

``Qwen3`` owns the device weights; ``Qwen3Cache`` is one sequence's paged KV cache and workspace (GpuCache,
gpu.rs:56-100). ``forward`` returns the last token's logits like ``CausalLm::forward``; ``generate`` is the greedy
loop of runtime::generate_reusing with the lowest-index argmax of the sampler, run on the device.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import Gpu, KvFormat, check
from ._lib import LaunchRecordC, Qwen3ConfigC, StepProfileC, alive, lib

# Benchmark shapes (BASELINE.json configs 0 and 3).
SHAPES = {
    "qwen3-1.7b": dict(layers=28, hidden=2048, heads=16, kv_heads=8, head_dim=128, ffn=6144, vocab=151936,
                       eps=1e-6, theta=1.0e6, tied=True, group=128),
    "qwen3-8b": dict(layers=36, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=12288, vocab=151936,
                     eps=1e-6, theta=1.0e6, tied=False, group=128),
}


def config_struct(shape: dict) -> Qwen3ConfigC:
    return Qwen3ConfigC(layers=shape["layers"], hidden=shape["hidden"], heads=shape["heads"],
                        kv_heads=shape["kv_heads"], head_dim=shape["head_dim"], ffn=shape["ffn"],
                        vocab=shape["vocab"], rms_eps=shape["eps"], rope_theta=shape["theta"],
                        tie_embeddings=int(shape["tied"]), group=shape["group"])


def weight_bytes(shape: dict) -> int:
    """Algorithmic bytes one decode token reads from the weights: int8 codes plus f32 scales of every projection
    and of the output head (the embedding row read is negligible and not counted)."""
    H, F, V = shape["hidden"], shape["ffn"], shape["vocab"]
    qd, kvd = shape["heads"] * shape["head_dim"], shape["kv_heads"] * shape["head_dim"]
    per_layer = H * (qd + 2 * kvd) + qd * H + 2 * F * H + F * H
    params = shape["layers"] * per_layer + V * H
    return params + params // shape["group"] * 4


class Qwen3:
    def __init__(self, gpu: Gpu, shape: dict, seed: int | None = None):
        self.gpu = gpu
        self.shape = dict(shape)
        self._cfg = config_struct(shape)
        h = C.c_void_p()
        if seed is None:
            check(lib.marin_qwen3_new_empty(gpu.handle, C.byref(self._cfg), C.byref(h)))
        else:
            check(lib.marin_qwen3_new_synthetic(gpu.handle, C.byref(self._cfg), seed, C.byref(h)))
        self._h = h

    @staticmethod
    def shape_from_hf(hf_config: dict, group: int) -> dict:
        """The model shape from an HF config.json (model/src/qwen3/config.rs:1-330; rope_theta may sit in
        rope_parameters, config.rs:87-90)."""
        hd = hf_config.get("head_dim", hf_config["hidden_size"] // hf_config["num_attention_heads"])
        rp = hf_config.get("rope_parameters") or {}
        return dict(layers=hf_config["num_hidden_layers"], hidden=hf_config["hidden_size"],
                    heads=hf_config["num_attention_heads"], kv_heads=hf_config["num_key_value_heads"],
                    head_dim=hd, ffn=hf_config["intermediate_size"], vocab=hf_config["vocab_size"],
                    eps=hf_config["rms_norm_eps"], theta=rp.get("rope_theta", hf_config.get("rope_theta", 1e4)),
                    tied=bool(hf_config.get("tie_word_embeddings", False)), group=group)

    LAYER_MATRICES = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                      "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")
    LAYER_VECTORS = ("input_layernorm", "post_attention_layernorm", "self_attn.q_norm", "self_attn.k_norm")

    @classmethod
    def from_hf(cls, gpu: Gpu, hf_config: dict, weights: dict, quantize, group: int) -> "Qwen3":
        """Loads HF-named f32 weights, quantizing every matrix int8 with ``quantize(bf16_bits, rows, cols, bits,
        group) -> (codes, scales)`` (tensor::quantize's contract)."""
        shape = cls.shape_from_hf(hf_config, group)
        m = cls(gpu, shape)

        def put(layer, tensor, name):
            w = np.asarray(weights[name], np.float32)
            rows, cols = w.shape
            codes, scales = quantize(_bf16_bits(w).ravel(), rows, cols, 8, group)
            m.load_matrix(layer, tensor, rows, cols, codes, scales)

        for i in range(shape["layers"]):
            p = f"model.layers.{i}."
            for t, n in enumerate(cls.LAYER_MATRICES):
                put(i, t, p + n + ".weight")
            for v, n in enumerate(cls.LAYER_VECTORS):
                m.load_vector(i, v, weights[p + n + ".weight"])
        put(-1, 0, "model.embed_tokens.weight")
        if not shape["tied"]:
            put(-1, 1, "lm_head.weight")
        m.load_vector(-1, 0, weights["model.norm.weight"])
        return m

    @classmethod
    def from_packed(cls, gpu: Gpu, directory: str, verify: bool = True) -> "Qwen3":
        """Loads a marin-q8-v1 artifact (GpuStore::packed, model/src/qwen3/gpu.rs:47-50): the reference's own int8
        codes and f32 scales are uploaded as they are, with no requantization."""
        from .packed import PackedError, open_packed

        pw = open_packed(directory, verify)
        if pw.manifest["architecture"] != "qwen3":
            raise PackedError(f"a {pw.manifest['architecture']} artifact is not a Qwen3 model")
        shape = cls.shape_from_hf(pw.config, pw.group)
        m = cls(gpu, shape)

        def put(layer, tensor, name):
            rows, cols, codes, scales = pw.matrix(name)
            m.load_matrix(layer, tensor, rows, cols, codes, scales)

        for i in range(shape["layers"]):
            p = f"model.layers.{i}."
            for t, n in enumerate(cls.LAYER_MATRICES):
                put(i, t, p + n + ".weight")
            for v, n in enumerate(cls.LAYER_VECTORS):
                m.load_vector(i, v, pw.vector(p + n + ".weight"))
        put(-1, 0, "model.embed_tokens.weight")
        if not shape["tied"]:
            put(-1, 1, "lm_head.weight")
        m.load_vector(-1, 0, pw.vector("model.norm.weight"))
        return m

    def load_matrix(self, layer, tensor, rows, cols, codes, scales):
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        check(lib.marin_qwen3_load_matrix(self._h, layer, tensor, rows, cols, codes.ctypes.data, scales.ctypes.data))

    def load_vector(self, layer, which, values):
        v = np.ascontiguousarray(values, np.float32).ravel()
        check(lib.marin_qwen3_load_vector(self._h, layer, which, v.ctypes.data, v.size))

    def new_cache(self, capacity: int, fmt: KvFormat = KvFormat.F32) -> "Qwen3Cache":
        return Qwen3Cache(self, capacity, fmt)

    def new_batch(self, batch: int, capacity: int, fmt: KvFormat = KvFormat.F32) -> "Qwen3Batch":
        """A decode batch of `batch` (1..8) sequences of `capacity` positions each (extension; see
        include/marin_hip.h)."""
        return Qwen3Batch(self, batch, capacity, fmt)

    def forward(self, tokens, cache: "Qwen3Cache") -> np.ndarray:
        ids = np.ascontiguousarray(tokens, np.uint32).ravel()
        logits = np.empty(self.shape["vocab"], np.float32)
        check(lib.marin_qwen3_forward(self._h, cache._h, ids.ctypes.data, ids.size, logits.ctypes.data))
        return logits

    def forward_rows(self, tokens, cache: "Qwen3Cache") -> np.ndarray:
        """CausalLm::forward_rows (runtime/src/lib.rs:86-99): the logits after every token of a pass of at most 8,
        [len(tokens)][vocab]."""
        ids = np.ascontiguousarray(tokens, np.uint32).ravel()
        rows = np.empty((ids.size, self.shape["vocab"]), np.float32)
        check(lib.marin_qwen3_forward_rows(self._h, cache._h, ids.ctypes.data, ids.size, rows.ctypes.data))
        return rows

    def max_rows(self) -> int:
        """CausalLm::max_rows (model/src/qwen3/gpu.rs:388-390)."""
        return 8

    def generate(self, prompt, steps: int, cache: "Qwen3Cache") -> np.ndarray:
        ids = np.ascontiguousarray(prompt, np.uint32).ravel()
        out = np.zeros(steps, np.uint32)
        check(lib.marin_qwen3_generate(self._h, cache._h, ids.ctypes.data, ids.size, steps, out.ctypes.data))
        return out

    def decode(self, steps: int, cache: "Qwen3Cache") -> np.ndarray:
        """Greedy tokens continuing from the cache's last logits; every chosen token is fed through the model."""
        out = np.zeros(steps, np.uint32)
        check(lib.marin_qwen3_decode(self._h, cache._h, steps, out.ctypes.data))
        return out

    def profile_step(self, cache: "Qwen3Cache") -> dict:
        """One decode step with an event after every launch: summed seconds and algorithmic bytes per kernel kind."""
        p = StepProfileC()
        check(lib.marin_qwen3_profile_step(self._h, cache._h, C.byref(p)))
        return {f: getattr(p, f) for f, _ in StepProfileC._fields_}

    def profile_launches(self, cache: "Qwen3Cache") -> list:
        """One decode step with events around every launch: [(kind, kernel name, algorithmic bytes, seconds)] in
        launch order (kind 0 other, 1 quantized product, 2 attention)."""
        cap = 4096
        recs = (LaunchRecordC * cap)()
        n = C.c_size_t()
        check(lib.marin_qwen3_profile_launches(self._h, cache._h, recs, cap, C.byref(n)))
        return [(int(r.kind), r.name.decode(), float(r.bytes), float(r.seconds)) for r in recs[:min(n.value, cap)]]

    def time_kernel(self, cache: "Qwen3Cache", name: str, reps: int = 20) -> tuple:
        """Mean seconds per launch of kernel `name` over graph replays of one decode pass's launches of it, and the
        launches per pass (the cache's activations are left unspecified)."""
        sec, n = C.c_double(), C.c_uint32()
        check(lib.marin_qwen3_time_kernel(self._h, cache._h, name.encode(), reps, C.byref(sec), C.byref(n)))
        return sec.value, n.value

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_qwen3_free(self._h)
            self._h = None


class Qwen3Cache:
    def __init__(self, model: Qwen3, capacity: int, fmt: KvFormat):
        h = C.c_void_p()
        check(lib.marin_qwen3_cache_new(model._h, capacity, int(fmt), C.byref(h)))
        self._h = h
        self._model = model

    def __len__(self):
        return int(lib.marin_qwen3_cache_len(self._h))

    def truncate(self, length: int) -> None:
        check(lib.marin_qwen3_cache_truncate(self._h, length))

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_qwen3_cache_free(self._h)
            self._h = None


class Qwen3Batch:
    """Sequences decoded together: prompts one sequence at a time, then every sequence one greedy token per step."""

    def __init__(self, model: Qwen3, batch: int, capacity: int, fmt: KvFormat):
        h = C.c_void_p()
        check(lib.marin_qwen3_batch_new(model._h, batch, capacity, int(fmt), C.byref(h)))
        self._h = h
        self._model = model
        self.batch = batch

    def length(self, seq: int) -> int:
        return int(lib.marin_qwen3_batch_len(self._h, seq))

    def prefill(self, seq: int, tokens) -> None:
        ids = np.ascontiguousarray(tokens, np.uint32).ravel()
        check(lib.marin_qwen3_batch_prefill(self._h, seq, ids.ctypes.data, ids.size))

    def decode(self, steps: int) -> np.ndarray:
        """[batch][steps] greedy tokens."""
        out = np.zeros((self.batch, steps), np.uint32)
        check(lib.marin_qwen3_batch_decode(self._h, steps, out.ctypes.data))
        return out

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_qwen3_batch_free(self._h)
            self._h = None


def _bf16_bits(values: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (weights that came from bf16 are exact)."""
    u = np.asarray(values, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
