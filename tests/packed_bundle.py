"""Writes a marin-q8-v1 artifact from bf16 HF weights, for the packed-format tests (the role of export_int8,
crates/model/src/qwen3/export.rs:12-121, and PackedWriter, crates/loader/src/packed.rs:158-378).

Matrices are quantized int8 with the CPU oracle (the reference's tensor::quantize rule); the header is padded with
spaces to a multiple of 8 bytes as PackedWriter::new pads it.
"""
import hashlib
import json
import os
import shutil

import numpy as np

from oracle import oracle as o

METADATA = ("config.json", "tokenizer.json", "generation_config.json", "tokenizer_config.json")


def qwen3_tensor_names(cfg: dict) -> list:
    """Qwen3's weights in HF names: (name, is_matrix)."""
    names = [("model.embed_tokens.weight", True)]
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}."
        names += [(p + n + ".weight", True) for n in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                                      "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj",
                                                      "mlp.down_proj")]
        names += [(p + n + ".weight", False) for n in ("input_layernorm", "post_attention_layernorm",
                                                       "self_attn.q_norm", "self_attn.k_norm")]
    names.append(("model.norm.weight", False))
    if not cfg.get("tie_word_embeddings", False):
        names.append(("lm_head.weight", True))
    return names


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """f32 values that are exactly bf16 -> their bf16 bits."""
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def write_packed(source_dir: str, weights: dict, destination: str, group: int) -> dict:
    """weights: HF name -> f32 array holding bf16 values. Returns the manifest written."""
    cfg = json.load(open(os.path.join(source_dir, "config.json")))
    os.makedirs(destination, exist_ok=False)
    manifest = {"format": "marin-q8-v1", "quantizer": "symmetric-maxabs-round-v1", "architecture": cfg["model_type"],
                "group": group, "files": {}, "tensors": {}, "source_tensors": {}}
    for name in METADATA:
        src = os.path.join(source_dir, name)
        if os.path.exists(src):
            shutil.copyfile(src, os.path.join(destination, name))
            manifest["files"][name] = list(hashlib.sha256(open(src, "rb").read()).digest())
    blobs = []
    header = {}
    offset = 0

    def add(name, dtype, shape, data: bytes):
        nonlocal offset
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + len(data)]}
        manifest["tensors"][name] = list(hashlib.sha256(data).digest())
        blobs.append(data)
        offset += len(data)

    for name, matrix in qwen3_tensor_names(cfg):
        w = np.asarray(weights[name], np.float32)
        bits = bf16_bits(w)
        manifest["source_tensors"][name] = list(hashlib.sha256(bits.astype("<u2").tobytes()).digest())
        if matrix:
            rows, cols = w.shape
            codes, scales = o.quantize(bits.ravel(), rows, cols, 8, group)
            add(name, "I8", (rows, cols), np.ascontiguousarray(codes, np.uint8).tobytes())
            add(name + ".scales", "F32", (rows, cols // group), np.ascontiguousarray(scales, "<f4").tobytes())
        else:
            add(name, "F32", w.shape, np.ascontiguousarray(w, "<f4").tobytes())
    hb = json.dumps(header).encode()
    while len(hb) % 8:
        hb += b" "
    with open(os.path.join(destination, "model.safetensors"), "wb") as f:
        f.write(len(hb).to_bytes(8, "little"))
        f.write(hb)
        for b in blobs:
            f.write(b)
    with open(os.path.join(destination, "marin-int8.json"), "w") as f:
        json.dump(manifest, f)
    return manifest
