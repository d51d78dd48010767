"""Reader of Marin's packed int8 artifacts (format "marin-q8-v1"), so this backend loads the reference's own exported
weights byte for byte.

The format (crates/loader/src/packed.rs:11-13, 158-277; export crates/model/src/qwen3/export.rs:12-121):
- one ``model.safetensors`` whose tensors are, for every 2-D weight ``name``, the int8 codes ``name`` (dtype I8,
  shape [rows][cols], two's complement as tensor::Quantized holds them) and its scales ``name.scales`` (F32,
  [rows][cols / group]); every 1-D weight (norms) is F32. Spans are contiguous from offset 0 with nothing after the
  last one (packed_read.rs:14-43);
- ``marin-int8.json``: format, quantizer ("symmetric-maxabs-round-v1"), architecture, group (a multiple of 32), and
  SHA-256 digests (arrays of 32 byte values) of the metadata files (config.json and tokenizer.json required,
  generation_config.json and tokenizer_config.json optional: present exactly when listed), of every tensor's bytes,
  and of the source tensors (packed.rs:60-135).

``open_packed`` applies the reference's checks and raises ``PackedError`` with the reason; tensor digests are
verified as each tensor is read (packed_read.rs:45-90).
"""
from __future__ import annotations

import hashlib
import json
import os
import stat

import numpy as np

MANIFEST = "marin-int8.json"
FORMAT = "marin-q8-v1"
QUANTIZER = "symmetric-maxabs-round-v1"
ARCHITECTURES = ("qwen3", "qwen3_5", "granitemoe")
METADATA = ("config.json", "tokenizer.json", "generation_config.json", "tokenizer_config.json")


class PackedError(ValueError):
    """LoaderError::Packed (crates/loader/src/packed.rs:30-32)."""


def _unique_keys(pairs):
    """object_pairs_hook refusing a key seen twice in one object, as packed_read.rs:139-164 (`unique`) and serde's
    duplicate-field check do; json.loads alone would keep the last value silently."""
    out = {}
    for key, value in pairs:
        if key in out:
            raise PackedError(f"duplicate key: {key}")
        out[key] = value
    return out


def _loads(data):
    try:
        return json.loads(data, object_pairs_hook=_unique_keys)
    except json.JSONDecodeError as e:
        raise PackedError(str(e)) from None


def _regular(path: str) -> bool:
    try:
        return stat.S_ISREG(os.lstat(path).st_mode)
    except FileNotFoundError:
        return False


def _file_digest(path: str) -> bytes:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.digest()


def _digest_map(value, what: str) -> dict:
    if not isinstance(value, dict):
        raise PackedError(f"{what} must be an object of digests")
    out = {}
    for name, d in value.items():
        if not (isinstance(d, list) and len(d) == 32 and all(isinstance(b, int) and 0 <= b < 256 for b in d)):
            raise PackedError(f"{what}: bad digest for {name}")
        out[name] = bytes(d)
    return out


def read_manifest(directory: str) -> dict:
    """Manifest::open (packed.rs:60-135): the manifest and model.safetensors are regular files, the manifest is at
    most 4 MiB, format/quantizer/architecture/group are the supported ones, config.json and tokenizer.json digests
    are listed, every metadata file is present exactly when listed and matches its digest, and config.json's
    model_type is the manifest's architecture."""
    path = os.path.join(directory, MANIFEST)
    if not _regular(path) or not _regular(os.path.join(directory, "model.safetensors")):
        raise PackedError("artifact files must be regular files")
    if os.path.getsize(path) > 4 << 20:
        raise PackedError("manifest exceeds 4 MiB")
    with open(path, "rb") as f:
        raw = _loads(f.read())
    keys = {"format", "quantizer", "architecture", "group", "files", "tensors", "source_tensors"}
    if not isinstance(raw, dict) or set(raw) != keys:
        raise PackedError("manifest fields differ from the format's")
    group = raw["group"]
    if (raw["format"] != FORMAT or raw["quantizer"] != QUANTIZER or raw["architecture"] not in ARCHITECTURES
            or not isinstance(group, int) or group <= 0 or group % 32):
        raise PackedError("incompatible format, architecture, quantizer or group")
    files = _digest_map(raw["files"], "files")
    tensors = _digest_map(raw["tensors"], "tensors")
    _digest_map(raw["source_tensors"], "source_tensors")
    for required in ("config.json", "tokenizer.json"):
        if required not in files:
            raise PackedError(f"missing {required} digest")
    for name in METADATA:
        p = os.path.join(directory, name)
        present = os.path.lexists(p)
        if present and not _regular(p):
            raise PackedError("artifact metadata must be regular files")
        want = files.get(name)
        if (want is None) != (not present) or (want is not None and want != _file_digest(p)):
            raise PackedError(f"metadata checksum/presence mismatch: {name}")
    if len(files) != 2 + ("generation_config.json" in files) + ("tokenizer_config.json" in files):
        raise PackedError("unknown metadata file")
    with open(os.path.join(directory, "config.json")) as f:
        config = json.load(f)
    if config.get("model_type") != raw["architecture"]:
        raise PackedError("artifact/config architecture mismatch")
    return {"architecture": raw["architecture"], "group": group, "tensors": tensors, "config": config}


class PackedWeights:
    """The tensors of a packed artifact, memory-mapped; every read verifies the tensor's digest."""

    def __init__(self, directory: str, verify: bool = True):
        self.manifest = read_manifest(directory)
        self.config = self.manifest["config"]
        self.group = self.manifest["group"]
        self.verify = verify
        path = os.path.join(directory, "model.safetensors")
        size = os.path.getsize(path)
        with open(path, "rb") as f:
            n = int.from_bytes(f.read(8), "little")
            if n > size - 8:
                raise PackedError("safetensors header exceeds the file")
            header = _loads(f.read(n))
        header.pop("__metadata__", None)
        self._data = np.memmap(path, dtype=np.uint8, mode="r", offset=8 + n)
        spans = []
        for name, info in header.items():
            dtype, shape, (begin, end) = info["dtype"], info["shape"], info["data_offsets"]
            if dtype not in ("I8", "F32"):
                raise PackedError("overlapping/noncontiguous spans or incompatible dtype")
            count = int(np.prod(shape)) if shape else 1
            if end - begin != count * (1 if dtype == "I8" else 4):
                raise PackedError(f"{name}: span length differs from its shape")
            spans.append((begin, end, name))
        spans.sort()
        at = 0
        for begin, end, _ in spans:
            if begin != at:
                raise PackedError("overlapping/noncontiguous spans or incompatible dtype")
            at = end
        if at != size - 8 - n:
            raise PackedError("trailing/unindexed payload")
        if set(header) != set(self.manifest["tensors"]):
            raise PackedError("tensor digest/name mismatch or sharded artifact")
        self._header = header

    def names(self):
        return list(self._header)

    def _bytes(self, name: str) -> np.ndarray:
        info = self._header.get(name)
        if info is None:
            raise PackedError(f"unknown tensor {name}")
        begin, end = info["data_offsets"]
        raw = self._data[begin:end]
        if self.verify and hashlib.sha256(raw).digest() != self.manifest["tensors"][name]:
            raise PackedError(f"tensor checksum mismatch: {name}")
        return raw

    def matrix(self, name: str):
        """(rows, cols, codes u8 [rows*cols], scales f32 [rows*cols/group]) of a quantized weight."""
        info = self._header.get(name)
        if info is None or info["dtype"] != "I8" or len(info["shape"]) != 2:
            raise PackedError(f"{name} is not an int8 matrix")
        rows, cols = info["shape"]
        s = self._header.get(name + ".scales")
        if s is None or s["dtype"] != "F32" or s["shape"] != [rows, cols // self.group] or cols % self.group:
            raise PackedError(f"{name}.scales does not fit {name}")
        codes = np.asarray(self._bytes(name))
        scales = np.asarray(self._bytes(name + ".scales")).view(np.float32)
        return rows, cols, codes, scales

    def vector(self, name: str) -> np.ndarray:
        info = self._header.get(name)
        if info is None or info["dtype"] != "F32":
            raise PackedError(f"{name} is not an f32 tensor")
        return np.asarray(self._bytes(name)).view(np.float32)


def open_packed(directory: str, verify: bool = True) -> PackedWeights:
    return PackedWeights(directory, verify)
