"""The marin-q8-v1 reader (marin_amd/packed.py) on CPU: an artifact written in the reference's format round-trips to
the oracle's codes and scales, and every check of Manifest::open / validate_packed / packed_chunks rejects what the
reference rejects (crates/loader/src/packed.rs:60-135, packed_read.rs:14-90)."""
import json
import os
import shutil

import numpy as np
import pytest

from marin_amd.packed import PackedError, open_packed
from oracle import oracle as o
from packed_bundle import bf16_bits, qwen3_tensor_names, write_packed

TINY = os.path.join(os.path.dirname(__file__), "golden", "tiny-qwen3")


def tiny_source(tmp_path):
    src = tmp_path / "src"
    src.mkdir()
    shutil.copyfile(os.path.join(TINY, "config.json"), src / "config.json")
    # the fixture has no tokenizer; the format needs one listed and present (its content is not read here)
    (src / "tokenizer.json").write_text('{"version": "1.0", "model": {"type": "BPE"}}')
    weights = o.load_safetensors_f32(os.path.join(TINY, "model.safetensors"))
    return str(src), weights


@pytest.fixture
def bundle(tmp_path):
    src, weights = tiny_source(tmp_path)
    dst = str(tmp_path / "packed")
    write_packed(src, weights, dst, 64)
    return dst, weights


def test_codes_and_scales_round_trip_to_the_oracle_quantizer(bundle):
    dst, weights = bundle
    pw = open_packed(dst)
    cfg = json.load(open(os.path.join(TINY, "config.json")))
    assert pw.group == 64 and pw.manifest["architecture"] == "qwen3"
    for name, matrix in qwen3_tensor_names(cfg):
        w = np.asarray(weights[name], np.float32)
        if matrix:
            rows, cols, codes, scales = pw.matrix(name)
            exp_c, exp_s = o.quantize(bf16_bits(w).ravel(), rows, cols, 8, 64)
            assert (rows, cols) == w.shape
            assert np.array_equal(codes, np.asarray(exp_c, np.uint8).ravel())
            assert np.array_equal(scales.view(np.uint32), np.asarray(exp_s, np.float32).ravel().view(np.uint32))
        else:
            assert np.array_equal(pw.vector(name), w.ravel())


def edit_manifest(dst, **changes):
    path = os.path.join(dst, "marin-int8.json")
    m = json.load(open(path))
    for k, v in changes.items():
        if v is None:
            m.pop(k)
        else:
            m[k] = v
    json.dump(m, open(path, "w"))


@pytest.mark.parametrize("change", [dict(format="marin-q8-v2"), dict(quantizer="other"), dict(architecture="llama"),
                                    dict(group=48), dict(group=0)])
def test_incompatible_manifests_are_refused(bundle, change):
    dst, _ = bundle
    edit_manifest(dst, **change)
    with pytest.raises(PackedError, match="incompatible format"):
        open_packed(dst)


def test_unknown_manifest_fields_are_refused(bundle):  # serde(deny_unknown_fields)
    dst, _ = bundle
    edit_manifest(dst, extra=1)
    with pytest.raises(PackedError, match="fields"):
        open_packed(dst)


def test_metadata_must_be_listed_present_and_unchanged(bundle):
    dst, _ = bundle
    m = json.load(open(os.path.join(dst, "marin-int8.json")))
    files = dict(m["files"])
    del files["tokenizer.json"]
    edit_manifest(dst, files=files)
    with pytest.raises(PackedError, match="missing tokenizer.json digest"):
        open_packed(dst)
    edit_manifest(dst, files=m["files"])
    open(os.path.join(dst, "config.json"), "a").write(" ")
    with pytest.raises(PackedError, match="checksum/presence mismatch: config.json"):
        open_packed(dst)


def test_an_unlisted_metadata_file_is_refused(bundle):
    dst, _ = bundle
    open(os.path.join(dst, "generation_config.json"), "w").write("{}")
    with pytest.raises(PackedError, match="generation_config.json"):
        open_packed(dst)


def test_architecture_must_match_the_config(bundle):
    dst, _ = bundle
    path = os.path.join(dst, "config.json")
    cfg = json.load(open(path))
    cfg["model_type"] = "qwen3_5"
    json.dump(cfg, open(path, "w"))
    m = json.load(open(os.path.join(dst, "marin-int8.json")))
    import hashlib
    m["files"]["config.json"] = list(hashlib.sha256(open(path, "rb").read()).digest())
    json.dump(m, open(os.path.join(dst, "marin-int8.json"), "w"))
    with pytest.raises(PackedError, match="architecture mismatch"):
        open_packed(dst)


def test_a_changed_tensor_byte_fails_its_digest_on_read(bundle):
    dst, _ = bundle
    pw = open_packed(dst)
    name = "model.layers.0.self_attn.q_proj.weight"
    begin = pw._header[name]["data_offsets"][0]
    path = os.path.join(dst, "model.safetensors")
    n = int.from_bytes(open(path, "rb").read(8), "little")
    with open(path, "r+b") as f:
        f.seek(8 + n + begin)
        b = f.read(1)
        f.seek(8 + n + begin)
        f.write(bytes([b[0] ^ 1]))
    pw = open_packed(dst)
    with pytest.raises(PackedError, match="checksum mismatch"):
        pw.matrix(name)
    assert open_packed(dst, verify=False).matrix(name)[0] > 0


def test_trailing_payload_is_refused(bundle):
    dst, _ = bundle
    open(os.path.join(dst, "model.safetensors"), "ab").write(b"\0" * 8)
    with pytest.raises(PackedError, match="trailing"):
        open_packed(dst)


def test_a_tensor_missing_from_the_manifest_is_refused(bundle):
    dst, _ = bundle
    m = json.load(open(os.path.join(dst, "marin-int8.json")))
    del m["tensors"]["model.norm.weight"]
    json.dump(m, open(os.path.join(dst, "marin-int8.json"), "w"))
    with pytest.raises(PackedError, match="name mismatch"):
        open_packed(dst)


def test_a_duplicate_manifest_key_is_refused(bundle):  # packed_read.rs:139-164 (unique)
    dst, _ = bundle
    path = os.path.join(dst, "marin-int8.json")
    m = json.load(open(path))
    name, digest = next(iter(m["tensors"].items()))
    other = [(b + 1) % 256 for b in digest]
    # the duplicate comes last, so a reader keeping the last value would see a digest that differs from the first
    text = json.dumps(m)
    tensors = json.dumps(m["tensors"])
    dup = tensors[:-1] + ", " + json.dumps(name) + ": " + json.dumps(other) + "}"
    open(path, "w").write(text.replace(tensors, dup))
    with pytest.raises(PackedError, match="duplicate key"):
        open_packed(dst)
    # a duplicated top-level field too (serde's duplicate field)
    open(path, "w").write(text[:-1] + ', "group": ' + json.dumps(m["group"]) + "}")
    with pytest.raises(PackedError, match="duplicate key"):
        open_packed(dst)


def test_a_duplicate_safetensors_header_key_is_refused(bundle):  # safetensors.rs:82-87 (packed_read::parse)
    dst, _ = bundle
    path = os.path.join(dst, "model.safetensors")
    raw = open(path, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + n])
    name = next(k for k in header if k != "__metadata__")
    text = json.dumps(header)
    text = text[:-1] + ", " + json.dumps(name) + ": " + json.dumps(header[name]) + "}"
    body = text.encode()
    body += b" " * ((8 - len(body) % 8) % 8)
    open(path, "wb").write(len(body).to_bytes(8, "little") + body + raw[8 + n:])
    with pytest.raises(PackedError, match="duplicate key"):
        open_packed(dst)
