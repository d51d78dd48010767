"""CPU checks of the boundary: the library loads and exports every function include/marin_hip.h declares."""
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "marin_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(marin_[a-z0-9_]+)\s*\(", text)))


def test_the_library_exports_every_declared_symbol():
    lib = os.path.join(ROOT, "marin_amd", "libmarin_hip.so")
    assert os.path.exists(lib), "build first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (marin_[a-z0-9_]+)", out))
    missing = [s for s in declared() if s not in exported]
    assert not missing, missing


def test_the_python_view_declares_every_symbol_and_loads():
    from marin_amd import _lib
    assert set(declared()) <= set(_lib.SIGNATURES)
    assert _lib.lib is not None


def test_no_gpu_means_unavailable_not_a_crash():
    import marin_amd as m
    try:
        m.Gpu()
    except m.Unavailable as e:
        assert "device" in str(e)
    except m.HipError:
        pass
