"""Loads libmarin_hip.so and declares the C ABI of include/marin_hip.h.

There is no fallback: if the library is missing this module raises, so nothing can silently run another path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# MARIN_HIP_LIB names another build of the library (a variant under test); the in-tree build otherwise.
LIB_PATH = os.environ.get("MARIN_HIP_LIB") or os.path.join(HERE, "libmarin_hip.so")

P = C.c_void_p
PP = C.POINTER(C.c_void_p)
sz = C.c_size_t
st = C.c_int  # marin_status


class GpuInfo(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("arch", C.c_char * 64), ("compute_units", C.c_int),
                ("free_bytes", sz), ("total_bytes", sz)]


class TrafficC(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("launches", "allocations", "uploads", "upload_bytes", "downloads",
                                          "download_bytes")]


class StepProfileC(C.Structure):
    _fields_ = [(n, C.c_double) for n in ("gemv_seconds", "gemv_bytes", "attention_seconds", "attention_bytes",
                                          "other_seconds", "step_seconds")] + [
        (n, C.c_uint32) for n in ("gemv_launches", "attention_launches", "other_launches")]


class LaunchRecordC(C.Structure):
    _fields_ = [("kind", C.c_uint32), ("bytes", C.c_double), ("seconds", C.c_double), ("name", C.c_char * 96)]


class Qwen3ConfigC(C.Structure):
    _fields_ = [(n, sz) for n in ("layers", "hidden", "heads", "kv_heads", "head_dim", "ffn", "vocab")] + [
        ("rms_eps", C.c_float), ("rope_theta", C.c_float), ("tie_embeddings", C.c_int), ("group", sz)]


SIGNATURES = {
    "marin_last_error": (C.c_char_p, []),
    "marin_last_error_fields": (None, [C.POINTER(sz), C.POINTER(sz), C.POINTER(sz)]),
    "marin_last_error_is_oom": (C.c_int, []),
    "marin_gpu_new": (st, [PP]),
    "marin_gpu_free": (None, [P]),
    "marin_gpu_info_get": (st, [P, C.POINTER(GpuInfo)]),
    "marin_gpu_synchronize": (st, [P]),
    "marin_gpu_stream": (P, [P]),
    "marin_gpu_bind_to_thread": (st, [P]),
    "marin_set_fast_attention": (None, [P, C.c_int]),
    "marin_upload_matrix": (st, [P, sz, sz, P, sz, PP]),
    "marin_matrix_free": (None, [P]),
    "marin_matrix_shape": (None, [P, C.POINTER(sz), C.POINTER(sz)]),
    "marin_embed": (st, [P, P, P, sz, P, P]),
    "marin_matmul": (st, [P, P, P, sz, P]),
    "marin_matmul_precise": (st, [P, P, P, sz, P]),
    "marin_matmul_pair": (st, [P, P, P, P, sz, P, P]),
    "marin_matmul_triple": (st, [P, P, P, P, P, sz, P, P, P]),
    "marin_matmul_quant_bf16_noalloc": (st, [P, P, P, sz, P]),
    "marin_qwen3_forward_rows": (st, [P, P, P, sz, P]),
    "marin_kv_is_empty": (C.c_int, [P]),
    "marin_kv_format_of": (C.c_int, [P]),
    "marin_kv_auxiliary_bytes": (sz, [P]),
    "marin_gpu_traffic": (st, [P, C.POINTER(TrafficC)]),
    "marin_mark_new": (st, [P, PP]),
    "marin_mark_since": (st, [P, P, C.POINTER(C.c_double)]),
    "marin_mark_free": (None, [P]),
    "marin_buffer_zeros": (st, [P, sz, PP]),
    "marin_buffer_upload": (st, [P, P, sz, PP]),
    "marin_buffer_upload_into": (st, [P, P, sz, P]),
    "marin_buffer_download": (st, [P, P, P, sz]),
    "marin_buffer_download_range": (st, [P, P, sz, sz, P]),
    "marin_buffer_copy_range_into": (st, [P, P, sz, P]),
    "marin_buffer_copy_into_range": (st, [P, P, P, sz]),
    "marin_buffer_len": (sz, [P]),
    "marin_buffer_free": (None, [P]),
    "marin_buffer_new_typed": (st, [P, C.c_int, sz, P, PP]),
    "marin_buffer_download_raw": (st, [P, P, P, sz]),
    "marin_buffer_dtype": (C.c_int, [P]),
    "marin_buffer_device_ptr": (P, [P]),
    "marin_tokens_new": (st, [P, sz, PP]),
    "marin_tokens_free": (None, [P]),
    "marin_upload_quantized": (st, [P, sz, sz, C.c_int, sz, P, sz, P, sz, PP]),
    "marin_upload_quantized_bf16_scales": (st, [P, sz, sz, C.c_int, sz, P, sz, P, sz, PP]),
    "marin_quant_matrix_free": (None, [P]),
    "marin_quant_matrix_shape": (None, [P, C.POINTER(sz), C.POINTER(sz), C.POINTER(C.c_int), C.POINTER(sz)]),
    "marin_quant_matrix_bytes": (sz, [P]),
    "marin_embed_quant": (st, [P, P, P, sz, P, P]),
    "marin_matmul_quant": (st, [P, P, P, sz, P]),
    "marin_matmul_quant_precise": (st, [P, P, P, sz, P]),
    "marin_matmul_quant_bf16": (st, [P, P, P, sz, P]),
    "marin_rms_norm": (st, [P, P, P, C.c_float]),
    "marin_rms_norm_into": (st, [P, P, P, P, C.c_float]),
    "marin_rope": (st, [P, P, sz, sz, sz, C.c_float]),
    "marin_silu_mul": (st, [P, P, P]),
    "marin_add": (st, [P, P, P]),
    "marin_kv_new": (st, [P, sz, sz, sz, sz, sz, C.c_int, PP]),
    "marin_kv_free": (None, [P]),
    "marin_kv_write": (st, [P, P, sz, P, P]),
    "marin_kv_advance": (st, [P, sz]),
    "marin_kv_truncate": (st, [P, sz]),
    "marin_kv_clear": (None, [P]),
    "marin_kv_len": (sz, [P]),
    "marin_kv_capacity": (sz, [P]),
    "marin_kv_pages_held": (sz, [P]),
    "marin_kv_pages_in_use": (sz, [P]),
    "marin_kv_bytes_held": (sz, [P]),
    "marin_kv_page_bytes": (sz, [P]),
    "marin_kv_slab_bytes": (sz, [P]),
    "marin_kv_page_ids": (sz, [P, P, sz]),
    "marin_kv_startup_bytes": (sz, [sz, sz, sz, sz, sz, C.c_int]),
    "marin_attention": (st, [P, P, P, sz, sz, sz, P]),
    "marin_page_pool_new": (st, [P, sz, sz, sz, sz, C.c_int, PP]),
    "marin_page_pool_free": (None, [P]),
    "marin_page_pool_write": (st, [P, P, sz, P, sz]),
    "marin_paged_attention_batch": (st, [P, P, P, P, sz, P, sz, sz, P]),
    "marin_qwen3_new_synthetic": (st, [P, C.POINTER(Qwen3ConfigC), C.c_uint64, PP]),
    "marin_qwen3_new_empty": (st, [P, C.POINTER(Qwen3ConfigC), PP]),
    "marin_qwen3_load_matrix": (st, [P, C.c_int, C.c_int, sz, sz, P, P]),
    "marin_qwen3_load_vector": (st, [P, C.c_int, C.c_int, P, sz]),
    "marin_qwen3_free": (None, [P]),
    "marin_qwen3_cache_new": (st, [P, sz, C.c_int, PP]),
    "marin_qwen3_cache_free": (None, [P]),
    "marin_qwen3_cache_len": (sz, [P]),
    "marin_qwen3_cache_truncate": (st, [P, sz]),
    "marin_qwen3_forward": (st, [P, P, P, sz, P]),
    "marin_qwen3_generate": (st, [P, P, P, sz, sz, P]),
    "marin_qwen3_decode": (st, [P, P, sz, P]),
    "marin_qwen3_batch_new": (st, [P, sz, sz, C.c_int, PP]),
    "marin_qwen3_batch_free": (None, [P]),
    "marin_qwen3_batch_len": (sz, [P, sz]),
    "marin_qwen3_batch_prefill": (st, [P, sz, P, sz]),
    "marin_qwen3_batch_decode": (st, [P, sz, P]),
    "marin_qwen3_profile_step": (st, [P, P, C.POINTER(StepProfileC)]),
    "marin_probe_copy": (st, [P, sz, C.c_int, C.POINTER(C.c_double)]),
    "marin_moe_route": (st, [P, P, sz, sz, sz, C.c_int, P, P]),
    "marin_time_matmul_bf16": (st, [P, P, sz, P, sz, P, C.c_int, C.POINTER(C.c_double)]),
    "marin_moe_ffn": (st, [P, P, P, P, P, C.c_float, P, P, sz, sz, sz, P, P]),
    "marin_moe_stack_time": (st, [P, sz, P, P, P, P, C.c_float, P, P, sz, sz, sz, P, P, C.c_int, C.c_int,
                                  C.POINTER(C.c_double)]),
    "marin_qwen3_time_kernel": (st, [P, P, C.c_char_p, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_uint32)]),
    "marin_qwen3_profile_launches": (st, [P, P, C.POINTER(LaunchRecordC), sz, C.POINTER(sz)]),
    "marin_quantized_synthetic": (st, [P, sz, sz, sz, C.c_uint64, C.c_uint64, C.c_double, PP]),
}


def load(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(there is no fallback path)")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()

# Once the interpreter is shutting down, handles are left to the process exit instead of being freed from __del__
# in whatever order finalization reaches them.
import atexit  # noqa: E402

SHUTTING_DOWN = [False]
atexit.register(lambda: SHUTTING_DOWN.__setitem__(0, True))


def alive() -> bool:
    return not SHUTTING_DOWN[0]
