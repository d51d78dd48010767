"""marin_amd: the MI355X backend of Marin's quantized decode path.

A Python view of the C ABI in include/marin_hip.h with the names of the reference's `cuda` crate
(crates/cuda/src/lib.rs:21-28): ``Gpu``, ``Buffer``, ``DeviceQuantMatrix``, ``Tokens``, ``DeviceKv``, ``KvFormat``,
``PAGE_TOKENS``, ``SLAB_PAGES``, ``pages_for`` and the ``CudaError`` variants (here ``HipError`` and subclasses).
Every method checks sizes in the native library before anything is launched; failures raise the matching error.
"""
from __future__ import annotations

import ctypes as C
import enum

import numpy as np

from ._lib import GpuInfo, TrafficC, alive, lib

PAGE_TOKENS = 64  # crates/cuda/src/pages.rs:4
SLAB_PAGES = 8  # crates/cuda/src/pages.rs:7


def pages_for(tokens: int) -> int:
    """crates/cuda/src/pages.rs:9-11"""
    return -(-tokens // PAGE_TOKENS)


class HipError(Exception):
    """crates/cuda/src/error.rs:6-36 (CudaError)."""

    def __init__(self, status: int, message: str, expected: int = 0, actual: int = 0, extra: int = 0,
                 oom: bool = False):
        super().__init__(message)
        self.status = status
        self.expected, self.actual, self.extra = expected, actual, extra
        self.oom = oom

    def is_out_of_memory(self) -> bool:
        """error.rs:40-49"""
        return self.oom


class Unavailable(HipError):
    pass


class Driver(HipError):
    pass


class Shape(HipError):
    pass


class KvMemory(HipError):
    pass


class Overflow(HipError):
    pass


class SelfCheck(HipError):
    pass


class Unsupported(HipError):
    pass


_ERRORS = {1: Unavailable, 2: Driver, 3: Shape, 4: KvMemory, 5: Overflow, 6: SelfCheck, 7: Unsupported}


def check(status: int) -> None:
    if status == 0:
        return
    e, a, x = C.c_size_t(), C.c_size_t(), C.c_size_t()
    lib.marin_last_error_fields(C.byref(e), C.byref(a), C.byref(x))
    msg = (lib.marin_last_error() or b"").decode(errors="replace")
    raise _ERRORS.get(status, HipError)(status, msg, e.value, a.value, x.value, bool(lib.marin_last_error_is_oom()))


def _out() -> C.c_void_p:
    return C.c_void_p()


class KvFormat(enum.IntEnum):
    """crates/cuda/src/kv_format.rs:1-46, plus BF16 for the benchmark layout."""
    F32 = 0
    F16 = 1
    BF16 = 2

    def row_bytes(self, kv_heads: int, head_dim: int) -> int:
        return kv_heads * head_dim * (4 if self == KvFormat.F32 else 2)


class Dtype(enum.IntEnum):
    F32 = 0
    BF16 = 1
    F16 = 2
    U8 = 3
    U32 = 4


_NP = {Dtype.F32: np.float32, Dtype.BF16: np.uint16, Dtype.F16: np.float16, Dtype.U8: np.uint8,
       Dtype.U32: np.uint32}


class Buffer:
    """A flat device array (gpu.rs:87-123). f32 unless made with a dtype."""

    def __init__(self, gpu: "Gpu", handle: C.c_void_p):
        self._gpu = gpu
        self._h = handle

    @property
    def handle(self):
        return self._h

    def __len__(self) -> int:
        return int(lib.marin_buffer_len(self._h))

    @property
    def dtype(self) -> Dtype:
        return Dtype(lib.marin_buffer_dtype(self._h))

    def device_ptr(self) -> int:
        return int(lib.marin_buffer_device_ptr(self._h) or 0)

    def free(self) -> None:
        if self._h and alive():
            lib.marin_buffer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Tokens:
    """gpu.rs:94-97: device memory for the token ids of one pass."""

    def __init__(self, handle, capacity):
        self._h = handle
        self.capacity = capacity

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_tokens_free(self._h)
            self._h = None


class DeviceQuantMatrix:
    """crates/cuda/src/quant.rs:16-45"""

    def __init__(self, handle):
        self._h = handle
        r, c, b, g = C.c_size_t(), C.c_size_t(), C.c_int(), C.c_size_t()
        lib.marin_quant_matrix_shape(handle, C.byref(r), C.byref(c), C.byref(b), C.byref(g))
        self._rows, self._cols, self.bits, self.group = r.value, c.value, b.value, g.value

    def rows(self) -> int:
        return self._rows

    def cols(self) -> int:
        return self._cols

    def device_bytes(self) -> int:
        return int(lib.marin_quant_matrix_bytes(self._h))

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_quant_matrix_free(self._h)
            self._h = None


class DeviceMatrix:
    """gpu.rs:87-93: a bf16 matrix, row-major, on the device."""

    def __init__(self, handle):
        self._h = handle
        r, c = C.c_size_t(), C.c_size_t()
        lib.marin_matrix_shape(handle, C.byref(r), C.byref(c))
        self._rows, self._cols = r.value, c.value

    @property
    def handle(self):
        return self._h

    def rows(self) -> int:
        return self._rows

    def cols(self) -> int:
        return self._cols

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_matrix_free(self._h)
            self._h = None


class Traffic:
    def __init__(self, t: TrafficC):
        for f, _ in TrafficC._fields_:
            setattr(self, f, int(getattr(t, f)))


class Mark:
    """counters.rs:91-111"""

    def __init__(self, handle):
        self._h = handle

    def since(self, earlier: "Mark") -> float:
        s = C.c_double()
        check(lib.marin_mark_since(self._h, earlier._h, C.byref(s)))
        return s.value

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_mark_free(self._h)
            self._h = None


def _f32(values) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(values, dtype=np.float32)).ravel()


class Gpu:
    """crates/cuda/src/gpu.rs:68-76 and its methods (gpu.rs, ops.rs, quant.rs, attention.rs)."""

    def __init__(self):
        h = _out()
        check(lib.marin_gpu_new(C.byref(h)))
        self._h = h

    @property
    def handle(self):
        return self._h

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_gpu_free(self._h)
            self._h = None

    # ---- context ----
    def info(self) -> dict:
        i = GpuInfo()
        check(lib.marin_gpu_info_get(self._h, C.byref(i)))
        return {"name": i.name.decode(), "arch": i.arch.decode(), "compute_units": i.compute_units,
                "free_bytes": i.free_bytes, "total_bytes": i.total_bytes}

    def synchronize(self) -> None:
        check(lib.marin_gpu_synchronize(self._h))

    def bind_to_thread(self) -> None:
        check(lib.marin_gpu_bind_to_thread(self._h))

    def set_fast_attention(self, on: bool) -> None:
        lib.marin_set_fast_attention(self._h, int(bool(on)))

    # ---- dense bf16 matrices (gpu.rs:248, matmul.rs, ops.rs:55) ----
    def upload_matrix(self, rows: int, cols: int, bits) -> "DeviceMatrix":
        a = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16)).ravel()
        h = _out()
        check(lib.marin_upload_matrix(self._h, rows, cols, a.ctypes.data, a.size, C.byref(h)))
        return DeviceMatrix(h)

    def embed(self, table: "DeviceMatrix", ids, scratch: "Tokens", out: "Buffer") -> None:
        a = np.ascontiguousarray(np.asarray(ids, dtype=np.uint32)).ravel()
        check(lib.marin_embed(self._h, table.handle, a.ctypes.data, a.size, scratch._h, out.handle))

    def matmul(self, w: "DeviceMatrix", x: "Buffer", tokens: int, out: "Buffer") -> None:
        check(lib.marin_matmul(self._h, w.handle, x.handle, tokens, out.handle))

    def matmul_precise(self, w: "DeviceMatrix", x: "Buffer", tokens: int, out: "Buffer") -> None:
        check(lib.marin_matmul_precise(self._h, w.handle, x.handle, tokens, out.handle))

    def matmul_pair(self, ws, x: "Buffer", tokens: int, ys) -> None:
        (w0, w1), (y0, y1) = ws, ys
        check(lib.marin_matmul_pair(self._h, w0.handle, w1.handle, x.handle, tokens, y0.handle, y1.handle))

    def matmul_triple(self, ws, x: "Buffer", tokens: int, ys) -> None:
        (w0, w1, w2), (y0, y1, y2) = ws, ys
        check(lib.marin_matmul_triple(self._h, w0.handle, w1.handle, w2.handle, x.handle, tokens, y0.handle,
                                      y1.handle, y2.handle))

    def traffic(self) -> Traffic:
        t = TrafficC()
        check(lib.marin_gpu_traffic(self._h, C.byref(t)))
        return Traffic(t)

    def mark(self) -> Mark:
        h = _out()
        check(lib.marin_mark_new(self._h, C.byref(h)))
        return Mark(h)

    # ---- buffers ----
    def zeros(self, length: int) -> Buffer:
        h = _out()
        check(lib.marin_buffer_zeros(self._h, length, C.byref(h)))
        return Buffer(self, h)

    def upload(self, values) -> Buffer:
        a = _f32(values)
        h = _out()
        check(lib.marin_buffer_upload(self._h, a.ctypes.data, a.size, C.byref(h)))
        return Buffer(self, h)

    def upload_into(self, values, dst: Buffer) -> None:
        a = _f32(values)
        check(lib.marin_buffer_upload_into(self._h, a.ctypes.data, a.size, dst.handle))

    def download(self, buf: Buffer) -> np.ndarray:
        if buf.dtype != Dtype.F32:
            return self.download_typed(buf)
        out = np.empty(len(buf), np.float32)
        check(lib.marin_buffer_download(self._h, buf.handle, out.ctypes.data, out.size))
        return out

    def download_range(self, buf: Buffer, start: int, length: int) -> np.ndarray:
        out = np.empty(length, np.float32)
        check(lib.marin_buffer_download_range(self._h, buf.handle, start, length, out.ctypes.data))
        return out

    def copy_range_into(self, src: Buffer, start: int, dst: Buffer) -> None:
        check(lib.marin_buffer_copy_range_into(self._h, src.handle, start, dst.handle))

    def copy_into_range(self, src: Buffer, dst: Buffer, start: int) -> None:
        check(lib.marin_buffer_copy_into_range(self._h, src.handle, dst.handle, start))

    def typed(self, dtype: Dtype, length: int = 0, host=None) -> Buffer:
        h = _out()
        if host is not None:
            host = np.ascontiguousarray(host, dtype=_NP[Dtype(dtype)]).ravel()
            length = host.size
        check(lib.marin_buffer_new_typed(self._h, int(dtype), length,
                                         host.ctypes.data if host is not None else None, C.byref(h)))
        return Buffer(self, h)

    def download_typed(self, buf: Buffer) -> np.ndarray:
        out = np.empty(len(buf), _NP[buf.dtype])
        check(lib.marin_buffer_download_raw(self._h, buf.handle, out.ctypes.data, out.nbytes))
        return out

    def tokens(self, capacity: int) -> Tokens:
        h = _out()
        check(lib.marin_tokens_new(self._h, capacity, C.byref(h)))
        return Tokens(h, capacity)

    # ---- quantized matrices (quant.rs) ----
    def upload_quantized(self, rows: int, cols: int, bits: int, group: int, codes, scales,
                         bf16_scales: bool = False) -> DeviceQuantMatrix:
        """Gpu::upload_quantized (quant.rs:56-97); ``codes``/``scales`` as tensor::Quantized holds them."""
        codes = np.ascontiguousarray(codes, np.uint8).ravel()
        h = _out()
        if bf16_scales:
            scales = np.ascontiguousarray(scales, np.uint16).ravel()
            check(lib.marin_upload_quantized_bf16_scales(self._h, rows, cols, bits, group, codes.ctypes.data,
                                                         codes.size, scales.ctypes.data, scales.size, C.byref(h)))
        else:
            scales = np.ascontiguousarray(scales, np.float32).ravel()
            check(lib.marin_upload_quantized(self._h, rows, cols, bits, group, codes.ctypes.data, codes.size,
                                             scales.ctypes.data, scales.size, C.byref(h)))
        return DeviceQuantMatrix(h)

    def quantized_synthetic(self, rows: int, cols: int, group: int, seed: int, stream: int,
                            std: float = 0.02) -> DeviceQuantMatrix:
        """A synthetic int8 matrix generated and quantized on the device (extension; see include/marin_hip.h)."""
        h = _out()
        check(lib.marin_quantized_synthetic(self._h, rows, cols, group, seed, stream, std, C.byref(h)))
        return DeviceQuantMatrix(h)

    def probe_copy(self, nbytes: int, reps: int = 20) -> float:
        """Mean seconds of one device-to-device copy of `nbytes` by a plain streaming kernel (extension; see
        include/marin_hip.h)."""
        sec = C.c_double()
        check(lib.marin_probe_copy(self._h, nbytes, reps, C.byref(sec)))
        return sec.value

    def time_matmul_bf16(self, mats, x: Buffer, tokens: int, out: Buffer, reps: int = 200) -> float:
        """Mean seconds per bf16 product over a graph of `reps` products cycling through `mats` (extension; see
        include/marin_hip.h)."""
        n = len(mats)
        arr = (C.c_void_p * n)(*[mm._h.value if hasattr(mm._h, "value") else mm._h for mm in mats])
        sec = C.c_double()
        check(lib.marin_time_matmul_bf16(self._h, arr, n, x.handle, tokens, out.handle, reps, C.byref(sec)))
        return sec.value

    # ---- mixture of experts (config 4; see include/marin_hip.h) ----
    def moe_route(self, logits: Buffer, tokens: int, experts: int, k: int, renorm: bool, ids: Buffer,
                  weights: Buffer) -> None:
        check(lib.marin_moe_route(self._h, logits.handle, tokens, experts, k, int(renorm), ids.handle,
                                  weights.handle))

    def moe_ffn(self, gate_up: DeviceQuantMatrix, down: DeviceQuantMatrix, x: Buffer, norm, eps: float,
                ids: Buffer, weights: Buffer, tokens: int, experts: int, k: int, act: Buffer, out: Buffer) -> None:
        check(lib.marin_moe_ffn(self._h, gate_up._h, down._h, x.handle, norm.handle if norm is not None else None,
                                eps, ids.handle, weights.handle, tokens, experts, k, act.handle, out.handle))

    def moe_stack_time(self, gate_ups, downs, x: Buffer, norm, eps: float, ids: Buffer, weights: Buffer,
                       tokens: int, experts: int, k: int, act: Buffer, out: Buffer, reps: int = 10, part: int = 0) -> float:
        n = len(gate_ups)
        gu = (C.c_void_p * n)(*[m._h.value if hasattr(m._h, "value") else m._h for m in gate_ups])
        dn = (C.c_void_p * n)(*[m._h.value if hasattr(m._h, "value") else m._h for m in downs])
        sec = C.c_double()
        check(lib.marin_moe_stack_time(self._h, n, gu, dn, x.handle, norm.handle if norm is not None else None,
                                       eps, ids.handle, weights.handle, tokens, experts, k, act.handle, out.handle,
                                       part, reps, C.byref(sec)))
        return sec.value

    def embed_quant(self, table: DeviceQuantMatrix, ids, scratch: Tokens, out: Buffer) -> None:
        ids = np.ascontiguousarray(ids, np.uint32).ravel()
        check(lib.marin_embed_quant(self._h, table._h, ids.ctypes.data if ids.size else None, ids.size,
                                    scratch._h, out.handle))

    def matmul_quant(self, w: DeviceQuantMatrix, x: Buffer, tokens: int, out: Buffer) -> None:
        check(lib.marin_matmul_quant(self._h, w._h, x.handle, tokens, out.handle))

    def matmul_quant_precise(self, w: DeviceQuantMatrix, x: Buffer, tokens: int, out: Buffer) -> None:
        check(lib.marin_matmul_quant_precise(self._h, w._h, x.handle, tokens, out.handle))

    def matmul_quant_bf16(self, w: DeviceQuantMatrix, x: Buffer, tokens: int, out: Buffer) -> None:
        check(lib.marin_matmul_quant_bf16(self._h, w._h, x.handle, tokens, out.handle))

    def matmul_quant_bf16_noalloc(self, w: DeviceQuantMatrix, x: Buffer, tokens: int, out: Buffer) -> None:
        """matmul_quant_bf16 with its scratch in the library's fixed device array (no allocation; see
        include/marin_hip.h)."""
        check(lib.marin_matmul_quant_bf16_noalloc(self._h, w._h, x.handle, tokens, out.handle))

    # ---- elementwise (ops.rs) ----
    def rms_norm(self, x: Buffer, weight: Buffer, eps: float) -> None:
        check(lib.marin_rms_norm(self._h, x.handle, weight.handle, eps))

    def rms_norm_into(self, x: Buffer, weight: Buffer, out: Buffer, eps: float) -> None:
        check(lib.marin_rms_norm_into(self._h, x.handle, weight.handle, out.handle, eps))

    def rope(self, x: Buffer, heads: int, head_dim: int, start: int, theta: float) -> None:
        check(lib.marin_rope(self._h, x.handle, heads, head_dim, start, theta))

    def silu_mul(self, gate: Buffer, up: Buffer) -> None:
        check(lib.marin_silu_mul(self._h, gate.handle, up.handle))

    def add(self, a: Buffer, b: Buffer) -> None:
        check(lib.marin_add(self._h, a.handle, b.handle))

    # ---- attention (attention.rs:90) ----
    def attention(self, q: Buffer, kv: "DeviceKv", layer: int, heads: int, tokens: int, out: Buffer) -> None:
        check(lib.marin_attention(self._h, q.handle, kv._h, layer, heads, tokens, out.handle))


class DeviceKv:
    """crates/cuda/src/kv.rs:11-346: pages of PAGE_TOKENS positions in slabs of SLAB_PAGES, mapped on first use."""

    def __init__(self, gpu: Gpu, layers: int, dims, capacity: int, fmt: KvFormat = KvFormat.F32):
        heads, kv_heads, head_dim = dims
        h = _out()
        check(lib.marin_kv_new(gpu.handle, layers, heads, kv_heads, head_dim, capacity, int(fmt), C.byref(h)))
        self._h = h
        self._gpu = gpu
        self.format = KvFormat(fmt)

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_kv_free(self._h)
            self._h = None

    def write(self, gpu: Gpu, layer: int, keys: Buffer, values: Buffer) -> None:
        check(lib.marin_kv_write(gpu.handle, self._h, layer, keys.handle, values.handle))

    def advance(self, tokens: int) -> None:
        check(lib.marin_kv_advance(self._h, tokens))

    def truncate(self, length: int) -> None:
        check(lib.marin_kv_truncate(self._h, length))

    def clear(self) -> None:
        lib.marin_kv_clear(self._h)

    def len(self) -> int:
        return int(lib.marin_kv_len(self._h))

    def is_empty(self) -> bool:
        return bool(lib.marin_kv_is_empty(self._h))

    def kv_format(self) -> KvFormat:
        return KvFormat(int(lib.marin_kv_format_of(self._h)))

    def auxiliary_bytes(self) -> int:
        return int(lib.marin_kv_auxiliary_bytes(self._h))

    def capacity(self) -> int:
        return int(lib.marin_kv_capacity(self._h))

    def pages_held(self) -> int:
        return int(lib.marin_kv_pages_held(self._h))

    def pages_in_use(self) -> int:
        return int(lib.marin_kv_pages_in_use(self._h))

    def bytes_held(self) -> int:
        return int(lib.marin_kv_bytes_held(self._h))

    def page_bytes(self) -> int:
        return int(lib.marin_kv_page_bytes(self._h))

    def slab_bytes(self) -> int:
        return int(lib.marin_kv_slab_bytes(self._h))

    def page_ids(self) -> list:
        n = int(lib.marin_kv_page_ids(self._h, None, 0))
        out = (C.c_size_t * max(n, 1))()
        lib.marin_kv_page_ids(self._h, out, n)
        return [int(out[i]) for i in range(n)]

    @staticmethod
    def startup_bytes(layers: int, dims, capacity: int, fmt: KvFormat) -> int:
        heads, kv_heads, head_dim = dims
        return int(lib.marin_kv_startup_bytes(layers, heads, kv_heads, head_dim, capacity, int(fmt)))


class PagePool:
    """A page pool shared by a batch of sequences (the paged-attention benchmark layout; no reference counterpart)."""

    def __init__(self, gpu: Gpu, pages: int, page_tokens: int, kv_heads: int, head_dim: int,
                 fmt: KvFormat = KvFormat.BF16):
        h = _out()
        check(lib.marin_page_pool_new(gpu.handle, pages, page_tokens, kv_heads, head_dim, int(fmt), C.byref(h)))
        self._h = h
        self._gpu = gpu
        self.pages, self.page_tokens, self.kv_heads, self.head_dim, self.format = (pages, page_tokens, kv_heads,
                                                                                   head_dim, KvFormat(fmt))

    def __del__(self):
        if getattr(self, "_h", None) and alive():
            lib.marin_page_pool_free(self._h)
            self._h = None

    def write_page(self, page: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data)
        check(lib.marin_page_pool_write(self._gpu.handle, self._h, page, data.ctypes.data, data.nbytes))

    def attention(self, q: Buffer, tables: np.ndarray, ctx_lens, heads: int, out: Buffer) -> None:
        tables = np.ascontiguousarray(tables, np.uint32)
        ctx = np.ascontiguousarray(ctx_lens, np.uint32)
        check(lib.marin_paged_attention_batch(self._gpu.handle, q.handle, self._h, tables.ctypes.data,
                                              tables.shape[1], ctx.ctypes.data, ctx.size, heads, out.handle))


__all__ = ["Gpu", "Buffer", "Tokens", "DeviceQuantMatrix", "DeviceMatrix", "DeviceKv", "KvFormat", "PagePool", "Dtype",
           "PAGE_TOKENS", "SLAB_PAGES", "pages_for", "HipError", "Unavailable", "Driver", "Shape", "KvMemory",
           "Overflow", "SelfCheck", "Unsupported", "check"]
