"""Device buffers and sync over the HIP C-ABI.

Mirrors the device-tensor half of the reference's kernels/_sllm_cuda.py
(DeviceBuffer :200-258, DeviceView :261-280, to_bf16 :283-287,
to_device :290-296, alloc / sync :377-386, T_F32 / T_BF16 / alloc_n /
gemm_ex :490-506) with the same names and argument meaning, backed by
libsllm_moe.so.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_void_p

import numpy as np

from . import _lib

T_F32 = 0
T_BF16 = 1


def ptr(obj):
    """Device address of a DeviceBuffer / DeviceView / torch tensor / int
    (None stays None)."""
    if obj is None:
        return None
    if isinstance(obj, int):
        return obj
    if hasattr(obj, "data_ptr"):
        return int(obj.data_ptr())
    if hasattr(obj, "ptr"):
        return int(obj.ptr)
    raise TypeError(f"not a device buffer: {type(obj).__name__}")


def stream_handle(stream):
    """hipStream_t of a torch stream / int / None (None = default stream)."""
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return int(stream.cuda_stream)


def device_count() -> int:
    return int(_lib.lib().sllm_device_count())


def mem_free_bytes() -> int:
    return int(_lib.lib().sllm_mem_free_bytes())


def sync() -> None:
    """Blocking device synchronisation (one per step is the caller's job)."""
    _lib.check(_lib.lib().sllm_sync(), "sllm_sync")


class DeviceBuffer:
    """Owning device allocation (ref kernels/_sllm_cuda.py:200-258)."""

    def __init__(self, nbytes: int):
        if not isinstance(nbytes, int) or nbytes <= 0:
            raise ValueError("nbytes must be a positive int")
        self.nbytes = nbytes
        self._ptr = _lib.lib().sllm_buf_new(nbytes)
        if not self._ptr:
            raise RuntimeError("sllm_buf_new failed: " + _lib.last_error())
        self._closed = False

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def ptr(self) -> int:
        if self._closed:
            raise RuntimeError("DeviceBuffer already freed")
        return self._ptr

    def free(self) -> None:
        if not getattr(self, "_closed", True):
            _lib.check(_lib.lib().sllm_buf_free(c_void_p(self._ptr)), "sllm_buf_free")
            self._closed = True

    def copy_host(self) -> np.ndarray:
        """float32 copy of the device bytes."""
        if self.nbytes % 4:
            raise ValueError("non-float32-sized buffer")
        y = np.empty(self.nbytes // 4, np.float32)
        _lib.check(_lib.lib().sllm_buf_d2h(y.ctypes.data_as(POINTER(c_float)),
                                           c_void_p(self.ptr), self.nbytes),
                   "sllm_buf_d2h")
        return y

    def copy_host_raw(self, dtype, shape=None) -> np.ndarray:
        """Copy of the device bytes viewed as `dtype` (e.g. uint8, int32)."""
        y = np.empty(self.nbytes, np.uint8)
        _lib.check(_lib.lib().sllm_buf_d2h_raw(y.ctypes.data_as(c_void_p),
                                               c_void_p(self.ptr), self.nbytes),
                   "sllm_buf_d2h_raw")
        y = y.view(dtype)
        return y.reshape(shape) if shape is not None else y

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr, dtype=np.float32)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: {arr.nbytes} != {self.nbytes}")
        _lib.check(_lib.lib().sllm_buf_h2d(c_void_p(self.ptr),
                                           arr.ctypes.data_as(POINTER(c_float)),
                                           arr.nbytes), "sllm_buf_h2d")

    def upload_raw(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes != self.nbytes:
            raise ValueError(f"size mismatch: {arr.nbytes} != {self.nbytes}")
        _lib.check(_lib.lib().sllm_buf_h2d_raw(c_void_p(self.ptr),
                                               arr.ctypes.data_as(c_void_p),
                                               arr.nbytes), "sllm_buf_h2d_raw")


class DeviceView:
    """Non-owning byte window into a DeviceBuffer (ref :261-280)."""

    def __init__(self, base: DeviceBuffer, off_bytes: int, nbytes: int):
        if off_bytes < 0 or nbytes < 0 or off_bytes + nbytes > base.nbytes:
            raise ValueError("view out of range")
        self._base = base
        self._off = off_bytes
        self.nbytes = nbytes
        base.ptr

    @property
    def ptr(self) -> int:
        return self._base.ptr + self._off


def to_bf16(arr: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even
    (ref :283-287)."""
    u = np.asarray(arr, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return np.ascontiguousarray(((u + 0x7FFF + ((u >> 16) & 1)) >> 16)
                                .astype(np.uint16))


def to_device(arr: np.ndarray) -> DeviceBuffer:
    """Upload a float32 array (ref :290-296)."""
    arr = np.ascontiguousarray(arr, dtype=np.float32)
    buf = DeviceBuffer(max(arr.nbytes, 4))
    if arr.nbytes:
        buf.upload(arr)
    return buf


def to_device_raw(arr: np.ndarray) -> DeviceBuffer:
    """Upload the raw bytes of any array (uint8 codes, bf16 bits, ...)."""
    arr = np.ascontiguousarray(arr)
    buf = DeviceBuffer(max(arr.nbytes, 4))
    if arr.nbytes:
        _lib.check(_lib.lib().sllm_buf_h2d_raw(c_void_p(buf.ptr),
                                               arr.ctypes.data_as(c_void_p),
                                               arr.nbytes), "sllm_buf_h2d_raw")
    return buf


def alloc(nfloats: int) -> DeviceBuffer:
    return DeviceBuffer(int(nfloats) * 4)


def alloc_n(nbytes: int) -> DeviceBuffer:
    return DeviceBuffer(int(nbytes))


class Event:
    """hipEvent on the library's side of the process (torch must not touch
    the GPU in a process that uses this library: it bundles its own HIP
    runtime)."""

    def __init__(self):
        self._ev = _lib.lib().sllm_event_new()
        if not self._ev:
            raise RuntimeError("sllm_event_new failed: " + _lib.last_error())

    def record(self, stream=None) -> None:
        _lib.check(_lib.lib().sllm_event_record(c_void_p(self._ev),
                                                stream_handle(stream)), "event")

    def synchronize(self) -> None:
        _lib.check(_lib.lib().sllm_event_sync(c_void_p(self._ev)), "event")

    def elapsed_ms(self, end: "Event") -> float:
        ms = _lib.lib().sllm_event_elapsed_ms(c_void_p(self._ev), c_void_p(end._ev))
        if ms < 0:
            raise RuntimeError("hipEventElapsedTime failed: " + _lib.last_error())
        return float(ms)

    def __del__(self):
        try:
            _lib.lib().sllm_event_free(c_void_p(self._ev))
        except Exception:
            pass


def fill_normal(buf, n: int, seed: int, std: float = 1.0, stream=None) -> None:
    """buf[:n] (fp32) ~ N(0, std^2), deterministic in (seed, index)."""
    _lib.check(_lib.lib().sllm_fill_normal(ptr(buf), int(n), int(seed) & (2**64 - 1),
                                           float(std), stream_handle(stream)),
               "sllm_fill_normal")


def copy(dst, src, nbytes: int, stream=None) -> None:
    """Device-to-device copy of ``nbytes`` by the library's copy kernel."""
    _lib.check(_lib.lib().sllm_buf_copy(ptr(dst), ptr(src), int(nbytes),
                                        stream_handle(stream)), "sllm_buf_copy")


def memset(buf, value: int, nbytes: int, stream=None) -> None:
    _lib.check(_lib.lib().sllm_memset(ptr(buf), int(value), int(nbytes),
                                      stream_handle(stream)), "sllm_memset")


def gemm_ex(a, w, c, m: int, n: int, k: int, atype: int = T_F32) -> None:
    """c (m,n) fp32 = a (m,k) . w (n,k)^T with a, w in dtype `atype`
    (ref kernels/_sllm_cuda.py:503-506)."""
    _lib.check(_lib.lib().sllm_gemm_ex(ptr(a), int(atype), ptr(w), ptr(c),
                                       int(m), int(n), int(k)), "sllm_gemm_ex")
