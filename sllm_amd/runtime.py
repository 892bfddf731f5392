"""Device buffers and sync over the HIP C-ABI.

Mirrors the device-tensor half of the reference's kernels/_sllm_cuda.py
(DeviceBuffer :200-258, DeviceView :261-280, to_bf16 :283-287,
to_device :290-296, alloc / sync :377-386, T_F32 / T_BF16 / alloc_n /
gemm_ex :490-506) with the same names and argument meaning, backed by
libsllm_moe.so.
"""

from __future__ import annotations

import weakref
from ctypes import c_void_p

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


def _byte_count(n) -> int:
    """A strictly positive Python int (bools rejected), else ValueError."""
    if isinstance(n, bool) or not isinstance(n, int) or n < 1:
        raise ValueError(f"device allocation size must be an int >= 1, got {n!r}")
    return n


def _release(addr: int) -> None:
    # weakref.finalize callback: runs once, at free() or at collection
    try:
        _lib.lib().sllm_buf_free(c_void_p(addr))
    except Exception:
        pass


class DeviceBuffer:
    """Device allocation owned by a Python object.

    Interface of ref kernels/_sllm_cuda.py:200-258 (``.ptr``, ``.nbytes``,
    ``upload``, ``upload_raw``, ``copy_host``, ``free``); the allocation is
    released by a ``weakref.finalize`` hook, so an explicit ``free()`` and
    garbage collection share one release path and it runs exactly once.
    """

    def __init__(self, nbytes: int):
        self.nbytes = _byte_count(nbytes)
        addr = _lib.lib().sllm_buf_new(self.nbytes)
        if not addr:
            raise RuntimeError(
                f"could not allocate {self.nbytes} device bytes ({_lib.last_error()})")
        self._addr = int(addr)
        self._release = weakref.finalize(self, _release, self._addr)

    @property
    def alive(self) -> bool:
        return self._release.alive

    @property
    def ptr(self) -> int:
        if not self._release.alive:
            raise RuntimeError(f"use of a released {self.nbytes}-byte device buffer")
        return self._addr

    def free(self) -> None:
        """Release the device memory now (later calls are no-ops)."""
        if self._release.alive:
            self._release.detach()
            _lib.check(_lib.lib().sllm_buf_free(c_void_p(self._addr)), "sllm_buf_free")

    def _host_to_device(self, arr: np.ndarray, fn: str) -> None:
        if arr.nbytes != self.nbytes:
            raise ValueError(f"{fn}: host array holds {arr.nbytes} bytes, the device "
                             f"buffer {self.nbytes}")
        _lib.check(getattr(_lib.lib(), fn)(c_void_p(self.ptr), arr.ctypes.data_as(c_void_p),
                                          arr.nbytes), fn)

    def copy_host_raw(self, dtype, shape=None) -> np.ndarray:
        """The device bytes, copied to the host and viewed as ``dtype``."""
        host = np.empty(self.nbytes, np.uint8)
        _lib.check(_lib.lib().sllm_buf_d2h_raw(host.ctypes.data_as(c_void_p),
                                               c_void_p(self.ptr), self.nbytes),
                   "sllm_buf_d2h_raw")
        host = host.view(dtype)
        return host if shape is None else host.reshape(shape)

    def copy_host(self) -> np.ndarray:
        """The device bytes as a flat float32 array."""
        if self.nbytes & 3:
            raise ValueError(f"{self.nbytes} bytes is not a whole number of float32")
        return self.copy_host_raw(np.float32)

    def upload(self, arr: np.ndarray) -> None:
        """Overwrite the buffer with ``arr`` converted to float32."""
        self._host_to_device(np.ascontiguousarray(arr, dtype=np.float32), "sllm_buf_h2d_raw")

    def upload_raw(self, arr: np.ndarray) -> None:
        """Overwrite the buffer with the bytes of ``arr`` (any dtype)."""
        self._host_to_device(np.ascontiguousarray(arr), "sllm_buf_h2d_raw")


class DeviceView:
    """Window ``[off_bytes, off_bytes + nbytes)`` of a DeviceBuffer, not owning
    it (interface of ref kernels/_sllm_cuda.py:261-280). It holds a reference
    to the buffer, and its ``ptr`` goes through the buffer's, so a window on
    a released buffer raises instead of yielding a stale address."""

    def __init__(self, base: DeviceBuffer, off_bytes: int, nbytes: int):
        if not base.alive:
            raise RuntimeError("window on a released device buffer")
        if min(off_bytes, nbytes) < 0 or off_bytes + nbytes > base.nbytes:
            raise ValueError(f"window [{off_bytes}, {off_bytes + nbytes}) exceeds "
                             f"the {base.nbytes}-byte buffer")
        self._base, self._off, self.nbytes = base, off_bytes, nbytes

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
    """A new device buffer holding ``arr`` as float32 (interface of ref
    kernels/_sllm_cuda.py:290-296; an empty array gets a 4-byte buffer)."""
    host = np.ascontiguousarray(arr, dtype=np.float32)
    return to_device_raw(host)


def to_device_raw(arr: np.ndarray) -> DeviceBuffer:
    """A new device buffer holding the bytes of ``arr`` (uint8 codes, bf16
    bits, ...); arrays under 4 bytes fill the front of a 4-byte buffer."""
    host = np.ascontiguousarray(arr)
    buf = DeviceBuffer(max(host.nbytes, 4))
    if host.nbytes:
        _lib.check(_lib.lib().sllm_buf_h2d_raw(c_void_p(buf.ptr), host.ctypes.data_as(c_void_p),
                                               host.nbytes), "sllm_buf_h2d_raw")
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


def silu_mul(g, u, out, out_type: int = T_F32) -> None:
    """out = silu(g) * u over g's floats, stored as `out_type` (fp32 or bf16)
    (ref kernels/_sllm_cuda.py:529-532)."""
    n = g.nbytes // 4
    _lib.check(_lib.lib().sllm_silu_mul(ptr(g), ptr(u), ptr(out), int(n),
                                        int(out_type)), "sllm_silu_mul")


def gemm_ex(a, w, c, m: int, n: int, k: int, atype: int = T_F32) -> None:
    """c (m,n) fp32 = a (m,k) . w (n,k)^T with a, w in dtype `atype`
    (ref kernels/_sllm_cuda.py:503-506)."""
    _lib.check(_lib.lib().sllm_gemm_ex(ptr(a), int(atype), ptr(w), ptr(c),
                                       int(m), int(n), int(k)), "sllm_gemm_ex")
