"""DeepSeek FP4 expert linear over libsllm_moe.so.

Mirrors kernels/_deepseek_cuda.py:fp4_moe_linear (:79-97): x (M,K) times a
packed E2M1 weight (N, K/2) with per-row-per-32 E8M0 scales -> (M,N) fp32.
Two deliberate differences: the FP4 bytes go to the device as they are (the
reference dequantizes them on the host, :89-94), and there is no numpy
fallback -- a missing library raises RuntimeError.
"""

from __future__ import annotations

from ctypes import POINTER, c_float, c_void_p

import numpy as np

from . import _lib
from .runtime import ptr


def available() -> bool:
    return _lib.available()


def fp4_moe_linear(x, packed, scale_u8, fp4_block_w: int = 32) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scale_u8 = np.ascontiguousarray(scale_u8, dtype=np.uint8)
    M, K = x.shape
    N = packed.shape[0]
    if packed.shape != (N, K // 2):
        raise ValueError(f"packed {packed.shape} must be (N, K/2) for K={K}")
    if scale_u8.shape != (N, -(-K // fp4_block_w)):
        raise ValueError(f"scale {scale_u8.shape} must be (N, ceil(K/{fp4_block_w}))")
    out = np.empty((M, N), np.float32)
    _lib.check(_lib.lib().sllm_ds_fp4_gemm_packed(
        out.ctypes.data_as(POINTER(c_float)), x.ctypes.data_as(POINTER(c_float)),
        packed.ctypes.data_as(c_void_p), scale_u8.ctypes.data_as(c_void_p),
        M, N, K, int(fp4_block_w)), "sllm_ds_fp4_gemm_packed")
    return out


def fp4_gemm_dequantized(x, w) -> np.ndarray:
    """The reference's sllm_ds_fp4_gemm contract: fp32 x (M,K) times an
    already-dequantized fp32 weight (N,K) (kernels/cuda/deepseek.cu:57-73)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    F = POINTER(c_float)
    _lib.check(_lib.lib().sllm_ds_fp4_gemm(out.ctypes.data_as(F), x.ctypes.data_as(F),
                                           w.ctypes.data_as(F), x.shape[0], w.shape[0],
                                           x.shape[1], 1.0, None), "sllm_ds_fp4_gemm")
    return out


def fp4_moe_linear_dev(x, packed, scale_u8, out, M, N, K, fp4_block_w=32):
    _lib.check(_lib.lib().sllm_ds_fp4_gemm_packed_dev(ptr(out), ptr(x), ptr(packed),
                                                      ptr(scale_u8), M, N, K,
                                                      int(fp4_block_w)),
               "sllm_ds_fp4_gemm_packed_dev")
