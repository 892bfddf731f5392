"""FP8 E4M3 block-dequant GEMM over libsllm_moe.so.

Mirrors kernels/_fp8_cuda.py (fp8_gemm :87-106, fp8_gemm_dev :108-112):
C (M,N) = A (M,K) @ dequant(B)^T, B (N,K) uint8 e4m3 with fp32 block
inverse scales. The scale orientation is the one the reference's own test
pins (tests/test_fp8_gemm.py:49-55 compares against
loaders/fp8.dequant_weight_blocked): (ceil(N/block_h), ceil(K/block_w)),
W[n,k] = e4m3(B[n,k]) * scale_inv[n // block_h, k // block_w].
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float

import numpy as np

from . import _lib
from .runtime import ptr


def available() -> bool:
    return _lib.available()


def fp8_gemm(A, B, scale_inv, block_h=128, block_w=128) -> np.ndarray:
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.uint8)
    scale_inv = np.ascontiguousarray(scale_inv, dtype=np.float32)
    M, K = A.shape
    N = B.shape[0]
    if B.shape != (N, K):
        raise ValueError(f"fp8_gemm: weight codes {B.shape} do not have the activation's K={K} columns")
    want = (-(-N // block_h), -(-K // block_w))
    if scale_inv.shape != want:
        raise ValueError(f"scale_inv {scale_inv.shape} != {want}")
    out = np.empty((M, N), np.float32)
    _lib.check(_lib.lib().sllm_fp8_gemm(
        A.ctypes.data_as(POINTER(c_float)),
        B.ctypes.data_as(POINTER(ctypes.c_ubyte)),
        scale_inv.ctypes.data_as(POINTER(c_float)),
        out.ctypes.data_as(POINTER(c_float)), M, N, K, int(block_h),
        int(block_w)), "fp8 kernel")
    return out


def fp8_gemm_dev(A, B, scale_inv, out, M, N, K, block_h=128, block_w=128):
    _lib.check(_lib.lib().sllm_fp8_gemm_dev(ptr(A), ptr(B), ptr(scale_inv),
                                            ptr(out), M, N, K, int(block_h),
                                            int(block_w)), "fp8 kernel")
