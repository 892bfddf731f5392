"""Qwen MoE kernel surface over libsllm_moe.so.

Mirrors the MoE subset of the reference's kernels/_q4_cuda.py:
moe_router (:281-290), swiglu (:293-299), axpy_rows (:302-307),
shared_gate_accum (:310-315) and their device-pointer variants
(:405-424), with the same signatures, return values and RuntimeError
contract. `available()` / `dev_available()` keep the reference's probe
semantics; there is no fallback.
"""

from __future__ import annotations

from ctypes import POINTER, c_float, c_int

import numpy as np

from . import _lib
from .runtime import ptr


def available() -> bool:
    return _lib.available()


def dev_available() -> bool:
    return _lib.available()


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a):
    return a.ctypes.data_as(POINTER(c_float))


def _check(rc: int) -> None:
    _lib.check(rc, "q4 kernel")


def moe_router(logits, topk):
    """softmax -> top-k (ties to the lower id) -> renorm; returns
    (w (n,k) float32, ids (n,k) int32)."""
    logits = _f(logits)
    n, E = logits.shape
    w = np.empty((n, topk), np.float32)
    ids = np.empty((n, topk), np.int32)
    _check(_lib.lib().sllm_q4_moe_router(_fp(logits), _fp(w),
                                         ids.ctypes.data_as(POINTER(c_int)),
                                         n, E, int(topk)))
    return w, ids


def swiglu(g, u) -> np.ndarray:
    g, u = _f(g), _f(u)
    out = np.empty_like(g)
    _check(_lib.lib().sllm_q4_swiglu(_fp(g), _fp(u), _fp(out), int(g.size)))
    return out


def axpy_rows(out, y, w) -> np.ndarray:
    out, y, w = _f(out).copy(), _f(y), _f(w)
    _check(_lib.lib().sllm_q4_axpy_rows(_fp(out), _fp(y), _fp(w),
                                        out.shape[0], out.shape[1]))
    return out


def shared_gate_accum(out, shared, g) -> np.ndarray:
    out, shared, g = _f(out).copy(), _f(shared), _f(g)
    _check(_lib.lib().sllm_q4_shared_gate_accum(_fp(out), _fp(shared), _fp(g),
                                                out.shape[0], out.shape[1]))
    return out


def gemv_rows(A, W, post=0, scale=1.0) -> np.ndarray:
    """out (rows, O) = A (rows, K) . W (O, K)^T, then post 1: silu(x /
    scale), 2: sigmoid(x / scale) (ref kernels/_q4_cuda.py:167-175)."""
    A, W = _f(A), _f(W)
    rows, K = A.shape
    O = W.shape[0]
    out = np.empty((rows, O), np.float32)
    _check(_lib.lib().sllm_q4_gemv_rows(_fp(A), _fp(W), _fp(out), rows, K, O,
                                        int(post), float(scale)))
    return out


def gemv_rows_dev(A, W, out, rows, K, O, post=0, scale=1.0):
    _check(_lib.lib().sllm_q4_gemv_rows_dev(ptr(A), ptr(W), ptr(out), rows, K,
                                            O, int(post), float(scale)))


def moe_router_dev(logits, w_out, id_out, n, E, topk):
    _check(_lib.lib().sllm_q4_moe_router_dev(ptr(logits), ptr(w_out),
                                             ptr(id_out), n, E, int(topk)))


def swiglu_dev(g, u, out, n):
    _check(_lib.lib().sllm_q4_swiglu_dev(ptr(g), ptr(u), ptr(out), int(n)))


def axpy_rows_dev(out, y, w, n, H):
    _check(_lib.lib().sllm_q4_axpy_rows_dev(ptr(out), ptr(y), ptr(w), n, H))


def shared_gate_accum_dev(out, shared, g, n, H):
    _check(_lib.lib().sllm_q4_shared_gate_accum_dev(ptr(out), ptr(shared),
                                                    ptr(g), n, H))
