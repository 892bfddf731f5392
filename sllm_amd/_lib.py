"""ctypes loader for libsllm_moe.so (the HIP C-ABI declared in
include/sllm_moe.h).

Same lazy-load contract as the reference's bindings
(kernels/_q4_cuda.py:46-105): the library is opened once, the symbol set is
probed, a failure is latched, and `available()` reports the outcome. Unlike
the reference's DeepSeek binding there is NO numpy fallback: every wrapper
raises RuntimeError when the library is missing, so a GPU run can never pass
on a silent CPU path.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import (POINTER, Structure, c_char_p, c_float, c_int, c_long,
                    c_ubyte, c_void_p)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib",
                        "libsllm_moe.so")

F = POINTER(c_float)
I = POINTER(c_int)
U8 = POINTER(c_ubyte)
P = c_void_p


class QwenArgs(Structure):
    """Mirror of `sllm_moe_qwen_args` (include/sllm_moe.h)."""
    _fields_ = [
        ("T", c_int), ("H", c_int), ("E", c_int), ("I", c_int), ("Is", c_int),
        ("topk", c_int), ("mode", c_int), ("out_f32", c_int),
        ("logits_given", c_int), ("wdtype", c_int), ("renorm_eps", c_float),
        ("x", P), ("logits", P), ("router_w", P),
        ("wg", P), ("wg_s", P), ("wu", P), ("wu_s", P), ("wd", P), ("wd_s", P),
        ("sg", P), ("sg_s", P), ("su", P), ("su_s", P), ("sd", P), ("sd_s", P),
        ("sgl", P), ("out", P), ("logits_out", P), ("w_out", P),
        ("ids_out", P), ("counts_out", P), ("workspace", P),
        ("workspace_bytes", c_long), ("stream", P), ("stage_events", P),
        ("wgu_packed", P), ("wd_packed", P), ("sgu_packed", P), ("sd_packed", P),
        ("sorted_out", P), ("inv_pos_out", P), ("router_bias", P),
    ]


class DeepseekArgs(Structure):
    """Mirror of `sllm_moe_ds_args` (include/sllm_moe.h)."""
    _fields_ = [
        ("T", c_int), ("H", c_int), ("E", c_int), ("I", c_int), ("Is", c_int),
        ("topk", c_int), ("mode", c_int), ("out_f32", c_int),
        ("logits_given", c_int), ("n_group", c_int), ("topk_group", c_int),
        ("scoring", c_int), ("route_scale", c_float),
        ("swiglu_limit", c_float),
        ("x", P), ("logits", P), ("router_w", P), ("bias", P),
        ("w1", P), ("w1_s", P), ("w3", P), ("w3_s", P), ("w2", P), ("w2_s", P),
        ("s1", P), ("s1_s", P), ("s3", P), ("s3_s", P), ("s2", P), ("s2_s", P),
        ("out", P), ("logits_out", P), ("w_out", P), ("ids_out", P),
        ("counts_out", P), ("workspace", P), ("workspace_bytes", c_long),
        ("stream", P), ("stage_events", P),
        ("w13_packed", P), ("w13_s_packed", P), ("w2_packed", P),
        ("w2_s_packed", P), ("s13_packed", P), ("s2_packed", P),
        ("token_ids", P), ("tid2eid", P), ("vocab", c_int),
        ("sorted_out", P), ("inv_pos_out", P),
    ]


# name -> (restype, argtypes); every symbol declared in include/sllm_moe.h
SIGNATURES = {
    "sllm_last_error": (c_char_p, []),
    "sllm_q4_last_error": (c_char_p, []),
    "sllm_fp8_last_error": (c_char_p, []),
    "sllm_ds_last_error": (c_char_p, []),
    "sllm_moe_last_error": (c_char_p, []),
    "sllm_device_count": (c_int, []),
    "sllm_buf_new": (c_void_p, [c_long]),
    "sllm_buf_free": (c_int, [P]),
    "sllm_buf_h2d": (c_int, [P, F, c_long]),
    "sllm_buf_h2d_raw": (c_int, [P, P, c_long]),
    "sllm_buf_d2h": (c_int, [F, P, c_long]),
    "sllm_buf_d2h_raw": (c_int, [P, P, c_long]),
    "sllm_mem_free_bytes": (c_long, []),
    "sllm_sync": (c_int, []),
    "sllm_host_new": (c_void_p, [c_long]),
    "sllm_host_free": (c_int, [P]),
    "sllm_copy_async": (c_int, [P, P, c_long, P]),
    "sllm_stream_sync": (c_int, [P]),
    "sllm_host_f32_to_bf16": (c_int, [P, P, c_long]),
    "sllm_event_new": (c_void_p, []),
    "sllm_event_free": (c_int, [P]),
    "sllm_event_record": (c_int, [P, P]),
    "sllm_event_sync": (c_int, [P]),
    "sllm_event_elapsed_ms": (c_float, [P, P]),
    "sllm_memset": (c_int, [P, c_int, c_long, P]),
    "sllm_buf_copy": (c_int, [P, P, c_long, P]),
    "sllm_fill_normal": (c_int, [P, c_long, ctypes.c_ulonglong, c_float, P]),
    "sllm_q4_moe_router": (c_int, [F, F, I, c_int, c_int, c_int]),
    "sllm_q4_moe_router_dev": (c_int, [P, P, P, c_int, c_int, c_int]),
    "sllm_q4_swiglu": (c_int, [F, F, F, c_long]),
    "sllm_q4_swiglu_dev": (c_int, [P, P, P, c_long]),
    "sllm_q4_gemv_rows": (c_int, [F, F, F, c_int, c_int, c_int, c_int, c_float]),
    "sllm_q4_gemv_rows_dev": (c_int, [P, P, P, c_int, c_int, c_int, c_int,
                                      c_float]),
    "sllm_q4_axpy_rows": (c_int, [F, F, F, c_int, c_int]),
    "sllm_q4_axpy_rows_dev": (c_int, [P, P, P, c_int, c_int]),
    "sllm_q4_shared_gate_accum": (c_int, [F, F, F, c_int, c_int]),
    "sllm_q4_shared_gate_accum_dev": (c_int, [P, P, P, c_int, c_int]),
    "sllm_fp8_gemm": (c_int, [F, U8, F, F, c_int, c_int, c_int, c_int, c_int]),
    "sllm_fp8_gemm_dev": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int,
                                  c_int]),
    "sllm_ds_fp4_gemm": (c_int, [F, F, F, c_int, c_int, c_int, c_float, F]),
    "sllm_ds_fp4_gemm_packed": (c_int, [F, F, P, P, c_int, c_int, c_int,
                                        c_int]),
    "sllm_ds_fp4_gemm_packed_dev": (c_int, [P, P, P, P, c_int, c_int, c_int,
                                            c_int]),
    "sllm_gemm_ex": (c_int, [P, c_int, P, P, c_int, c_int, c_int]),
    "sllm_silu_mul": (c_int, [P, P, P, c_long, c_int]),
    "sllm_moe_router_gemm": (c_int, [P, P, P, c_int, c_int, c_int, P]),
    "sllm_moe_route_hash": (c_int, [P, P, P, c_int, P, P, c_int, c_int, c_int,
                                    c_int, c_float, P]),
    "sllm_moe_route_softmax": (c_int, [P, P, P, c_int, c_int, c_int, c_float,
                                       P]),
    "sllm_moe_route_grouped": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int,
                                       c_int, c_int, c_float, P]),
    "sllm_moe_permute_scratch_bytes": (c_long, [c_int, c_int]),
    "sllm_moe_permute": (c_int, [P, c_int, c_int, c_int, P, P, P, P, P, P,
                                 c_int, P, P]),
    "sllm_moe_act_quant": (c_int, [P, c_int, c_int, c_int, P, P, P, P, P]),
    "sllm_moe_combine": (c_int, [P, c_int, P, c_int, P, c_int, c_int, c_int,
                                 P, P]),
    "sllm_moe_packed_bytes": (c_long, [c_int, c_int, c_int, c_int, c_int]),
    "sllm_moe_packed_scale_bytes": (c_long, [c_int, c_int, c_int, c_int]),
    "sllm_moe_pack_weights": (c_int, [c_int, c_int, P, P, P, P, c_int, c_int,
                                      c_int, P, P, P]),
    "sllm_moe_stream_status": (c_int, [P]),
    "sllm_moe_tile_bound": (c_long, [c_long, c_int, c_int]),
    "sllm_moe_stream_grid": (c_long, [c_long, c_int]),
    "sllm_moe_stream_dec_grid": (c_long, [c_long, c_int, c_long]),
    "sllm_moe_plan_query": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int,
                                    c_int, c_int, c_int, c_void_p, c_int]),
    "sllm_quantize_weight_fp8": (c_int, [P, c_int, c_int, c_int, P, P, P]),
    "sllm_quantize_weight_mxfp4": (c_int, [P, c_int, c_int, P, P, P]),
    "sllm_moe_qwen_workspace_bytes": (c_long, [POINTER(QwenArgs)]),
    "sllm_moe_qwen_forward": (c_int, [POINTER(QwenArgs)]),
    "sllm_moe_qwen_graph_new": (c_void_p, [POINTER(QwenArgs)]),
    "sllm_moe_graph_launch": (c_int, [P, P]),
    "sllm_moe_graph_free": (c_int, [P]),
    "sllm_moe_qwen_forward_noalloc_max_bytes": (c_long, []),
    "sllm_moe_qwen_forward_noalloc": (c_int, [POINTER(QwenArgs)]),
    "sllm_moe_ds_workspace_bytes": (c_long, [POINTER(DeepseekArgs)]),
    "sllm_moe_ds_forward": (c_int, [POINTER(DeepseekArgs)]),
}

_lib = None
_lib_failed = False
_lib_error = ""


def _setup():
    global _lib, _lib_failed, _lib_error
    if _lib is not None or _lib_failed:
        return _lib
    try:
        if not os.path.isfile(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} not built (run: python -m sllm_amd.build)")
        lib = ctypes.CDLL(LIB_PATH)
        missing = [n for n in SIGNATURES if not hasattr(lib, n)]
        if missing:
            raise AttributeError(f"symbols missing from {LIB_PATH}: {missing}")
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    except Exception as exc:  # latched, reported by lib()
        _lib_failed = True
        _lib_error = f"{type(exc).__name__}: {exc}"
        _lib = None
    return _lib


def available() -> bool:
    """True when libsllm_moe.so loads and exports the full symbol set."""
    return _setup() is not None


def lib():
    """The loaded library; raises RuntimeError (never falls back) if absent."""
    l = _setup()
    if l is None:
        raise RuntimeError(f"libsllm_moe.so unavailable: {_lib_error}")
    return l


def last_error() -> str:
    try:
        return lib().sllm_last_error().decode(errors="replace")
    except Exception:
        return _lib_error or "library unavailable"


def check(rc: int, what: str = "sllm") -> None:
    """Reference error contract (kernels/_q4_cuda.py:127-136)."""
    if rc != 0:
        raise RuntimeError(f"{what} failed rc={rc}: {last_error()}")
