"""Qwen-style MoE layer (oracle side).

Restates ref/qwen4_exp.py:118-184 (with silu / sigmoid from
ref/qwen3_5.py:28-37):

- softmax_rows: fp32 row softmax, exp(x - max) / sum.
- moe_route: top-k by a stable descending sort of the probabilities (ties go
  to the lower expert id), weights renormalised as p / (sum p + fp32(1e-20)).
- swiglu_mlp: down(silu(x gate^T) * (x up^T)), weights stored (out, in).
- moe_block_forward: sum_j w_j * expert_{ids_j}(x) + sigmoid(x W_sg^T) *
  shared(x), the literal per-token loop of the reference.

plus the quantized layer this build defines (moe_layer_fp8): the same
routing and combine with the upstream FP8 quantization points inserted,
activation quant per 1x128 (scale amax/448) before the gate/up GEMM, the
SwiGLU output re-quantized per 1x128 before the down GEMM, and block-scaled
accumulation (oracle.quant). Routing weights multiply the down-projection
output, as in ref/qwen4_exp.py:175-179.

Pinned by tests/test_oracle_qwen.py: the reference's own MoE tests
(tests/test_ref_qwen4_exp.py:88-136 restated: route order/renorm, the
all-zero-logit tie, block vs a manual fp64 loop) and the quantized layer
against the un-quantized one (closed-form error bound) and against a
dequantize-then-matmul restatement.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import quant
from .permute import permute


def silu(x):
    """ref/qwen3_5.py:28-29: x * 1/(1 + exp(-x))."""
    return x * (1.0 / (1.0 + np.exp(-x)))


def sigmoid(x):
    """ref/qwen3_5.py:36-37."""
    return 1.0 / (1.0 + np.exp(-x))


def softmax_rows(x) -> np.ndarray:
    """ref/qwen4_exp.py:118-122 (fp32)."""
    x = np.asarray(x, np.float32)
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def moe_route(logits, top_k: int, eps: float = 1e-20):
    """ref/qwen4_exp.py:125-140 -> (weights (n, k) f32, ids (n, k) int64)."""
    p = softmax_rows(logits)
    n, e = p.shape
    if top_k > e:
        raise ValueError(f"top_k {top_k} > num_experts {e}")
    ids = np.argsort(-p, axis=-1, kind="stable")[:, :top_k].astype(np.int64)
    w = np.take_along_axis(p, ids, axis=-1)
    w = w / (w.sum(-1, keepdims=True) + np.float32(eps))
    return w.astype(np.float32), ids


def swiglu_mlp(x, gate_w, up_w, down_w):
    """ref/qwen4_exp.py:143-150."""
    return (silu(x @ gate_w.T) * (x @ up_w.T)) @ down_w.T


def moe_block_forward(x, router_w, eg, eu, ed, sg, sgl, su, sd, top_k,
                      eps: float = 1e-20):
    """ref/qwen4_exp.py:153-184, the literal per-token loop (fp32)."""
    n, h = x.shape
    weights, ids = moe_route(x @ router_w.T, top_k, eps)
    out = np.zeros((n, h), np.float32)
    for i in range(n):
        for j in range(top_k):
            e = ids[i, j]
            y = swiglu_mlp(x[i:i + 1], eg[e], eu[e], ed[e])
            out[i] += weights[i, j] * y[0]
    if su is not None:
        shared = swiglu_mlp(x, sg, su, sd)
        out += sigmoid(x @ sgl.T) * shared.astype(np.float32)
    return out


def moe_block_grouped(x, logits, eg, eu, ed, top_k, shared=None,
                      eps: float = 1e-20):
    """Expert-grouped form of moe_block_forward (same math, BLAS GEMMs with
    M = tokens per expert; the CPU-baseline form). ``shared`` is None or a
    tuple (sg, su, sd, sgl). ``logits`` are the fp32 router logits."""
    x = np.asarray(x, np.float32)
    n, h = x.shape
    w, ids = moe_route(logits, top_k, eps)
    contrib = np.zeros((n, top_k, h), np.float32)
    for e in np.unique(ids):
        t, j = np.nonzero(ids == e)
        contrib[t, j] = swiglu_mlp(x[t], eg[e], eu[e], ed[e])
    out = np.zeros((n, h), np.float32)
    for j in range(top_k):
        out += w[:, j:j + 1] * contrib[:, j]
    if shared is not None:
        sg, su, sd, sgl = shared
        out += sigmoid(x @ sgl.T) * swiglu_mlp(x, sg, su, sd)
    return out


@dataclass
class QwenFp8Weights:
    """Quantized layer weights, reference tensor orientation (out, in).

    e4m3 codes (uint8) with fp32 block scales of shape
    (ceil(out/128), ceil(in/128)):
    wg_q/wu_q (E, I, H), wd_q (E, H, I); shared sg_q/su_q (Is, H),
    sd_q (H, Is); router_w (E, H) and sgl (1, H) are float32 holding bf16
    values (None when the layer has no shared expert).
    """
    router_w: np.ndarray
    wg_q: np.ndarray
    wg_s: np.ndarray
    wu_q: np.ndarray
    wu_s: np.ndarray
    wd_q: np.ndarray
    wd_s: np.ndarray
    sg_q: np.ndarray = None
    sg_s: np.ndarray = None
    su_q: np.ndarray = None
    su_s: np.ndarray = None
    sd_q: np.ndarray = None
    sd_s: np.ndarray = None
    sgl: np.ndarray = None

    @property
    def has_shared(self) -> bool:
        return self.su_q is not None


def expert_fp8(xq, sx, gq, gs, uq, us, dq, ds):
    """One quantized SwiGLU expert on pre-quantized rows:
    g, u = block GEMMs; h = silu(g) * u (fp32); h re-quantized per 1x128;
    y = block GEMM with the down weight."""
    g = quant.fp8_block_gemm(xq, sx, gq, gs)
    u = quant.fp8_block_gemm(xq, sx, uq, us)
    h = (silu(g) * u).astype(np.float32)
    hq, hs = quant.act_quant(h)
    return quant.fp8_block_gemm(hq, hs, dq, ds)


def moe_layer_fp8(x, logits, W: QwenFp8Weights, top_k: int,
                  eps: float = 1e-20, return_parts: bool = False):
    """The quantized Qwen-style layer.

    x (T, H) float32 holding bf16 values; logits (T, E) fp32 router logits
    (the routing boundary: pass the logits the device produced to compare
    routing bit for bit). Returns out (T, H) fp32, combined as
    out = sum_{j ascending} w_j * y_j, then + sigmoid(x sgl^T) * shared(x).
    """
    x = np.asarray(x, np.float32)
    T, H = x.shape
    E = W.wg_q.shape[0]
    w, ids = moe_route(logits, top_k, eps)
    perm = permute(ids, E)
    xq, sx = quant.act_quant(x)
    y = np.zeros((T, top_k, H), np.float32)
    for e in np.nonzero(perm["counts"])[0]:
        t, j = np.nonzero(ids == e)
        y[t, j] = expert_fp8(xq[t], sx[t], W.wg_q[e], W.wg_s[e], W.wu_q[e],
                             W.wu_s[e], W.wd_q[e], W.wd_s[e])
    out = np.zeros((T, H), np.float32)
    for j in range(top_k):
        out += w[:, j:j + 1] * y[:, j]
    gate = None
    shared_y = None
    if W.has_shared:
        shared_y = expert_fp8(xq, sx, W.sg_q, W.sg_s, W.su_q, W.su_s,
                              W.sd_q, W.sd_s)
        gate = sigmoid((x @ W.sgl.T).astype(np.float32))   # (T, 1)
        out += gate * shared_y
    if return_parts:
        return out, dict(w=w, ids=ids, perm=perm, xq=xq, sx=sx, y=y,
                         gate=gate, shared_y=shared_y)
    return out


def moe_layer_fp8_dequant(x, logits, W: QwenFp8Weights, top_k: int,
                          eps: float = 1e-20):
    """The same layer WITHOUT activation quantization: each touched expert's
    weights dequantized to fp32 (codecs.dequant_fp8_block), then the
    un-quantized SwiGLU and combine of moe_block_grouped. This is the
    semantics of the decode path (fp32 activations against block-scaled
    weights) and the information-only comparison for the prefill path."""
    from .codecs import dequant_fp8_block
    x = np.asarray(x, np.float32)
    n, h = x.shape
    w, ids = moe_route(logits, top_k, eps)
    contrib = np.zeros((n, top_k, h), np.float32)
    for e in np.unique(ids):
        t, j = np.nonzero(ids == e)
        contrib[t, j] = swiglu_mlp(x[t], dequant_fp8_block(W.wg_q[e], W.wg_s[e]),
                                   dequant_fp8_block(W.wu_q[e], W.wu_s[e]),
                                   dequant_fp8_block(W.wd_q[e], W.wd_s[e]))
    out = np.zeros((n, h), np.float32)
    for j in range(top_k):
        out += w[:, j:j + 1] * contrib[:, j]
    if W.has_shared:
        sh = swiglu_mlp(x, dequant_fp8_block(W.sg_q, W.sg_s),
                        dequant_fp8_block(W.su_q, W.su_s),
                        dequant_fp8_block(W.sd_q, W.sd_s))
        out += sigmoid((x @ W.sgl.T).astype(np.float32)) * sh
    return out
