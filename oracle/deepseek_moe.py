"""DeepSeek-style MoE layer (oracle side).

Restates ref/deepseek_v4.py:522-570:

- gate_scores (:522-531): sigmoid evaluated in fp64 and rounded to fp32;
  softmax (fp64 internal, :84-97); sqrt(softplus) (:534-537).
- moe_route (:540-561): the per-expert bias is added to the scores for
  SELECTION only; the weights are the un-biased scores of the selected
  experts, normalised by their sum unless scoring is softmax, then times
  route_scale. The reference sorts with np.argsort's default (non-stable)
  kind, which leaves exact ties unpinned; this oracle breaks them to the
  lower expert id, the order the device router produces.
- expert_ffn (:564-570): gate = x W1^T, up = x W3^T; when limit > 0,
  up = clip(up, -L, L) and gate = min(gate, L); y = (silu(gate) * up) W2^T.
- combine per upstream ref/hf_sources/dsv4/model.py:684-699: every
  (token, slot) contributes weight * expert(x) (the reference's
  Block.moe at ref/deepseek_v4.py:1084 picks the slot of the first routed
  row for every row -- a known defect this build does not reproduce), then
  the un-gated shared expert is added.

Group-limited top-k (absent from the reference; DeepSeek-V3 noaux_tc
semantics): the biased scores are viewed as (T, G, E/G); a group's score is
the sum of its two largest biased scores; the topk_group best groups are
kept (ties to the lower group id) and the top-k is taken over experts of
kept groups only. Pinned by reduction to the plain route at G=1, brute-force
enumeration on tiny inputs, and its invariants (tests/test_oracle_deepseek.py).

The quantized layer (moe_layer_mxfp4) inserts the upstream quantization
points: activation quant per 1x128 with a power-of-two (ue8m0) scale before
W1/W3 and before W2; routed weights MXFP4 (e2m1 + e8m0 per 32 along K) via
quant.fp4_block_gemm; the shared expert FP8 128x128 via
quant.fp8_block_gemm. As in upstream Expert.forward
(ref/hf_sources/dsv4/model.py:652-660) the routing weight multiplies the
SwiGLU output before it is quantized for W2.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import quant


def silu(x):
    """ref/deepseek_v4.py:79-81 (fp32)."""
    x = np.asarray(x, np.float32)
    return (x / (1.0 + np.exp(-x, dtype=np.float32))).astype(np.float32)


def softplus(x):
    """ref/deepseek_v4.py:534-537 (fp64 internal, fp32 out)."""
    x = np.asarray(x, np.float64)
    return (np.log1p(np.exp(-np.abs(x))) + np.maximum(x, 0.0)).astype(np.float32)


def gate_scores(logits, scoring: str = "sigmoid") -> np.ndarray:
    """ref/deepseek_v4.py:522-531 on precomputed fp32 logits."""
    s = np.asarray(logits, np.float32)
    if scoring == "softmax":
        x = s.astype(np.float64)
        e = np.exp(x - x.max(-1, keepdims=True))
        return (e / e.sum(-1, keepdims=True)).astype(np.float32)
    if scoring == "sigmoid":
        return (1.0 / (1.0 + np.exp(-s.astype(np.float64)))).astype(np.float32)
    if scoring == "sqrtsoftplus":
        return np.sqrt(softplus(s))
    raise ValueError(f"unknown scoring {scoring}")


def _stable_topk_desc(v, k):
    return np.argsort(-v, axis=-1, kind="stable")[..., :k]


def select_experts(biased, top_k: int, n_group: int = 1, topk_group: int = 1):
    """Indices (T, k) of the selected experts in descending biased-score
    order (ties to the lower id), optionally group-limited."""
    biased = np.asarray(biased, np.float32)
    T, E = biased.shape
    if n_group <= 1:
        return _stable_topk_desc(biased, top_k)
    if E % n_group:
        raise ValueError("E must be a multiple of n_group")
    g = biased.reshape(T, n_group, E // n_group)
    top2 = -np.sort(-g, axis=-1)[..., :2]
    gscore = (top2[..., 0] + top2[..., 1]).astype(np.float32)   # (T, G)
    keep = _stable_topk_desc(gscore, topk_group)                 # (T, kg)
    mask = np.zeros((T, n_group), bool)
    np.put_along_axis(mask, keep, True, axis=-1)
    masked = np.where(np.repeat(mask, E // n_group, axis=1), biased,
                      np.float32(-np.inf))
    return _stable_topk_desc(masked, top_k)


def hash_select(token_ids, tid2eid):
    """Hash-layer expert ids, ref/deepseek_v4.py:545-552 (text branch):
    tid2eid[clip(token_ids, 0, vocab - 1)] -> (T, k) int64, in table order."""
    table = np.asarray(tid2eid, np.int64)
    ids = np.clip(np.asarray(token_ids, np.int64), 0, table.shape[0] - 1)
    return table[ids]


def moe_route(logits, bias, top_k: int, scoring: str = "sigmoid",
              route_scale: float = 1.0, n_group: int = 1, topk_group: int = 1,
              token_ids=None, tid2eid=None):
    """ref/deepseek_v4.py:540-561 on fp32 logits -> (weights (T, k) f32,
    idx (T, k) int64). With tid2eid (a hash layer) the ids come from the
    token-id table and the bias is not used (:545-552); otherwise the
    biased top-k, optionally group-limited."""
    scores = gate_scores(logits, scoring)
    if tid2eid is not None:
        idx = hash_select(token_ids, tid2eid)
        if idx.shape[1] != top_k:
            raise ValueError("tid2eid must have top_k columns")
    else:
        biased = scores + np.asarray(bias, np.float32) if bias is not None else scores
        idx = select_experts(biased, top_k, n_group, topk_group).astype(np.int64)
    w = np.take_along_axis(scores, idx, axis=-1)
    if scoring != "softmax":
        w = w / w.sum(-1, keepdims=True)
    w = w * np.float32(route_scale)
    return w.astype(np.float32), idx


def expert_ffn(x, w1, w3, w2, limit: float):
    """ref/deepseek_v4.py:564-570 (fp32)."""
    gate = (x @ w1.T).astype(np.float32)
    up = (x @ w3.T).astype(np.float32)
    if limit > 0:
        up = np.clip(up, -limit, limit)
        gate = np.minimum(gate, np.float32(limit))
    return ((silu(gate) * up) @ w2.T).astype(np.float32)


def moe_block_forward(x, logits, bias, experts, shared, top_k, limit,
                      scoring="sigmoid", route_scale=1.0, n_group=1,
                      topk_group=1, token_ids=None, tid2eid=None):
    """Un-quantized layer with the upstream combine. ``experts`` maps
    e -> (w1, w3, w2) fp32 (a callable or a sequence); ``shared`` is
    (w1, w3, w2) or None."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    w, idx = moe_route(logits, bias, top_k, scoring, route_scale, n_group,
                       topk_group, token_ids, tid2eid)
    y = np.zeros((T, top_k, H), np.float32)
    get = experts if callable(experts) else (lambda e: experts[e])
    for e in np.unique(idx):
        t, j = np.nonzero(idx == e)
        y[t, j] = expert_ffn(x[t], *get(int(e)), limit)
    out = np.zeros((T, H), np.float32)
    for j in range(top_k):
        out += w[:, j:j + 1] * y[:, j]
    if shared is not None:
        out += expert_ffn(x, *shared, limit)
    return out


@dataclass
class DeepseekMxfp4Weights:
    """Routed experts MXFP4: w1/w3 (E, I, H/2) packed e2m1 + (E, I, H/32)
    e8m0; w2 (E, H, I/2) + (E, H, I/32). Shared expert FP8 e4m3 with fp32
    power-of-two 128x128 block scales: s1/s3 (I_s, H), s2 (H, I_s).
    router_w (E, H) f32 holding bf16 values, bias (E,) f32."""
    router_w: np.ndarray
    bias: np.ndarray
    w1_p: np.ndarray
    w1_s: np.ndarray
    w3_p: np.ndarray
    w3_s: np.ndarray
    w2_p: np.ndarray
    w2_s: np.ndarray
    s1_q: np.ndarray = None
    s1_s: np.ndarray = None
    s3_q: np.ndarray = None
    s3_s: np.ndarray = None
    s2_q: np.ndarray = None
    s2_s: np.ndarray = None

    @property
    def has_shared(self) -> bool:
        return self.s1_q is not None


def _swiglu_clamped(g, u, limit):
    if limit > 0:
        u = np.clip(u, -limit, limit)
        g = np.minimum(g, np.float32(limit))
    return (silu(g) * u).astype(np.float32)


def moe_layer_mxfp4(x, logits, W: DeepseekMxfp4Weights, top_k: int,
                    limit: float, scoring="sigmoid", route_scale=1.0,
                    n_group=1, topk_group=1, return_parts=False,
                    token_ids=None, tid2eid=None):
    """The quantized DeepSeek-style layer. x (T, H) float32 holding bf16
    values; logits (T, E) fp32. out = sum_{j ascending} y_j + shared(x)
    where y_j = W2(q(w_j * swiglu(W1 q(x), W3 q(x))))."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    w, idx = moe_route(logits, W.bias, top_k, scoring, route_scale, n_group,
                       topk_group, token_ids, tid2eid)
    xq, sx = quant.act_quant(x, pow2=True)
    y = np.zeros((T, top_k, H), np.float32)
    for e in np.unique(idx):
        t, j = np.nonzero(idx == e)
        g = quant.fp4_block_gemm(xq[t], sx[t], W.w1_p[e], W.w1_s[e])
        u = quant.fp4_block_gemm(xq[t], sx[t], W.w3_p[e], W.w3_s[e])
        h = (_swiglu_clamped(g, u, limit) * w[t, j][:, None]).astype(np.float32)
        hq, hs = quant.act_quant(h, pow2=True)
        y[t, j] = quant.fp4_block_gemm(hq, hs, W.w2_p[e], W.w2_s[e])
    out = np.zeros((T, H), np.float32)
    for j in range(top_k):
        out += y[:, j]
    shared_y = None
    if W.has_shared:
        g = quant.fp8_block_gemm(xq, sx, W.s1_q, W.s1_s)
        u = quant.fp8_block_gemm(xq, sx, W.s3_q, W.s3_s)
        hq, hs = quant.act_quant(_swiglu_clamped(g, u, limit), pow2=True)
        shared_y = quant.fp8_block_gemm(hq, hs, W.s2_q, W.s2_s)
        out += shared_y
    if return_parts:
        return out, dict(w=w, ids=idx, y=y, shared_y=shared_y, xq=xq, sx=sx)
    return out
