"""Pins oracle.deepseek_moe: scoring closed forms, the selection-only bias,
group-limited top-k by reduction (G=1) and brute force, the upstream
combine, and the quantized layer against a dequantize restatement."""
import itertools

import numpy as np

from oracle import codecs, quant
from oracle import deepseek_moe as dm


def test_sigmoid_scores_fp64_then_fp32():
    rng = np.random.default_rng(0)
    lg = (rng.standard_normal((7, 33)) * 4).astype(np.float32)
    s = dm.gate_scores(lg, "sigmoid")
    want = (1.0 / (1.0 + np.exp(-lg.astype(np.float64)))).astype(np.float32)
    np.testing.assert_array_equal(s, want)
    sp = dm.gate_scores(lg, "sqrtsoftplus")
    np.testing.assert_allclose(sp, np.sqrt(np.log1p(np.exp(lg.astype(np.float64)))), rtol=1e-6)


def test_bias_selects_but_does_not_weight():
    lg = np.zeros((1, 4), np.float32)               # all scores 0.5
    bias = np.float32([0.0, 0.3, 0.0, 0.2])
    w, idx = dm.moe_route(lg, bias, 2, route_scale=2.5)
    np.testing.assert_array_equal(idx[0], [1, 3])
    np.testing.assert_allclose(w[0], [1.25, 1.25], rtol=1e-7)


def test_route_matches_closed_form():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal((20, 16)).astype(np.float32)
    bias = (rng.standard_normal(16) * 0.1).astype(np.float32)
    w, idx = dm.moe_route(lg, bias, 4, route_scale=2.5)
    s = 1 / (1 + np.exp(-lg.astype(np.float64)))
    for t in range(20):
        key = (s[t].astype(np.float32) + bias)
        order = sorted(range(16), key=lambda e: (-key[e], e))[:4]
        np.testing.assert_array_equal(idx[t], order)
        ws = s[t, order] / s[t, order].sum() * 2.5
        np.testing.assert_allclose(w[t], ws, rtol=2e-6)


def test_hash_route_closed_form():
    """Hash layers (ref/deepseek_v4.py:545-552): ids from the token-id table
    with out-of-range ids clipped, table order kept, bias ignored; weights
    are the scores of those ids, renormalized unless softmax."""
    rng = np.random.default_rng(5)
    T, E, k, V = 12, 16, 4, 9
    lg = rng.standard_normal((T, E)).astype(np.float32)
    tid2eid = np.stack([rng.permutation(E)[:k] for _ in range(V)]).astype(np.int32)
    tok = rng.integers(-3, V + 3, T)                 # some out of range
    bias = np.full(E, 100.0, np.float32)             # would dominate a top-k
    for scoring in ("sigmoid", "softmax", "sqrtsoftplus"):
        w, idx = dm.moe_route(lg, bias, k, scoring, 1.5, token_ids=tok,
                              tid2eid=tid2eid)
        s = dm.gate_scores(lg, scoring)
        for t in range(T):
            row = tid2eid[min(max(int(tok[t]), 0), V - 1)]
            np.testing.assert_array_equal(idx[t], row)
            ws = s[t, row].astype(np.float64)
            if scoring != "softmax":
                ws = ws / ws.sum()
            np.testing.assert_allclose(w[t], ws * 1.5, rtol=2e-6)


def _brute_group(b, k, G, kg):
    E = b.size
    gs = E // G
    gscore = []
    for g in range(G):
        vals = sorted(b[g * gs:(g + 1) * gs].tolist(), reverse=True)
        gscore.append(np.float32(vals[0]) + np.float32(vals[1]))
    kept = sorted(range(G), key=lambda g: (-gscore[g], g))[:kg]
    cand = [e for e in range(E) if e // gs in kept]
    return sorted(cand, key=lambda e: (-b[e], e))[:k], kept


def test_group_limited_brute_force_and_invariants():
    rng = np.random.default_rng(2)
    T, E, G, kg, k = 40, 32, 8, 3, 5
    b = rng.standard_normal((T, E)).astype(np.float32)
    b[0, :] = 0.5                                   # a full tie row
    b[1, 4:8] = b[1, 0:4]                           # tied groups
    idx = dm.select_experts(b, k, G, kg)
    for t in range(T):
        want, kept = _brute_group(b[t], k, G, kg)
        np.testing.assert_array_equal(idx[t], want)
        assert all(e // (E // G) in kept for e in idx[t])


def test_group_limited_reduces_at_one_group():
    rng = np.random.default_rng(3)
    b = rng.standard_normal((30, 64)).astype(np.float32)
    np.testing.assert_array_equal(dm.select_experts(b, 8, 1, 1),
                                  dm.select_experts(b, 8))
    # keeping every group is the plain top-k too
    np.testing.assert_array_equal(dm.select_experts(b, 8, 8, 8),
                                  dm.select_experts(b, 8))


def test_group_limited_tiny_enumeration():
    # exhaustive over every 2-of-4 group choice on a tiny case: the selected
    # set maximises the biased score sum subject to lying in the kept groups
    rng = np.random.default_rng(4)
    for _ in range(50):
        b = rng.standard_normal((1, 8)).astype(np.float32)
        idx = dm.select_experts(b, 2, 4, 2)[0]
        _, kept = _brute_group(b[0], 2, 4, 2)
        best = max(itertools.combinations([e for e in range(8) if e // 2 in kept], 2),
                   key=lambda c: b[0, list(c)].sum())
        assert set(idx) == set(best)


def test_combine_matches_upstream_loop():
    # upstream model.py:689-698: for each expert, rows where it was picked
    rng = np.random.default_rng(5)
    T, H, E, I, k = 6, 8, 5, 4, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    bias = np.zeros(E, np.float32)
    ex = [tuple((rng.standard_normal(s) * 0.3).astype(np.float32)
                for s in ((I, H), (I, H), (H, I))) for _ in range(E)]
    sh = tuple((rng.standard_normal(s) * 0.3).astype(np.float32) for s in ((I, H), (I, H), (H, I)))
    got = dm.moe_block_forward(x, lg, bias, ex, sh, k, limit=5.0, route_scale=2.5)
    w, idx = dm.moe_route(lg, bias, k, route_scale=2.5)
    want = np.zeros((T, H))
    for e in range(E):
        tt, jj = np.nonzero(idx == e)
        for t, j in zip(tt, jj):
            want[t] += w[t, j] * dm.expert_ffn(x[t:t + 1], *ex[e], 5.0)[0]
    want += dm.expert_ffn(x, *sh, 5.0)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


def test_expert_ffn_limit_clamps():
    x = np.ones((1, 2), np.float32)
    w1 = np.full((1, 2), 10.0, np.float32)   # gate = 20 -> min(20, 5) = 5
    w3 = np.full((1, 2), -10.0, np.float32)  # up = -20 -> -5
    w2 = np.ones((1, 1), np.float32)
    y = dm.expert_ffn(x, w1, w3, w2, 5.0)
    np.testing.assert_allclose(y, [[5.0 / (1 + np.exp(-5.0)) * -5.0]], rtol=1e-6)
    y0 = dm.expert_ffn(x, w1, w3, w2, 0.0)
    np.testing.assert_allclose(y0, [[20.0 / (1 + np.exp(-20.0)) * -20.0]], rtol=1e-6)


def make_small_mxfp4_layer(rng, T=24, H=256, E=8, I=128, shared=True):
    bf = codecs.round_bf16
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)

    def q4(n, k):
        return quant.quantize_weight_mxfp4((rng.standard_normal((n, k)) * 0.02).astype(np.float32))

    def q8(n, k):
        return quant.quantize_weight_fp8_block((rng.standard_normal((n, k)) * 0.02).astype(np.float32), pow2=True)
    w1 = [q4(I, H) for _ in range(E)]
    w3 = [q4(I, H) for _ in range(E)]
    w2 = [q4(H, I) for _ in range(E)]
    W = dm.DeepseekMxfp4Weights(
        router_w=rw, bias=bias,
        w1_p=np.stack([a for a, _ in w1]), w1_s=np.stack([b for _, b in w1]),
        w3_p=np.stack([a for a, _ in w3]), w3_s=np.stack([b for _, b in w3]),
        w2_p=np.stack([a for a, _ in w2]), w2_s=np.stack([b for _, b in w2]))
    if shared:
        (W.s1_q, W.s1_s), (W.s3_q, W.s3_s), (W.s2_q, W.s2_s) = q8(I, H), q8(I, H), q8(H, I)
    return x, W


def test_mxfp4_layer_matches_dequant_restatement():
    rng = np.random.default_rng(6)
    x, W = make_small_mxfp4_layer(rng)
    lg = x @ W.router_w.T
    kw = dict(top_k=3, limit=10.0, route_scale=2.5, n_group=4, topk_group=2)
    got = dm.moe_layer_mxfp4(x, lg, W, **kw)
    w, idx = dm.moe_route(lg, W.bias, 3, "sigmoid", 2.5, 4, 2)
    xd = quant.act_dequant(*quant.act_quant(x, pow2=True))
    want = np.zeros_like(x)
    for t in range(x.shape[0]):
        for j in range(3):
            e = idx[t, j]
            g = xd[t:t + 1] @ codecs.dequant_fp4_block(W.w1_p[e], W.w1_s[e]).T
            u = xd[t:t + 1] @ codecs.dequant_fp4_block(W.w3_p[e], W.w3_s[e]).T
            u = np.clip(u, -10, 10)
            g = np.minimum(g, 10)
            h = (g / (1 + np.exp(-g)) * u * w[t, j]).astype(np.float32)
            hd = quant.act_dequant(*quant.act_quant(h, pow2=True))
            want[t] += (hd @ codecs.dequant_fp4_block(W.w2_p[e], W.w2_s[e]).T)[0]
    g = xd @ codecs.dequant_fp8_block(W.s1_q, W.s1_s).T
    u = xd @ codecs.dequant_fp8_block(W.s3_q, W.s3_s).T
    h = (np.minimum(g, 10) / (1 + np.exp(-np.minimum(g, 10))) * np.clip(u, -10, 10)).astype(np.float32)
    want += quant.act_dequant(*quant.act_quant(h, pow2=True)) @ codecs.dequant_fp8_block(W.s2_q, W.s2_s).T
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 2e-4
