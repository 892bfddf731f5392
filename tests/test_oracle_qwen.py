"""Pins oracle.qwen_moe.

Restates the reference's own MoE tests (tests/test_ref_qwen4_exp.py:88-136)
against this oracle, checks the expert-grouped form against the literal
per-token loop, and pins the quantized layer against (a) an independent
dequantize-then-matmul restatement with the same quantization points and
(b) the un-quantized layer within the e4m3 error budget.
"""
import numpy as np

from oracle import codecs, quant
from oracle import qwen_moe as qm


def _softmax64(x):
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def test_route_renormalizes_and_orders():
    rng = np.random.default_rng(3)
    logits = rng.normal(size=(5, 8)).astype(np.float32)
    w, ids = qm.moe_route(logits, 3)
    p = _softmax64(logits.astype(np.float64))
    for r in range(5):
        assert ids[r, 0] == np.argmax(p[r])
        order = np.argsort(-p[r], kind="stable")[:3]
        np.testing.assert_array_equal(ids[r], order)
        wr = p[r, order] / (p[r, order].sum() + 1e-20)
        np.testing.assert_allclose(w[r], wr, rtol=1e-5, atol=1e-7)
        np.testing.assert_allclose(w[r].sum(), 1.0, rtol=1e-6)


def test_route_ties_take_lowest_ids():
    w, ids = qm.moe_route(np.zeros((1, 6), np.float32), 3)
    np.testing.assert_array_equal(ids[0], [0, 1, 2])
    np.testing.assert_allclose(w[0], [1 / 3] * 3, rtol=1e-6)


def _tiny(rng, n=4, h=6, e=5, i=3, ts=3):
    x = rng.normal(size=(n, h)).astype(np.float32)
    router = rng.normal(size=(e, h)).astype(np.float32)
    eg = rng.normal(size=(e, i, h)).astype(np.float32) * 0.3
    eu = rng.normal(size=(e, i, h)).astype(np.float32) * 0.3
    ed = rng.normal(size=(e, h, i)).astype(np.float32) * 0.3
    sg = rng.normal(size=(ts, h)).astype(np.float32) * 0.3
    su = rng.normal(size=(ts, h)).astype(np.float32) * 0.3
    sd = rng.normal(size=(h, ts)).astype(np.float32) * 0.3
    sgl = rng.normal(size=(1, h)).astype(np.float32)
    return x, router, eg, eu, ed, sg, su, sd, sgl


def test_block_matches_manual_fp64_loop():
    x, router, eg, eu, ed, sg, su, sd, sgl = _tiny(np.random.default_rng(4))
    got = qm.moe_block_forward(x, router, eg, eu, ed, sg, sgl, su, sd, top_k=2)
    p = _softmax64(x @ router.T)
    want = np.zeros(x.shape)
    for r in range(x.shape[0]):
        ids = np.argsort(-p[r], kind="stable")[:2]
        wr = p[r, ids] / (p[r, ids].sum() + 1e-20)
        for eid, wgt in zip(ids, wr):
            g = x[r] @ eg[eid].T
            want[r] += wgt * (((g / (1 + np.exp(-g))) * (x[r] @ eu[eid].T)) @ ed[eid].T)
        gs = x[r] @ sg.T
        sh = ((gs / (1 + np.exp(-gs))) * (x[r] @ su.T)) @ sd.T
        want[r] += sh / (1 + np.exp(-(x[r] @ sgl.T)))
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def test_grouped_equals_literal_loop():
    x, router, eg, eu, ed, sg, su, sd, sgl = _tiny(np.random.default_rng(5), n=9)
    lit = qm.moe_block_forward(x, router, eg, eu, ed, sg, sgl, su, sd, top_k=3)
    grp = qm.moe_block_grouped(x, x @ router.T, eg, eu, ed, 3, (sg, su, sd, sgl))
    np.testing.assert_allclose(grp, lit, rtol=1e-5, atol=1e-6)


def make_small_fp8_layer(rng, T=32, H=256, E=8, I=256, Is=128, shared=True):
    bf = codecs.round_bf16
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.02).astype(np.float32))

    def qw(n, k):
        return quant.quantize_weight_fp8_block((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    g = [qw(I, H) for _ in range(E)]
    u = [qw(I, H) for _ in range(E)]
    d = [qw(H, I) for _ in range(E)]
    W = qm.QwenFp8Weights(
        router_w=rw,
        wg_q=np.stack([a for a, _ in g]), wg_s=np.stack([b for _, b in g]),
        wu_q=np.stack([a for a, _ in u]), wu_s=np.stack([b for _, b in u]),
        wd_q=np.stack([a for a, _ in d]), wd_s=np.stack([b for _, b in d]))
    if shared:
        (W.sg_q, W.sg_s), (W.su_q, W.su_s), (W.sd_q, W.sd_s) = qw(Is, H), qw(Is, H), qw(H, Is)
        W.sgl = bf((rng.standard_normal((1, H)) * 0.02).astype(np.float32))
    return x, W


def test_quantized_layer_matches_dequant_restatement():
    rng = np.random.default_rng(6)
    x, W = make_small_fp8_layer(rng)
    logits = x @ W.router_w.T
    got = qm.moe_layer_fp8(x, logits, W, top_k=2)
    # independent restatement: dequantize activations and weights, matmul
    w, ids = qm.moe_route(logits, 2)
    xd = quant.act_dequant(*quant.act_quant(x))
    want = np.zeros_like(x)

    def expert(xrows, gq, gs, uq, us, dq, ds):
        g = xrows @ codecs.dequant_fp8_block(gq, gs).T
        u = xrows @ codecs.dequant_fp8_block(uq, us).T
        h = (g / (1 + np.exp(-g)) * u).astype(np.float32)
        hd = quant.act_dequant(*quant.act_quant(h))
        return hd @ codecs.dequant_fp8_block(dq, ds).T
    for t in range(x.shape[0]):
        for j in range(2):
            e = ids[t, j]
            want[t] += w[t, j] * expert(xd[t:t + 1], W.wg_q[e], W.wg_s[e], W.wu_q[e],
                                        W.wu_s[e], W.wd_q[e], W.wd_s[e])[0]
    gate = 1 / (1 + np.exp(-(x @ W.sgl.T)))
    want += gate * expert(xd, W.sg_q, W.sg_s, W.su_q, W.su_s, W.sd_q, W.sd_s)
    d = got - want
    assert np.linalg.norm(d) / np.linalg.norm(want) < 2e-4


def test_quantized_layer_near_unquantized():
    rng = np.random.default_rng(7)
    x, W = make_small_fp8_layer(rng)
    logits = x @ W.router_w.T
    q = qm.moe_layer_fp8(x, logits, W, top_k=2)
    f = qm.moe_layer_fp8_dequant(x, logits, W, top_k=2)
    rel = np.linalg.norm(q - f) / np.linalg.norm(f)
    # two e4m3 activation roundings of ~2^-4 relative spacing each
    assert 1e-3 < rel < 6e-2
