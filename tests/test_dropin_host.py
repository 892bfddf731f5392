"""CPU checks of the drop-in moe_block_forward's host logic (no GPU).

- The zero padding QwenMoE applies to shapes off the kernels' granularity
  (hidden % 256, intermediates % 128; the reference's tiny dev model has
  hidden 16 and intermediates 8, serving/dev_model.py:244-257) changes no
  output: the oracle's literal per-token loop (ref/qwen4_exp.py:153-184) on
  the padded arrays equals it on the originals, and so does the FP8
  dequantized layer with the block scales padded by 1.0.
- The device-layer cache: one layer per weight set, reused while the same
  router object and matching weights come back (the pipeline's _moe_w
  stacks the experts anew on every call), dropped when the router object is
  freed, and bounded in size. QwenMoE is replaced by a recording stub.
"""
import gc

import numpy as np
import pytest

from oracle import codecs, quant
from oracle import qwen_moe as qm
from sllm_amd import moe

bf = codecs.round_bf16


def _pad_dims(H, I, Is):
    return (moe._round_up(H, moe.H_ALIGN), moe._round_up(I, moe.I_ALIGN),
            moe._round_up(Is, moe.I_ALIGN))


@pytest.mark.parametrize("T,H,E,I,k", [(5, 16, 4, 8, 2), (9, 20, 6, 12, 3),
                                       (3, 300, 3, 130, 1)])
def test_padding_leaves_the_layer_unchanged(T, H, E, I, k):
    rng = np.random.default_rng(T * H)
    Is = I
    Hp, Ip, Isp = _pad_dims(H, I, Is)
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf(rng.standard_normal((E, H)).astype(np.float32) * 0.5)
    eg, eu = (bf(rng.standard_normal((E, I, H)).astype(np.float32) * 0.3) for _ in range(2))
    ed = bf(rng.standard_normal((E, H, I)).astype(np.float32) * 0.3)
    sg, su = (bf(rng.standard_normal((Is, H)).astype(np.float32) * 0.3) for _ in range(2))
    sd = bf(rng.standard_normal((H, Is)).astype(np.float32) * 0.3)
    sgl = bf(rng.standard_normal((1, H)).astype(np.float32) * 0.3)
    want = qm.moe_block_forward(x, rw, eg, eu, ed, sg, sgl, su, sd, k)
    P = moe._pad_to
    got = qm.moe_block_forward(
        P(x, (T, Hp)), P(rw, (E, Hp)), P(eg, (E, Ip, Hp)), P(eu, (E, Ip, Hp)),
        P(ed, (E, Hp, Ip)), P(sg, (Isp, Hp)), P(sgl, (1, Hp)), P(su, (Isp, Hp)),
        P(sd, (Hp, Isp)), k)
    # equal up to the fp32 summation order BLAS picks for the longer rows
    assert np.all(got[:, H:] == 0)
    np.testing.assert_allclose(got[:, :H], want, rtol=1e-5,
                               atol=1e-6 * np.abs(want).max())

    # FP8 codes padded with code 0, scales with 1.0 (dequantized layer)
    def q8(n, kk):
        return quant.quantize_weight_fp8_block(
            rng.standard_normal((n, kk)).astype(np.float32) * 0.3)

    def stack(n, kk):
        qs = [q8(n, kk) for _ in range(E)]
        return np.stack([a for a, _ in qs]), np.stack([b for _, b in qs])

    def pq(q, s, n, kk):
        lead = q.shape[:-2]
        return (P(q, (*lead, n, kk)),
                P(s, (*lead, -(-n // 128), -(-kk // 128)), 1.0))
    (gq, gs), (uq, us), (dq, ds) = stack(I, H), stack(I, H), stack(H, I)
    (sgq, sgs), (suq, sus), (sdq, sds) = q8(Is, H), q8(Is, H), q8(H, Is)
    W = qm.QwenFp8Weights(router_w=rw, wg_q=gq, wg_s=gs, wu_q=uq, wu_s=us,
                          wd_q=dq, wd_s=ds, sg_q=sgq, sg_s=sgs, su_q=suq,
                          su_s=sus, sd_q=sdq, sd_s=sds, sgl=sgl)
    Wp = qm.QwenFp8Weights(P(rw, (E, Hp)), *pq(gq, gs, Ip, Hp),
                           *pq(uq, us, Ip, Hp), *pq(dq, ds, Hp, Ip),
                           sgl=P(sgl, (1, Hp)))
    Wp.sg_q, Wp.sg_s = pq(sgq, sgs, Isp, Hp)
    Wp.su_q, Wp.su_s = pq(suq, sus, Isp, Hp)
    Wp.sd_q, Wp.sd_s = pq(sdq, sds, Hp, Isp)
    lg = (x @ rw.T).astype(np.float32)
    want8 = qm.moe_layer_fp8_dequant(x, lg, W, k)
    got8 = qm.moe_layer_fp8_dequant(P(x, (T, Hp)), lg, Wp, k)
    assert np.all(got8[:, H:] == 0)
    np.testing.assert_allclose(got8[:, :H], want8, rtol=1e-5,
                               atol=1e-6 * np.abs(want8).max())


class _StubLayer:
    made = []

    def __init__(self, router_w, *a, **kw):
        # like QwenMoE, keeps no reference to the host arrays
        _StubLayer.made.append(self)

    def forward(self, x):
        return np.asarray(x, np.float32) * 0 + len(_StubLayer.made)


@pytest.fixture
def stub(monkeypatch):
    _StubLayer.made = []
    monkeypatch.setattr(moe, "QwenMoE", _StubLayer)
    moe.clear_block_cache()
    yield _StubLayer
    moe.clear_block_cache()


def _weights(seed, E=4, H=16, I=8):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    return f(E, H), f(E, I, H), f(E, I, H), f(E, H, I)


def test_block_cache_reuses_the_layer_for_the_same_weights(stub):
    rw, eg, eu, ed = _weights(0)
    x = np.ones((2, 16), np.float32)
    moe.moe_block_forward(x, rw, eg, eu, ed, None, None, None, None, 2)
    # the experts stacked anew (equal values, new arrays): a hit
    moe.moe_block_forward(x, rw, eg.copy(), eu.copy(), ed.copy(), None, None,
                          None, None, 2)
    assert len(stub.made) == 1 and len(moe._block_cache) == 1
    # other expert values, another top-k, another router object: misses
    moe.moe_block_forward(x, rw, eg + 1, eu, ed, None, None, None, None, 2)
    moe.moe_block_forward(x, rw, eg, eu, ed, None, None, None, None, 3)
    rw2 = rw.copy()
    moe.moe_block_forward(x, rw2, eg, eu, ed, None, None, None, None, 2)
    assert len(stub.made) == 4 and len(moe._block_cache) == 4


def test_block_cache_drops_a_freed_router_and_is_bounded(stub, monkeypatch):
    x = np.ones((1, 16), np.float32)
    rw, eg, eu, ed = _weights(1)
    moe.moe_block_forward(x, rw, eg, eu, ed, None, None, None, None, 2)
    assert len(moe._block_cache) == 1
    del rw
    gc.collect()
    assert len(moe._block_cache) == 0
    monkeypatch.setattr(moe, "BLOCK_CACHE_MAX", 3)
    keep = []
    for s in range(5):
        w = _weights(10 + s)
        keep.append(w)
        moe.moe_block_forward(x, *w, None, None, None, None, 2)
    assert len(moe._block_cache) == 3
    # the most recent three remain: the third call's weights hit
    n = len(stub.made)
    moe.moe_block_forward(x, *keep[2], None, None, None, None, 2)
    assert len(stub.made) == n
    moe.moe_block_forward(x, *keep[0], None, None, None, None, 2)
    assert len(stub.made) == n + 1
