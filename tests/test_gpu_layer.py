"""GPU parity of the fused MoE layers against the oracle.

Routing (ids, per-expert counts) must be bit-exact at the logits boundary:
the oracle routes the fp32 logits the device produced (the boundary the
reference's sllm_q4_moe_router exposes); the router GEMMs themselves are
bounded against fp64 x . W_r^T (the fused prefill router here, the others in
test_gpu_kernels.py, and at full size in test_gpu_fullsize.py). Layer
outputs must be
within the bf16-noise tolerance: relative L2 <= 1e-2 (asserted tighter where
the arithmetic allows) and a max-abs bound, both printed.
"""
import numpy as np
import pytest

from oracle import deepseek_moe as dm
from oracle import qwen_moe as qm

from tests._fixtures import (check_qwen_routing, check_router_logits, deepseek_layer,
                             deepseek_mxfp4, deepseek_mxfp4_gpu, qwen_checkpoint,
                             qwen_fp8, qwen_fp8_gpu, qwen_layer, rel_l2)

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    from sllm_amd import _lib
    if not _lib.available():
        pytest.fail(f"libsllm_moe.so not loadable: {_lib._lib_error}")


def _check_routing(r, W_router_E, k):
    tied = check_qwen_routing(r["logits"], r["ids"], r["w"], k)
    counts = np.bincount(r["ids"].ravel(), minlength=W_router_E)
    np.testing.assert_array_equal(r["counts"], counts)
    return len(tied)


def _report(name, got, want):
    rel = rel_l2(got, want)
    mabs = float(np.abs(got - want).max())
    scale = float(np.abs(want).max())
    print(f"{name}: rel-L2 {rel:.3e} max-abs {mabs:.3e} (max |ref| {scale:.3e})")
    return rel, mabs, scale


@pytest.mark.parametrize("packed", [True, False])
@pytest.mark.parametrize("T,E,k,shared", [(256, 8, 2, True), (130, 16, 4, False),
                                          (512, 64, 6, True)])
def test_qwen_prefill_small(T, E, k, shared, packed):
    x, W = qwen_fp8(seed=T, T=T, H=512, E=E, I=256, Is=256, shared=shared)
    layer = qwen_layer(W, k, packed=packed)
    y, r = layer.forward(x, mode="prefill", return_routing=True)
    _check_routing(r, E, k)
    want = qm.moe_layer_fp8(x, r["logits"], W, k)
    rel, mabs, scale = _report("qwen prefill", y, want)
    assert rel < 3e-3 and mabs < 0.05 * scale


def test_qwen_prefill_c2_shapes():
    """C2 geometry (H 2048, I = Is = 512, top-10) with E = 128 experts at
    T = 512 tokens (full E = 512 routing and permute are covered by
    test_gpu_kernels.py at T = 4096 / 16384)."""
    T, H, E, I, k = 512, 2048, 128, 512, 10
    x, W = qwen_fp8_gpu(seed=2, T=T, H=H, E=E, I=I, Is=I)
    layer = qwen_layer(W, k)
    y, r = layer.forward(x, mode="prefill", return_routing=True)
    _check_routing(r, E, k)
    want = qm.moe_layer_fp8(x, r["logits"], W, k)
    rel, mabs, scale = _report("qwen prefill C2 shapes", y, want)
    assert rel < 3e-3 and mabs < 0.05 * scale
    info = qm.moe_layer_fp8_dequant(x, r["logits"], W, k)
    print(f"  (information only) vs un-quantized-activation oracle: "
          f"rel-L2 {rel_l2(y, info):.3e}")


@pytest.mark.parametrize("T,E,k", [(200, 200, 8), (300, 512, 10),
                                   (130, 1024, 10), (257, 96, 16), (65, 128, 1),
                                   (100, 2048, 10), (80, 16, 16), (70, 129, 4)])
def test_qwen_fused_router_matches_full_row_routing(T, E, k):
    """Prefill router fused with routing: each 128-expert tile's top-k keys
    and softmax partials, merged by the routing launch, against the
    full-row routing kernel on the same logits (the layer given the logits
    the first call copied out). Ids bit-exact, weights to 2e-6 (only the
    normaliser's summation order differs), outputs within a few bf16 ulps;
    the default call (no logits copy) gives the same output bit for bit.
    Cases: a partial last tile (E 200, 96), 80 candidate keys (E 1024),
    top-16 from one tile, top-1, ragged 64-token tiles, 160 candidates
    (E 2048: the merge's wave-per-token form), every expert picked (E 16,
    top-16), a last tile of one expert (E 129). The fused router's logits
    (its copy for the caller) are bounded against fp64 x . W_r^T."""
    x, W = qwen_fp8_gpu(seed=T + E, T=T, H=512, E=E, I=128, Is=128)
    layer = qwen_layer(W, k)
    y_f, r_f = layer.forward(x, mode="prefill", return_routing=True)
    check_router_logits(f"fused router T={T} E={E}", x, W.router_w, r_f["logits"])
    assert _check_routing(r_f, E, k) == 0
    y_g, r_g = layer.forward(x, logits=r_f["logits"], mode="prefill",
                             return_routing=True)
    np.testing.assert_array_equal(r_f["ids"], r_g["ids"])
    np.testing.assert_array_equal(r_f["counts"], r_g["counts"])
    np.testing.assert_allclose(r_f["w"], r_g["w"], rtol=2e-6, atol=1e-9)
    rel = rel_l2(y_f, y_g)
    print(f"fused router T={T} E={E} k={k}: output vs full-row routing "
          f"rel-L2 {rel:.3e}")
    assert rel < 1e-4
    y_d = layer.forward(x, mode="prefill")
    np.testing.assert_array_equal(y_d, y_f)


@pytest.mark.parametrize("B", [1, 8, 32, 64])
def test_qwen_decode_c3_shapes(B):
    """C3 decode batches on C2 geometry (fp32-activation GEMV path)."""
    H, E, I, k = 2048, 512, 512, 10
    x, W = qwen_fp8_gpu(seed=100 + B, T=B, H=H, E=E, I=I, Is=I)
    layer = qwen_layer(W, k)
    y, r = layer.forward(x, mode="decode", return_routing=True)
    _check_routing(r, E, k)
    want = qm.moe_layer_fp8_dequant(x, r["logits"], W, k)
    rel, mabs, scale = _report(f"qwen decode B={B}", y, want)
    assert rel < 1e-4


@pytest.mark.parametrize("B,E,k", [(17, 2, 2), (40, 4, 2), (64, 4, 2)])
def test_qwen_decode_32_row_tiles(B, E, k):
    """Decode with experts averaging more than 16 rows: 32-row tiles for the
    routed and shared segments (ragged last tiles, experts of 17-32 and of
    more than 32 rows)."""
    H, I = 1024, 256
    x, W = qwen_fp8(seed=120 + B, T=B, H=H, E=E, I=I, Is=I)
    layer = qwen_layer(W, k)
    y, r = layer.forward(x, mode="decode", return_routing=True)
    _check_routing(r, E, k)
    want = qm.moe_layer_fp8_dequant(x, r["logits"], W, k)
    rel, mabs, scale = _report(f"qwen decode 32-row B={B} E={E}", y, want)
    assert rel < 1e-4


@pytest.mark.parametrize("B,E,k,biased", [(1, 512, 10, False), (3, 64, 6, True),
                                          (4, 512, 10, True), (6, 512, 10, False),
                                          (8, 8, 4, True), (8, 512, 10, False),
                                          (16, 64, 6, False), (17, 64, 6, True),
                                          (32, 512, 10, True), (40, 4, 2, False),
                                          (64, 512, 10, False)])
def test_decode_inline_routing_matches_launches(B, E, k, biased, monkeypatch):
    """Streamed decode builds the expert-major permutation inside the
    gate/up launch (every workgroup in LDS, workgroup 0 writing the tables
    for the later launches): up to 8 tokens after routing them there too
    (one token per wave, the router split in K), above 16 tokens from the
    routing launch's ids; 9-16 tokens keep the one-workgroup route +
    permute launch (B=16 here). Against the same logits routed and
    permuted in launches of their own, the output, route weights, ids,
    counts, sorted rows and inverse positions agree bit for bit, on
    repeated calls: above 8 tokens with SLLM_MOE_ROUTE_INLINE=0; up to 8
    with a call that also copies the logits (a split router's slices then
    go to the one-workgroup route + permute launch). Covered: with and
    without a router bias, the fused gate/up finish (B <= 4), the split
    router's logit slices and shared-gate partials, and 32-row tiles
    (E = 4). Up to 64 assignments the launch sorts them in one wave (B=6:
    60 assignments; E = 8 at B=8: several rows per expert). The output
    also matches the oracle layer on the logits."""
    from sllm_amd.moe import QwenMoE, _up, qwen_forward_dev
    from sllm_amd.runtime import DeviceBuffer, to_bf16
    H, I = 512, 256
    make = qwen_fp8_gpu if E >= 256 else qwen_fp8
    x, W = make(seed=700 + B + E, T=B, H=H, E=E, I=I, Is=I)
    rng = np.random.default_rng(B + E)
    bias = (-rng.random(E) * 2.0).astype(np.float32) if biased else None
    layer = QwenMoE(W.router_w, W.wg_q, W.wu_q, W.wd_q, W.wg_s, W.wu_s, W.wd_s,
                    sg=W.sg_q, su=W.su_q, sd=W.sd_q, sg_s=W.sg_s, su_s=W.su_s,
                    sd_s=W.sd_s, sgl=W.sgl, top_k=k, router_bias=bias)
    N = B * k
    shapes = {"w_out": (np.float32, (B, k)), "ids_out": (np.int32, (B, k)),
              "counts_out": (np.int32, (E,)), "sorted_out": (np.int32, (N,)),
              "inv_pos_out": (np.int32, (N,))}

    def run(with_logits=False):
        dbg = {n: DeviceBuffer(int(np.prod(s)) * 4) for n, (_, s) in shapes.items()}
        if with_logits:
            dbg["logits_out"] = DeviceBuffer(B * E * 4)
        out = DeviceBuffer(B * H * 4)
        qwen_forward_dev(_up(to_bf16(x)), out, layer._w, T=B, H=H, E=E, I=I,
                         Is=I, topk=k, mode="decode", out_f32=True,
                         eps=layer.eps, workspace=layer._workspace(B, "decode", False),
                         debug=dbg)
        res = {"y": out.copy_host().reshape(B, H)}
        for n, (dt, s) in shapes.items():
            res[n] = dbg[n].copy_host_raw(dt, s)
        if with_logits:
            res["logits"] = dbg["logits_out"].copy_host().reshape(B, E)
        return res

    def same(a, b, what):
        for n in a:
            if n in b:
                np.testing.assert_array_equal(a[n].view(np.uint32), b[n].view(np.uint32),
                                              err_msg=f"{what}: {n}")

    monkeypatch.setenv("SLLM_MOE_ROUTE_INLINE", "1")
    inl = run()
    same(inl, run(), "inline, second call")
    if B <= 8:
        ref = run(with_logits=True)
    else:
        monkeypatch.setenv("SLLM_MOE_ROUTE_INLINE", "0")
        ref = run(with_logits=True)
    same(inl, ref, "inline vs launches")
    lg = ref["logits"] + (bias[None, :] if biased else 0.0)
    assert check_qwen_routing(lg.astype(np.float32), inl["ids_out"], inl["w_out"], k,
                              name=f"inline B={B}").size == 0
    want = qm.moe_layer_fp8_dequant(x, lg.astype(np.float32), W, k)
    rel, _, _ = _report(f"inline routing B={B} E={E}", inl["y"], want)
    assert rel < 1e-4


def test_qwen_logits_given_and_auto_mode():
    x, W = qwen_fp8(seed=5, T=96, H=512, E=8, I=256, Is=256)
    layer = qwen_layer(W, 3)
    logits = (x @ W.router_w.T).astype(np.float32)
    y, r = layer.forward(x, logits=logits, mode="auto", return_routing=True)
    np.testing.assert_array_equal(r["logits"], logits)
    want = qm.moe_layer_fp8(x, logits, W, 3)      # T=96 > 64: prefill
    assert rel_l2(y, want) < 3e-3
    yd = layer.forward(x[:10], logits=logits[:10], mode="auto")  # decode
    assert rel_l2(yd, qm.moe_layer_fp8_dequant(x[:10], logits[:10], W, 3)) < 1e-4


def test_c1_bf16_literal_oracle():
    """C1: 64 tokens, H 1024, E 16, top-4, I 512, no shared expert, bf16
    weights, seed 0 -- against the reference's literal per-token loop."""
    from oracle.codecs import round_bf16 as bf
    from sllm_amd.moe import moe_block_forward
    rng = np.random.default_rng(0)
    T, H, E, k, I = 64, 1024, 16, 4, 512
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    eg = bf((rng.standard_normal((E, I, H)) * 0.02).astype(np.float32))
    eu = bf((rng.standard_normal((E, I, H)) * 0.02).astype(np.float32))
    ed = bf((rng.standard_normal((E, H, I)) * 0.02).astype(np.float32))
    got = moe_block_forward(x, rw, eg, eu, ed, None, None, None, None, k)
    want = qm.moe_block_forward(x, rw, eg, eu, ed, None, None, None, None, k)
    rel, mabs, scale = _report("C1 bf16", got, want)
    assert rel < 1e-4


@pytest.mark.parametrize("T,E,k,S,inter", [(5, 4, 2, 8, 8), (64, 4, 2, 8, 8),
                                           (3, 6, 3, 20, 12)])
def test_dev_model_shapes_through_drop_in(T, E, k, S, inter):
    """The reference's tiny dev model (serving/dev_model.py:244-257: hidden
    16, 4 experts, top-2, moe_inter = shared_inter = 8) through the drop-in
    moe_block_forward (ref/qwen4_exp_pipeline.py:278-284 calls it with these
    shapes), against the reference's literal per-token loop; hidden 20 /
    intermediate 12 as a ragged case. The layer pads the shapes to the
    kernels' granularity with zeros, which adds nothing. A second call with
    the same weights reuses the device layer (no upload) and gives the same
    bits; another router weight object gets a layer of its own."""
    from oracle.codecs import round_bf16 as bf
    from sllm_amd import moe
    rng = np.random.default_rng(T + S)
    H, I, Is = (16 if S == 8 else 20), inter, inter
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.5).astype(np.float32))
    eg = bf((rng.standard_normal((E, I, H)) * 0.3).astype(np.float32))
    eu = bf((rng.standard_normal((E, I, H)) * 0.3).astype(np.float32))
    ed = bf((rng.standard_normal((E, H, I)) * 0.3).astype(np.float32))
    sg = bf((rng.standard_normal((Is, H)) * 0.3).astype(np.float32))
    su = bf((rng.standard_normal((Is, H)) * 0.3).astype(np.float32))
    sd = bf((rng.standard_normal((H, Is)) * 0.3).astype(np.float32))
    sgl = bf((rng.standard_normal((1, H)) * 0.3).astype(np.float32))
    moe.clear_block_cache()
    got = moe.moe_block_forward(x, rw, eg, eu, ed, sg, sgl, su, sd, k)
    assert got.shape == (T, H) and got.dtype == np.float32
    want = qm.moe_block_forward(x, rw, eg, eu, ed, sg, sgl, su, sd, k)
    rel, mabs, scale = _report(f"dev-model shapes T={T} H={H} I={I}", got, want)
    assert rel < 1e-4
    assert len(moe._block_cache) == 1
    layer = next(iter(moe._block_cache.values()))[1]
    # the pipeline's _moe_w stacks the experts anew on each call
    again = moe.moe_block_forward(x, rw, eg.copy(), eu.copy(), ed.copy(), sg, sgl,
                                  su, sd, k)
    np.testing.assert_array_equal(again, got)
    assert len(moe._block_cache) == 1
    assert next(iter(moe._block_cache.values()))[1] is layer
    rw2 = rw.copy()
    moe.moe_block_forward(x, rw2, eg, eu, ed, sg, sgl, su, sd, k)
    assert len(moe._block_cache) == 2
    moe.clear_block_cache()


@pytest.mark.parametrize("T,mode", [(300, "prefill"), (300, "prefill-logits"),
                                    (40, "decode"), (8, "decode")])
def test_qwen_router_bias_every_routing_path(T, mode):
    """The per-expert routing bias (router_bias; the skewed-load
    configuration's) on each routing path: the fused prefill router (bias
    before the tiles' top-k and softmax partials), the full-row softmax
    routing with the logits given, the multi-workgroup decode routing (40
    tokens, split router slices) and the one-workgroup route + permute
    (8 tokens). Ids bit-exact against the oracle's moe_route of logits +
    bias (one fp32 addition), weights rtol 1e-5, the layer output against
    the oracle layer on those routes; logits_out holds the logits without
    the bias (bounded against fp64 x . W_r^T)."""
    from sllm_amd.moe import QwenMoE
    E, k, H, I = 64, 6, 512, 256
    x, W = qwen_fp8(seed=31 + T, T=T, H=H, E=E, I=I, Is=256)
    rng = np.random.default_rng(31)
    ranks = rng.permutation(E) + 1
    bias = (-2.0 * np.log(ranks)).astype(np.float32)
    bias[ranks > 50] = -40.0
    layer = QwenMoE(W.router_w, W.wg_q, W.wu_q, W.wd_q, W.wg_s, W.wu_s, W.wd_s,
                    sg=W.sg_q, su=W.su_q, sd=W.sd_q, sg_s=W.sg_s, su_s=W.su_s,
                    sd_s=W.sd_s, sgl=W.sgl, top_k=k, router_bias=bias)
    given = mode == "prefill-logits"
    lg_in = (x @ W.router_w.T).astype(np.float32) if given else None
    m = "prefill" if mode.startswith("prefill") else "decode"
    y, r = layer.forward(x, logits=lg_in, mode=m, return_routing=True)
    if given:
        np.testing.assert_array_equal(r["logits"], lg_in)
    else:
        check_router_logits(f"biased router {mode}", x, W.router_w, r["logits"])
    lg = (r["logits"] + bias[None, :]).astype(np.float32)
    assert check_qwen_routing(lg, r["ids"], r["w"], k, name=f"bias {mode}").size == 0
    np.testing.assert_array_equal(r["counts"], np.bincount(r["ids"].ravel(), minlength=E))
    assert r["counts"][ranks > 50].sum() == 0
    if m == "prefill":
        want = qm.moe_layer_fp8(x, lg, W, k)
        rel, mabs, scale = _report(f"bias {mode}", y, want)
        assert rel < 3e-3 and mabs < 0.05 * scale
    else:
        want = qm.moe_layer_fp8_dequant(x, lg, W, k)
        rel, mabs, scale = _report(f"bias {mode}", y, want)
        assert rel < 1e-4


def test_qwen_skewed_with_empty_experts():
    """C5-style skew: biased logits concentrate load, many experts empty."""
    T, H, E, I, k = 2048, 512, 64, 256, 6
    x, W = qwen_fp8(seed=9, T=T, H=H, E=E, I=I, Is=256)
    rng = np.random.default_rng(9)
    ranks = rng.permutation(E) + 1
    bias = (-3.0 * np.log(ranks)).astype(np.float32)
    bias[ranks > 40] = -60.0          # these experts never win
    logits = (x @ W.router_w.T + bias).astype(np.float32)
    layer = qwen_layer(W, k)
    y, r = layer.forward(x, logits=logits, mode="prefill", return_routing=True)
    assert (r["counts"] == 0).sum() >= 20 and r["counts"].max() > 128
    _check_routing(r, E, k)
    want = qm.moe_layer_fp8(x, logits, W, k)
    rel, mabs, scale = _report("qwen skewed", y, want)
    assert rel < 3e-3


@pytest.mark.parametrize("T,E,k,shared", [(1024, 8, 2, True), (777, 16, 4, True),
                                          (2048, 64, 6, False)])
def test_qwen_dense8_kernel_matches_stream(T, E, k, shared, monkeypatch):
    """With SLLM_MOE_DENSE8=2, prefill whose experts average more than one
    128-row tile (T k > 128 E) runs its FP8 projections (fp32 block scales)
    on the compute-dense kernel (gemm_dense8.hip), the shared expert's too
    when T > 128; SLLM_MOE_DENSE8=0 runs the same items on the streaming
    kernel. The same MFMA per K step, the same rescale order and
    epilogues: the outputs agree bit for bit, on every call, and match the
    oracle. T=777 leaves partial tiles."""
    x, W = qwen_fp8(seed=T + E, T=T, H=512, E=E, I=256, Is=256, shared=shared)
    layer = qwen_layer(W, k)
    monkeypatch.setenv("SLLM_MOE_DENSE8", "2")
    y_dense, r = layer.forward(x, mode="prefill", return_routing=True)
    for _ in range(3):  # the same bits on every call
        np.testing.assert_array_equal(layer.forward(x, mode="prefill"), y_dense)
    monkeypatch.setenv("SLLM_MOE_DENSE8", "0")
    y_stream = layer.forward(x, mode="prefill")
    np.testing.assert_array_equal(y_dense, y_stream)
    want = qm.moe_layer_fp8(x, r["logits"], W, k)
    rel, mabs, scale = _report("qwen dense8 prefill", y_dense, want)
    assert rel < 3e-3 and mabs < 0.05 * scale


@pytest.mark.parametrize("packed", [True, False])
@pytest.mark.parametrize("T,G,kg,L", [(200, 4, 2, 10.0), (256, 1, 1, 0.0)])
def test_deepseek_prefill_small(T, G, kg, L, packed):
    x, W = deepseek_mxfp4(seed=T, T=T, H=512, E=16, I=256, Is=256)
    route = dict(n_group=G, topk_group=kg, scoring="sigmoid", route_scale=2.5,
                 swiglu_limit=L)
    layer = deepseek_layer(W, 4, packed=packed, **route)
    y, r = layer.forward(x, mode="prefill", return_routing=True)
    w_ref, ids_ref = dm.moe_route(r["logits"], W.bias, 4, "sigmoid", 2.5, G, kg)
    np.testing.assert_array_equal(r["ids"], ids_ref.astype(np.int32))
    np.testing.assert_allclose(r["w"], w_ref, rtol=2e-6)
    want = dm.moe_layer_mxfp4(x, r["logits"], W, 4, L, "sigmoid", 2.5, G, kg)
    rel, mabs, scale = _report("deepseek prefill", y, want)
    assert rel < 3e-3 and mabs < 0.05 * scale


@pytest.mark.parametrize("T,E,H", [(200, 16, 512), (777, 200, 768), (96, 256, 1024)])
def test_deepseek_router_quant_matches_separate_launches(T, E, H):
    """Prefill from router_w: the router launch also quantizes the
    activations (power-of-two scales) from the x chunks it stages. Given
    the logits that call copied out, the layer runs the separate
    activation-quant launch instead. The router launch's logits are the
    logits GEMM's (same MFMA order), so the two calls route alike and, with
    the same quantized activations, give the same output bit for bit.
    E 200: a partial expert tile; T 777: a partial token tile; H 1024.
    The first case is also checked against the oracle."""
    small = E <= 16
    x, W = (deepseek_mxfp4(seed=T + E, T=T, H=H, E=E, I=256, Is=256) if small
            else deepseek_mxfp4_gpu(seed=T + E, T=T, H=H, E=E, I=256, Is=256))
    route = dict(n_group=1, topk_group=1, scoring="sigmoid", route_scale=2.5,
                 swiglu_limit=10.0)
    layer = deepseek_layer(W, 6, **route)
    y_f, r_f = layer.forward(x, mode="prefill", return_routing=True)
    y_g, r_g = layer.forward(x, logits=r_f["logits"], mode="prefill",
                             return_routing=True)
    np.testing.assert_array_equal(r_f["ids"], r_g["ids"])
    np.testing.assert_array_equal(y_f, y_g)
    if small:
        want = dm.moe_layer_mxfp4(x, r_f["logits"], W, 6, 10.0, "sigmoid", 2.5, 1, 1)
        rel, mabs, scale = _report(f"deepseek router+quant T={T} E={E}", y_f, want)
        assert rel < 3e-3 and mabs < 0.05 * scale


@pytest.mark.parametrize("T,L", [(1024, 10.0), (777, 0.0)])
def test_deepseek_dense_kernel_matches_stream(T, L, monkeypatch):
    """Prefill whose experts average more than one 128-row tile runs the
    routed MXFP4 projections on the compute-dense kernel (gemm_dense.hip);
    SLLM_MOE_DENSE=0 runs the same items on the streaming kernel. Same
    MFMAs over the K steps in the same order and the same epilogues: the
    outputs agree bit for bit, and match the oracle. T=777 leaves tiles of
    4 rows (skipped 16-row groups)."""
    x, W = deepseek_mxfp4(seed=T, T=T, H=512, E=16, I=256, Is=256)
    route = dict(n_group=4, topk_group=2, scoring="sigmoid", route_scale=2.5,
                 swiglu_limit=L)
    layer = deepseek_layer(W, 8, **route)
    y_dense, r = layer.forward(x, mode="prefill", return_routing=True)
    for _ in range(3):  # the same bits on every call
        np.testing.assert_array_equal(layer.forward(x, mode="prefill"), y_dense)
    monkeypatch.setenv("SLLM_MOE_DENSE", "0")
    y_stream = layer.forward(x, mode="prefill")
    np.testing.assert_array_equal(y_dense, y_stream)
    want = dm.moe_layer_mxfp4(x, r["logits"], W, 8, L, "sigmoid", 2.5, 4, 2)
    rel, mabs, scale = _report("deepseek dense prefill", y_dense, want)
    assert rel < 3e-3 and mabs < 0.05 * scale


@pytest.mark.parametrize("T,force", [(1024, False), (300, False), (1024, True)])
def test_deepseek_shared_dense8_matches_stream(T, force, monkeypatch):
    """The DeepSeek shared expert (FP8 with power-of-two scales) runs its
    gate/up on the compute-dense FP8 kernel once its T rows fill more than
    one tile (its down projection too with SLLM_MOE_DENSE8=2), the scales
    applied as e8m0 MFMA scales as in the streaming kernel: the same bits as
    SLLM_MOE_DENSE8=0, and the oracle's result."""
    x, W = deepseek_mxfp4(seed=T + 3, T=T, H=512, E=16, I=256, Is=256)
    route = dict(n_group=4, topk_group=2, scoring="sigmoid", route_scale=2.5,
                 swiglu_limit=10.0)
    layer = deepseek_layer(W, 8, **route)
    if force:
        monkeypatch.setenv("SLLM_MOE_DENSE8", "2")
    y_dense, r = layer.forward(x, mode="prefill", return_routing=True)
    for _ in range(2):
        np.testing.assert_array_equal(layer.forward(x, mode="prefill"), y_dense)
    monkeypatch.setenv("SLLM_MOE_DENSE8", "0")
    y_stream = layer.forward(x, mode="prefill")
    np.testing.assert_array_equal(y_dense, y_stream)
    want = dm.moe_layer_mxfp4(x, r["logits"], W, 8, 10.0, "sigmoid", 2.5, 4, 2)
    rel, mabs, scale = _report("deepseek shared dense8", y_dense, want)
    assert rel < 3e-3 and mabs < 0.05 * scale


@pytest.mark.parametrize("T,mode", [(200, "prefill"), (8, "decode")])
def test_deepseek_hash_layer(T, mode):
    """A hash layer (first n_hash_layers of DeepSeek-V4): experts from the
    token-id table, weights from the sigmoid scores."""
    x, W = deepseek_mxfp4(seed=T + 7, T=T, H=512, E=16, I=256, Is=256)
    rng = np.random.default_rng(T)
    V, k = 40, 4
    tid2eid = np.stack([rng.permutation(16)[:k] for _ in range(V)]).astype(np.int32)
    tok = rng.integers(0, V, T).astype(np.int32)
    layer = deepseek_layer(W, k, scoring="sigmoid", route_scale=2.5,
                           tid2eid=tid2eid)
    y, r = layer.forward(x, mode=mode, return_routing=True, token_ids=tok)
    w_ref, ids_ref = dm.moe_route(r["logits"], W.bias, k, "sigmoid", 2.5,
                                  token_ids=tok, tid2eid=tid2eid)
    np.testing.assert_array_equal(r["ids"], ids_ref.astype(np.int32))
    np.testing.assert_allclose(r["w"], w_ref, rtol=2e-6)
    if mode == "prefill":
        want = dm.moe_layer_mxfp4(x, r["logits"], W, k, 0.0, "sigmoid", 2.5,
                                  token_ids=tok, tid2eid=tid2eid)
        rel, mabs, scale = _report("deepseek hash prefill", y, want)
        assert rel < 3e-3 and mabs < 0.05 * scale
    else:  # decode keeps activations unquantized: dequantized-weight oracle
        from oracle.codecs import dequant_fp4_block, dequant_fp8_block

        def ex(e):
            return (dequant_fp4_block(W.w1_p[e], W.w1_s[e]),
                    dequant_fp4_block(W.w3_p[e], W.w3_s[e]),
                    dequant_fp4_block(W.w2_p[e], W.w2_s[e]))
        sh = (dequant_fp8_block(W.s1_q, W.s1_s), dequant_fp8_block(W.s3_q, W.s3_s),
              dequant_fp8_block(W.s2_q, W.s2_s))
        want = dm.moe_block_forward(x, r["logits"], W.bias, ex, sh, k, 0.0,
                                    "sigmoid", 2.5, token_ids=tok, tid2eid=tid2eid)
        rel, mabs, scale = _report("deepseek hash decode", y, want)
        assert rel < 1e-4


@pytest.mark.parametrize("scale_tag", ["BF16", "F32"])
def test_load_qwen_checkpoint(tmp_path, scale_tag):
    """A layer loaded from checkpoint bytes (no host dequantization) equals
    the layer built from the same arrays, bit for bit."""
    from oracle.codecs import decode_bf16, encode_bf16_rne
    from sllm_amd import loader
    x, W = qwen_fp8(seed=21, T=96, H=512, E=8, I=256, Is=256)
    if scale_tag == "BF16":  # the stored scales are the bf16-rounded ones
        for a in ("wg_s", "wu_s", "wd_s", "sg_s", "su_s", "sd_s"):
            setattr(W, a, decode_bf16(encode_bf16_rne(getattr(W, a))))
    prefix = "model.language_model.layers.0.mlp"
    p = str(tmp_path / "qwen.safetensors")
    qwen_checkpoint(p, W, prefix, scale_tag)
    got = loader.load_qwen_moe(loader.Checkpoint(p), prefix, top_k=4)
    want = qwen_layer(W, 4)
    for mode in ("prefill", "decode"):
        np.testing.assert_array_equal(got.forward(x, mode=mode),
                                      want.forward(x, mode=mode))


@pytest.mark.parametrize("hash_layer", [False, True])
def test_load_deepseek_checkpoint(tmp_path, hash_layer):
    """DeepSeek layer from converted-checkpoint bytes: packed E2M1 experts
    with F8_E8M0 scales, F8_E4M3 shared expert with E8M0 128x128 scales."""
    from oracle.codecs import encode_bf16_rne
    from sllm_amd import loader
    x, W = deepseek_mxfp4(seed=22, T=96, H=512, E=16, I=256, Is=256)
    k, pre = 4, "layers.0."
    rng = np.random.default_rng(22)
    tid2eid = np.stack([rng.permutation(16)[:k] for _ in range(30)]).astype(np.int32)
    tok = rng.integers(0, 30, x.shape[0]).astype(np.int32)

    def e8(sv):  # fp32 powers of two -> e8m0 codes
        return ((np.asarray(sv, np.float32).view(np.uint32) >> 23) & 0xFF).astype(np.uint8)
    t = {f"{pre}ffn.gate.weight": ("BF16", W.router_w.shape, encode_bf16_rne(W.router_w)),
         f"{pre}ffn.gate.bias": ("F32", W.bias.shape, W.bias),
         "tid2eid": ("I32", tid2eid.shape, tid2eid)}
    for e in range(16):
        for w, q, sv in (("w1", W.w1_p, W.w1_s), ("w3", W.w3_p, W.w3_s),
                         ("w2", W.w2_p, W.w2_s)):
            t[f"{pre}ffn.experts.{e}.{w}.weight"] = ("U8", q[e].shape, q[e])
            t[f"{pre}ffn.experts.{e}.{w}.scale"] = ("F8_E8M0", sv[e].shape, sv[e])
    for w, q, sv in (("w1", W.s1_q, W.s1_s), ("w3", W.s3_q, W.s3_s),
                     ("w2", W.s2_q, W.s2_s)):
        t[f"{pre}ffn.shared_experts.{w}.weight"] = ("F8_E4M3", q.shape, q)
        t[f"{pre}ffn.shared_experts.{w}.scale"] = ("F8_E8M0", sv.shape, e8(sv))
    p = str(tmp_path / "ds.safetensors")
    loader.write_safetensors(p, t)
    route = dict(scoring="sigmoid", route_scale=2.5, swiglu_limit=10.0)
    got = loader.load_deepseek_moe(loader.Checkpoint(p), pre, k,
                                   hash_layer=hash_layer, **route)
    want = deepseek_layer(W, k, tid2eid=tid2eid if hash_layer else None, **route)
    kw = {"token_ids": tok} if hash_layer else {}
    for mode in ("prefill", "decode"):
        np.testing.assert_array_equal(got.forward(x, mode=mode, **kw),
                                      want.forward(x, mode=mode, **kw))


def test_deepseek_prefill_c4_shapes():
    """C4 geometry (H 7168, I = Is = 2048, top-8, 8 groups keep 4) with
    E = 32 experts and T = 256 tokens so the CPU oracle stays fast."""
    T, H, E, I, k = 256, 7168, 32, 2048, 8
    x, W = deepseek_mxfp4_gpu(seed=4, T=T, H=H, E=E, I=I, Is=I)
    route = dict(n_group=8, topk_group=4, scoring="sigmoid", route_scale=2.5,
                 swiglu_limit=10.0)
    layer = deepseek_layer(W, k, **route)
    y, r = layer.forward(x, mode="prefill", return_routing=True)
    _, ids_ref = dm.moe_route(r["logits"], W.bias, k, "sigmoid", 2.5, 8, 4)
    np.testing.assert_array_equal(r["ids"], ids_ref.astype(np.int32))
    want = dm.moe_layer_mxfp4(x, r["logits"], W, k, 10.0, "sigmoid", 2.5, 8, 4)
    rel, mabs, scale = _report("deepseek prefill C4 shapes", y, want)
    assert rel < 3e-3


@pytest.mark.parametrize("B", [1, 8, 24, 64])
def test_deepseek_decode(B):
    x, W = deepseek_mxfp4(seed=50 + B, T=B, H=1024, E=16, I=512, Is=512)
    route = dict(n_group=4, topk_group=2, scoring="sigmoid", route_scale=2.5,
                 swiglu_limit=10.0)
    layer = deepseek_layer(W, 4, **route)
    y, r = layer.forward(x, mode="decode", return_routing=True)
    from oracle.codecs import dequant_fp4_block, dequant_fp8_block

    def ex(e):
        return (dequant_fp4_block(W.w1_p[e], W.w1_s[e]),
                dequant_fp4_block(W.w3_p[e], W.w3_s[e]),
                dequant_fp4_block(W.w2_p[e], W.w2_s[e]))
    sh = (dequant_fp8_block(W.s1_q, W.s1_s), dequant_fp8_block(W.s3_q, W.s3_s),
          dequant_fp8_block(W.s2_q, W.s2_s))
    want = dm.moe_block_forward(x, r["logits"], W.bias, ex, sh, 4, 10.0,
                                "sigmoid", 2.5, 4, 2)
    rel, mabs, scale = _report(f"deepseek decode B={B}", y, want)
    assert rel < 1e-4


@pytest.mark.parametrize("B,hashed", [(1, False), (8, False), (24, False),
                                      (64, False), (13, True)])
def test_deepseek_decode_inline_permutation_matches_launch(B, hashed, monkeypatch):
    """Streamed DeepSeek decode builds the expert-major permutation in the
    routed gate/up launch (every workgroup in LDS, workgroup 0 writing the
    tables for the down and combine launches) from the grouped or hash
    routing launch's ids; SLLM_MOE_ROUTE_INLINE=0 runs the permutation
    launch instead. The output and the routing agree bit for bit."""
    x, W = deepseek_mxfp4(seed=90 + B, T=B, H=1024, E=16, I=512, Is=512)
    kw = dict(n_group=4, topk_group=2, scoring="sigmoid", route_scale=2.5,
              swiglu_limit=10.0)
    fwd = {}
    if hashed:
        rng = np.random.default_rng(B)
        tid2eid = np.stack([rng.permutation(16)[:4] for _ in range(40)]).astype(np.int32)
        kw = dict(scoring="sigmoid", route_scale=2.5, tid2eid=tid2eid)
        fwd = dict(token_ids=rng.integers(0, 40, B).astype(np.int32))
    layer = deepseek_layer(W, 4, **kw)
    monkeypatch.setenv("SLLM_MOE_ROUTE_INLINE", "1")
    y1, r1 = layer.forward(x, mode="decode", return_routing=True, **fwd)
    np.testing.assert_array_equal(layer.forward(x, mode="decode", **fwd), y1)
    monkeypatch.setenv("SLLM_MOE_ROUTE_INLINE", "0")
    y0, r0 = layer.forward(x, mode="decode", return_routing=True, **fwd)
    np.testing.assert_array_equal(y1.view(np.uint32), y0.view(np.uint32))
    for n in ("logits", "w", "ids", "counts"):
        np.testing.assert_array_equal(np.asarray(r1[n]).view(np.uint32),
                                      np.asarray(r0[n]).view(np.uint32), err_msg=n)


@pytest.mark.parametrize("B,scoring,groups,shared,E", [
    (1, "softmax", (4, 2), True, 32), (3, "sqrtsoftplus", (4, 2), True, 32),
    (5, "sigmoid", (1, 1), True, 32), (8, "sigmoid", (4, 2), False, 32),
    (2, "sigmoid", (8, 3), True, 32), (4, "sigmoid", (16, 4), True, 64),
    (16, "sigmoid", (4, 2), True, 32), (17, "sigmoid", (4, 2), True, 32)])
def test_deepseek_decode_variants_match_launches(B, scoring, groups, shared, E,
                                                 monkeypatch):
    """DeepSeek decode across the paths this batch size selects, against
    the separate launches (SLLM_MOE_ROUTE_INLINE=0: routing, permutation,
    finish launches) bit for bit, and against the decode oracle: every
    scoring rule and a group limit or none routed in the gate/up launch (up
    to 8 tokens), no shared expert (routed-only stream-K launches), 16
    tokens (the last batch whose shared expert joins the routed launches)
    and 17 (its own launches, 32-row tiles). Group scores: E = 64 (groups
    of 4 adjacent lanes) merges them by lane shuffles, E = 32 scans them."""
    ng, kg = groups
    x, W = deepseek_mxfp4(seed=300 + B, T=B, H=1024, E=E, I=512, Is=512,
                          shared=shared)
    kw = dict(n_group=ng, topk_group=kg, scoring=scoring, route_scale=2.5,
              swiglu_limit=10.0)
    layer = deepseek_layer(W, 4, **kw)
    monkeypatch.setenv("SLLM_MOE_ROUTE_INLINE", "1")
    y1, r1 = layer.forward(x, mode="decode", return_routing=True)
    monkeypatch.setenv("SLLM_MOE_ROUTE_INLINE", "0")
    y0, r0 = layer.forward(x, mode="decode", return_routing=True)
    np.testing.assert_array_equal(y1.view(np.uint32), y0.view(np.uint32))
    for n in ("w", "ids", "counts"):
        np.testing.assert_array_equal(np.asarray(r1[n]).view(np.uint32),
                                      np.asarray(r0[n]).view(np.uint32), err_msg=n)
    from oracle.codecs import dequant_fp4_block, dequant_fp8_block

    def ex(e):
        return (dequant_fp4_block(W.w1_p[e], W.w1_s[e]),
                dequant_fp4_block(W.w3_p[e], W.w3_s[e]),
                dequant_fp4_block(W.w2_p[e], W.w2_s[e]))
    sh = ((dequant_fp8_block(W.s1_q, W.s1_s), dequant_fp8_block(W.s3_q, W.s3_s),
           dequant_fp8_block(W.s2_q, W.s2_s)) if shared else None)
    want = dm.moe_block_forward(x, r1["logits"], W.bias, ex, sh, 4, 10.0,
                                scoring, 2.5, ng, kg)
    rel, mabs, scale = _report(f"deepseek decode {scoring} g{ng}/{kg} "
                               f"shared={shared} B={B}", y1, want)
    assert rel < 1e-4


@pytest.mark.parametrize("B", [1, 3, 8, 16])
def test_deepseek_decode_streamk_matches_whole_items(B, monkeypatch):
    """DeepSeek decode up to 16 tokens deals its mixed-format launches
    stream-K: each workgroup an equal range of the units' K steps, a unit's
    steps across two ranges summed from K slices (the first item writing
    zeros to slices no range reached). SLLM_MOE_STREAMK=0 deals whole
    K-split items. The two differ only in how the fp32 K partials are
    grouped: outputs within 2e-6 relative L2 of each other and routing
    equal; at 1 and 3 tokens the stream-K output is also checked against
    the decode oracle (bf16 activations, dequantized experts)."""
    import functools
    from oracle.codecs import dequant_fp4_block, dequant_fp8_block
    x, W = deepseek_mxfp4_gpu(seed=70 + B, T=B, H=4096, E=64, I=1536, Is=1536)
    kw = dict(n_group=8, topk_group=4, scoring="sigmoid", route_scale=2.5,
              swiglu_limit=10.0)
    layer = deepseek_layer(W, 6, **kw)
    monkeypatch.setenv("SLLM_MOE_STREAMK", "1")
    y1, r1 = layer.forward(x, mode="decode", return_routing=True)
    monkeypatch.setenv("SLLM_MOE_STREAMK", "0")
    y0, r0 = layer.forward(x, mode="decode", return_routing=True)
    np.testing.assert_array_equal(r1["ids"], r0["ids"])
    assert rel_l2(y1, y0) < 2e-6
    if B > 3:
        return

    @functools.lru_cache(maxsize=None)
    def ex(e):
        return (dequant_fp4_block(W.w1_p[e], W.w1_s[e]),
                dequant_fp4_block(W.w3_p[e], W.w3_s[e]),
                dequant_fp4_block(W.w2_p[e], W.w2_s[e]))
    sh = (dequant_fp8_block(W.s1_q, W.s1_s), dequant_fp8_block(W.s3_q, W.s3_s),
          dequant_fp8_block(W.s2_q, W.s2_s))
    want = dm.moe_block_forward(x, r1["logits"], W.bias, ex, sh, 6, 10.0,
                                "sigmoid", 2.5, 8, 4)
    rel, mabs, scale = _report(f"deepseek decode stream-K B={B}", y1, want)
    assert rel < 1e-4


@pytest.mark.parametrize("T", [1, 13, 32, 64])
def test_decode_router_split_logits(T):
    """Decode-size router GEMM with its K split over workgroups: the
    partial-logit slices are summed in the routing kernel and stored back
    (the debug copy reads them). Logits within 8 units of fp32 rounding of
    the fp64 product, relative to sum |x||w|; routing exact on them."""
    x, W = qwen_fp8(seed=80 + T, T=T, H=2048, E=64, I=256, Is=256)
    layer = qwen_layer(W, 6)
    y, r = layer.forward(x, mode="decode", return_routing=True)
    want = x.astype(np.float64) @ W.router_w.astype(np.float64).T
    mag = np.abs(x.astype(np.float64)) @ np.abs(W.router_w.astype(np.float64)).T
    assert np.all(np.abs(r["logits"] - want) <= 8 * 2.0 ** -24 * mag + 1e-30)
    _check_routing(r, 64, 6)
    rel = rel_l2(y, qm.moe_layer_fp8_dequant(x, r["logits"], W, 6))
    assert rel < 1e-4
