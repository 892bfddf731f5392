"""GPU parity of the layer's building blocks against the oracle, through the
C-ABI (libsllm_moe.so). Integer / byte / index results are compared bit for
bit; fp32 routing weights to rtol 1e-5 (the reference kernel test's bar,
tests/test_qwen4_kernels.py:73-79)."""
import numpy as np
import pytest

from oracle import codecs, quant
from oracle import deepseek_moe as dm
from oracle import qwen_moe as qm
from oracle.permute import permute as oracle_permute

from tests._fixtures import check_qwen_routing

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    from sllm_amd import _lib
    if not _lib.available():
        pytest.fail(f"libsllm_moe.so not loadable: {_lib._lib_error}")
    return _lib


# Device buffers made by dev()/empty() stay referenced until the test ends:
# an inline temporary (dev(a).ptr) would otherwise be freed by Python before
# the kernel that reads it is launched.
_KEEP = []


@pytest.fixture(autouse=True)
def _pin_buffers():
    yield
    from sllm_amd.runtime import sync
    sync()
    _KEEP.clear()


def dev(a):
    from sllm_amd.runtime import to_device_raw
    b = to_device_raw(np.ascontiguousarray(a))
    _KEEP.append(b)
    return b


def empty(nbytes):
    from sllm_amd.runtime import DeviceBuffer
    b = DeviceBuffer(max(int(nbytes), 4))
    _KEEP.append(b)
    return b


def host(buf, dtype, shape):
    from sllm_amd.runtime import sync
    sync()
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    return buf.copy_host_raw(np.uint8)[:n].view(dtype).reshape(shape)


# ---------------------------------------------------------------- codecs --

def test_hw_e4m3_decode_all_codes(L):
    """fp8 GEMM with an identity A reproduces every finite e4m3 code."""
    from sllm_amd import fp8
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    K = 256
    B = np.zeros((1, K), np.uint8)
    B[0, :codes.size] = codes
    A = np.eye(K, dtype=np.float32)
    got = fp8.fp8_gemm(A, B, np.ones((1, 2), np.float32), 128, 128)[:, 0]
    want = codecs.decode_e4m3fn(B[0])
    np.testing.assert_array_equal(got, want)


def test_act_quant_bit_exact(L):
    import os
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "codecs.npz"))
    rng = np.random.default_rng(0)
    T, H = 256, 2048
    x = codecs.round_bf16((rng.standard_normal((T, H)) *
                           rng.uniform(0.01, 30, (T, 1))).astype(np.float32))
    # include exact e4m3 midpoints scaled so that s = 1 (amax 448)
    mids = gold["enc_x"][:H - 1]
    x[0, :H - 1] = codecs.round_bf16(mids)
    x[0, H - 1] = 448.0
    xb = dev(codecs.encode_bf16_rne(x))
    for pow2 in (0, 1):
        q = empty(T * H)
        s = empty(T * (H // 128) * 4)
        L.check(L.lib().sllm_moe_act_quant(xb.ptr, T, H, pow2, q.ptr, s.ptr,
                                           None, None, None))
        qh = host(q, np.uint8, (T, H))
        sh = host(s, np.float32, (T, H // 128))
        qr, sr = quant.act_quant(x, pow2=bool(pow2))
        np.testing.assert_array_equal(sh.view(np.uint32), sr.view(np.uint32))
        np.testing.assert_array_equal(qh, qr)


def test_act_quant_gate(L):
    rng = np.random.default_rng(1)
    T, H = 37, 1024
    x = codecs.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
    gw = codecs.round_bf16((rng.standard_normal(H) * 0.02).astype(np.float32))
    q, s, g = empty(T * H), empty(T * H // 128 * 4), empty(T * 4)
    L.check(L.lib().sllm_moe_act_quant(dev(codecs.encode_bf16_rne(x)).ptr, T, H, 0,
                                       q.ptr, s.ptr,
                                       dev(codecs.encode_bf16_rne(gw)).ptr, g.ptr,
                                       None))
    want = 1.0 / (1.0 + np.exp(-(x.astype(np.float64) @ gw.astype(np.float64))))
    np.testing.assert_allclose(host(g, np.float32, (T,)), want, rtol=2e-6, atol=1e-7)


def test_weight_quantizers_bit_exact(L):
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((384, 640)) * 0.02).astype(np.float32)
    w[0, :5] = [0.0, -0.0, 1e-9, -3e-3, 0.07]
    wd = dev(w)
    for pow2 in (0, 1):
        q, s = empty(w.size), empty(3 * 5 * 4)
        L.check(L.lib().sllm_quantize_weight_fp8(wd.ptr, 384, 640, pow2, q.ptr,
                                                 s.ptr, None))
        qr, sr = quant.quantize_weight_fp8_block(w, pow2=bool(pow2))
        np.testing.assert_array_equal(host(s, np.float32, (3, 5)), sr)
        np.testing.assert_array_equal(host(q, np.uint8, w.shape), qr)
    p, e = empty(w.size // 2), empty(w.size // 32)
    L.check(L.lib().sllm_quantize_weight_mxfp4(wd.ptr, 384, 640, p.ptr, e.ptr, None))
    pr, er = quant.quantize_weight_mxfp4(w)
    np.testing.assert_array_equal(host(e, np.uint8, er.shape), er)
    np.testing.assert_array_equal(host(p, np.uint8, pr.shape), pr)


# ---------------------------------------------------------------- router --

def test_router_reference_case(L):
    """tests/test_qwen4_kernels.py:73-79 restated (seed 33, (5,16), k=4)."""
    from sllm_amd import q4
    rng = np.random.default_rng(33)
    logits = rng.standard_normal((5, 16)).astype(np.float32) * 2.0
    w, ids = q4.moe_router(logits, 4)
    w_ref, ids_ref = qm.moe_route(logits, 4)
    np.testing.assert_array_equal(ids, ids_ref.astype(np.int32))
    np.testing.assert_allclose(w, w_ref, rtol=1e-5, atol=1e-7)


def test_router_ties_lowest_ids(L):
    from sllm_amd import q4
    w, ids = q4.moe_router(np.zeros((3, 6), np.float32), 3)
    np.testing.assert_array_equal(ids, [[0, 1, 2]] * 3)
    np.testing.assert_allclose(w, 1 / 3, rtol=1e-6)


@pytest.mark.parametrize("T,E,k", [(4096, 512, 10), (64, 16, 4), (300, 2048, 16),
                                   (17, 100, 7), (5, 64, 64)])
def test_route_softmax_matches_oracle(L, T, E, k):
    rng = np.random.default_rng(T + E)
    logits = (rng.standard_normal((T, E)) * 0.9).astype(np.float32)
    logits[0, :] = logits[0, 0]          # an all-tie row
    logits[1, 5:9] = logits[1, 1]        # partial ties
    w, ids = empty(T * k * 4), empty(T * k * 4)
    L.check(L.lib().sllm_moe_route_softmax(dev(logits).ptr, w.ptr, ids.ptr, T, E,
                                           k, np.float32(1e-20), None))
    tied = check_qwen_routing(logits, host(ids, np.int32, (T, k)),
                              host(w, np.float32, (T, k)), k,
                              name=f"route_softmax T={T} E={E} k={k}")
    # rows 0 and 1 hold exact logit ties (decided by the lower id, which the
    # oracle's stable sort matches): a certified tie needs distinct logits
    # with equal fp32 probabilities, rare at this scale
    assert len(tied) <= 2


@pytest.mark.parametrize("G,kg,scoring", [(1, 1, "sigmoid"), (8, 4, "sigmoid"),
                                          (4, 2, "softmax"), (8, 3, "sqrtsoftplus")])
def test_route_grouped_matches_oracle(L, G, kg, scoring):
    rng = np.random.default_rng(7 + G)
    T, E, k = 2048, 256, 8
    logits = (rng.standard_normal((T, E)) * 0.9).astype(np.float32)
    logits[0] = 0.25                       # full tie row
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    w, ids = empty(T * k * 4), empty(T * k * 4)
    sc = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}[scoring]
    L.check(L.lib().sllm_moe_route_grouped(dev(logits).ptr, dev(bias).ptr, w.ptr,
                                           ids.ptr, T, E, k, G, kg, sc,
                                           np.float32(2.5), None))
    wr, ir = dm.moe_route(logits, bias, k, scoring, 2.5, G, kg)
    np.testing.assert_array_equal(host(ids, np.int32, (T, k)), ir.astype(np.int32))
    np.testing.assert_allclose(host(w, np.float32, (T, k)), wr, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("scoring", ["sigmoid", "softmax", "sqrtsoftplus"])
def test_route_hash_matches_oracle(L, scoring):
    """Hash layers: ids from the token-id table (out-of-range token ids
    clipped), weights the chosen experts' scores (ref/deepseek_v4.py:545-552)."""
    rng = np.random.default_rng(11)
    T, E, k, V = 301, 256, 8, 50
    logits = (rng.standard_normal((T, E)) * 0.9).astype(np.float32)
    tid2eid = np.stack([rng.permutation(E)[:k] for _ in range(V)]).astype(np.int32)
    tok = rng.integers(-5, V + 5, T).astype(np.int32)
    w, ids = empty(T * k * 4), empty(T * k * 4)
    sc = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}[scoring]
    L.check(L.lib().sllm_moe_route_hash(dev(logits).ptr, dev(tok).ptr,
                                        dev(tid2eid).ptr, V, w.ptr, ids.ptr, T,
                                        E, k, sc, np.float32(1.5), None))
    wr, ir = dm.moe_route(logits, None, k, scoring, 1.5, token_ids=tok,
                          tid2eid=tid2eid)
    np.testing.assert_array_equal(host(ids, np.int32, (T, k)), ir.astype(np.int32))
    np.testing.assert_allclose(host(w, np.float32, (T, k)), wr, rtol=2e-6, atol=1e-7)


def test_router_gemm_matches_fp64(L):
    rng = np.random.default_rng(3)
    for T, E, H in [(4096, 512, 2048), (64, 16, 1024), (33, 100, 256),
                    (100, 300, 256), (1, 512, 2048), (65, 40, 384)]:
        x = codecs.round_bf16(rng.standard_normal((T, H)).astype(np.float32))
        wr = codecs.round_bf16((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
        out = empty(T * E * 4)
        L.check(L.lib().sllm_moe_router_gemm(dev(codecs.encode_bf16_rne(x)).ptr,
                                             dev(codecs.encode_bf16_rne(wr)).ptr,
                                             out.ptr, T, E, H, None))
        got = host(out, np.float32, (T, E))
        want = x.astype(np.float64) @ wr.astype(np.float64).T
        mag = np.abs(x.astype(np.float64)) @ np.abs(wr.astype(np.float64)).T
        assert np.all(np.abs(got - want) <= 4 * 2.0 ** -24 * mag + 1e-30)


# --------------------------------------------------------------- permute --

def _run_permute(L, ids, E, bm):
    from sllm_amd.runtime import sync
    T, k = ids.shape
    N = T * k
    max_tiles = -(-N // bm) + min(E, N)
    bufs = dict(counts=empty(E * 4), offsets=empty((E + 1) * 4),
                sorted=empty(N * 4), inv=empty(N * 4),
                tiles=empty(max_tiles * 16), nt=empty(4))
    scr = empty(L.lib().sllm_moe_permute_scratch_bytes(N, E))
    L.check(L.lib().sllm_moe_permute(dev(ids.astype(np.int32)).ptr, N, E, bm,
                                     bufs["counts"].ptr, bufs["offsets"].ptr,
                                     bufs["sorted"].ptr, bufs["inv"].ptr,
                                     bufs["tiles"].ptr, bufs["nt"].ptr, max_tiles,
                                     scr.ptr, None))
    sync()
    nt = int(host(bufs["nt"], np.int32, (1,))[0])
    return dict(counts=host(bufs["counts"], np.int32, (E,)),
                offsets=host(bufs["offsets"], np.int32, (E + 1,)),
                sorted_idx=host(bufs["sorted"], np.int32, (N,)),
                inv_pos=host(bufs["inv"], np.int32, (N,)),
                tiles=host(bufs["tiles"], np.int32, (max_tiles, 4))[:nt])


@pytest.mark.parametrize("T,E,k,skew", [(4096, 512, 10, False), (16384, 512, 10, True),
                                        (1, 512, 10, False), (3, 7, 2, False),
                                        (1000, 2048, 16, True), (2000, 1024, 8, True),
                                        (20000, 256, 8, False)])
def test_permute_bit_exact(L, T, E, k, skew):
    rng = np.random.default_rng(T + E)
    if skew:
        # Zipf-like popularity with many empty experts
        pop = 1.0 / np.arange(1, E + 1) ** 1.2
        pop[E // 2:] = 0.0
        pop /= pop.sum()
        ids = np.stack([rng.choice(E, size=k, replace=False, p=pop) for _ in range(T)])
    else:
        ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    got = _run_permute(L, ids, E, 128)
    want = oracle_permute(ids, E)
    for key in ("counts", "offsets", "sorted_idx", "inv_pos"):
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    # tile table: every non-empty expert in order, ceil(count/128) tiles of
    # {expert, first permuted row, rows, 0}
    c, o = want["counts"], want["offsets"]
    exp_tiles = [(e, o[e] + r, min(128, c[e] - r), 0)
                 for e in range(E) for r in range(0, c[e], 128)]
    np.testing.assert_array_equal(got["tiles"], np.array(exp_tiles, np.int32).reshape(-1, 4))


def test_fill_normal_deterministic_and_normal(L):
    from sllm_amd.runtime import fill_normal
    n = 1 << 20
    a, b = empty(n * 4), empty(n * 4)
    fill_normal(a, n, 7, 2.0)
    fill_normal(b, n, 7, 2.0)
    x = host(a, np.float32, (n,))
    np.testing.assert_array_equal(x, host(b, np.float32, (n,)))
    assert abs(x.mean()) < 0.01 and abs(x.std() - 2.0) < 0.01
    assert abs((np.abs(x) < 2.0).mean() - 0.6827) < 0.003


def _np_rows(up, nt, w, s, l):
    """Weight row fed by lane l of wave w, subtile s, column slab nt."""
    return (nt * 128 + w * 16 + (l & 15)) if up else \
        (nt * 256 + w * 32 + s * 16 + (l & 15))


def _np_pack_fp8(w0, w1, up):
    """numpy statement of the fp8 streaming layout (gemm_stream.hip):
    32 KB blocks [wave 8][subtile 2][half 2][lane 64][16 B] per
    (expert, slab, K step); gate/up subtile 1 is W3."""
    E, N, K = w0.shape
    NT, KB = (N // 128 if up else N // 256), K // 128
    out = np.empty(E * NT * KB * 32768, np.uint8)
    c = np.arange(out.size // 16)
    l, h, s, w = c & 63, (c >> 6) & 1, (c >> 7) & 1, (c >> 8) & 7
    blk = c >> 11
    kb, t = blk % KB, blk // KB
    nt, e = t % NT, t // NT
    row = _np_rows(up, nt, w, s, l)
    col = kb * 128 + (l >> 4) * 32 + h * 16
    src = np.where((s == 1) & bool(up), 1, 0)
    both = np.stack([w0, w1 if w1 is not None else w0])
    for b in range(16):
        out[c * 16 + b] = both[src, e, row, col + b]
    return out


def _np_pack_fp4(w0, w1, s0, s1, up):
    """fp4 streaming layout: 16 KB blocks [wave 8][subtile 2][lane 64][16 B]
    and 1 KB scale blocks [wave 8][lane 64][subtile 2] of e8m0 bytes."""
    E, N, Kh = w0.shape
    K = Kh * 2
    NT, KB = (N // 128 if up else N // 256), K // 128
    out = np.empty(E * NT * KB * 16384, np.uint8)
    outs = np.empty(E * NT * KB * 512, np.uint16)
    c = np.arange(out.size // 16)
    l, s, w = c & 63, (c >> 6) & 1, (c >> 7) & 7
    blk = c >> 10
    kb, t = blk % KB, blk // KB
    nt, e = t % NT, t // NT
    row = _np_rows(up, nt, w, s, l)
    col = kb * 64 + (l >> 4) * 16
    src = np.where((s == 1) & bool(up), 1, 0)
    both = np.stack([w0, w1 if w1 is not None else w0])
    sboth = np.stack([s0, s1 if s1 is not None else s0])
    for b in range(16):
        out[c * 16 + b] = both[src, e, row, col + b]
    sel = s == 0
    v = np.zeros(sel.sum(), np.uint16)
    for q in range(2):
        rq = _np_rows(up, nt[sel], w[sel], q, l[sel])
        sq = 1 if (q == 1 and up) else 0
        v |= sboth[sq, e[sel], rq, kb[sel] * 4 + (l[sel] >> 4)].astype(np.uint16) << (8 * q)
    outs[blk[sel] * 512 + w[sel] * 64 + l[sel]] = v
    return out, outs


@pytest.mark.parametrize("up", [1, 0])
def test_pack_weights_layout(L, up):
    from sllm_amd.moe import pack_weights
    rng = np.random.default_rng(11 + up)
    E, N, K = 3, 256, 384
    w0 = rng.integers(0, 256, (E, N, K), dtype=np.uint8)
    w1 = rng.integers(0, 256, (E, N, K), dtype=np.uint8) if up else None
    d0, d1 = dev(w0), (dev(w1) if up else None)
    p, _ = pack_weights(0, up, d0, d1, E, N, K)
    _KEEP.append(p)
    np.testing.assert_array_equal(host(p, np.uint8, (p.nbytes,)), _np_pack_fp8(w0, w1, up))
    f0 = rng.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    f1 = rng.integers(0, 256, (E, N, K // 2), dtype=np.uint8) if up else None
    s0 = rng.integers(0, 256, (E, N, K // 32), dtype=np.uint8)
    s1 = rng.integers(0, 256, (E, N, K // 32), dtype=np.uint8) if up else None
    p4, ps = pack_weights(1, up, dev(f0), dev(f1) if up else None, E, N, K,
                          dev(s0), dev(s1) if up else None)
    _KEEP.extend([p4, ps])
    want, wants = _np_pack_fp4(f0, f1, s0, s1, up)
    np.testing.assert_array_equal(host(p4, np.uint8, (p4.nbytes,)), want)
    np.testing.assert_array_equal(host(ps, np.uint16, (ps.nbytes // 2,)), wants)


@pytest.mark.parametrize("E,k", [(512, 10), (2048, 16), (64, 8)])
def test_route_heavy_ties(L, E, k):
    """Logits from a five-value set, signed zeros included: most picks tie
    with other lanes and within a lane, so the lower-id rule decides
    everywhere (both the sorted per-lane path, <= 8 keys per lane, and the
    32-keys-per-lane path). Equal logits give bitwise equal probabilities,
    so the oracle's order is exact and the ids must match bit for bit."""
    rng = np.random.default_rng(E + k)
    T = 40
    vals = np.array([-2.0, -1.0, -0.0, 0.0, 1.0], np.float32)
    logits = vals[rng.integers(0, 5, (T, E))]
    logits[3] = 0.0
    logits[4] = -0.0
    w, ids = empty(T * k * 4), empty(T * k * 4)
    L.check(L.lib().sllm_moe_route_softmax(dev(logits).ptr, w.ptr, ids.ptr, T, E,
                                           k, np.float32(1e-20), None))
    wr, ir = qm.moe_route(logits, k)
    np.testing.assert_array_equal(host(ids, np.int32, (T, k)), ir.astype(np.int32))
    np.testing.assert_allclose(host(w, np.float32, (T, k)), wr, rtol=1e-5, atol=1e-7)
