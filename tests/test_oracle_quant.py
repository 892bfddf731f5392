"""Pins oracle.quant: act_quant invariants, the reference's QAT identities
(tests/test_deepseek_v4.py:148-185 restated) and the block-scaled GEMMs
against brute-force fp64 dot products."""
import numpy as np

from oracle import codecs, quant


def test_act_quant_invariants():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((37, 512)) * rng.random((37, 1)) * 50).astype(np.float32)
    q, s = quant.act_quant(x)
    assert q.dtype == np.uint8 and s.shape == (37, 4)
    v = codecs.decode_e4m3fn(q).reshape(37, 4, 128)
    assert np.abs(v).max() <= 448.0
    # amax element maps to +-448 exactly when s = amax * (1/448) rounds down
    amax = np.abs(x.reshape(37, 4, 128)).max(-1)
    np.testing.assert_allclose(s, np.maximum(amax, 1e-4) / 448.0, rtol=1e-6)
    # dequant error <= half an e4m3 step (relative 2^-4) times |x| (normals)
    deq = quant.act_dequant(q, s)
    err = np.abs(deq - x)
    assert np.all(err <= np.abs(x) * 2.0 ** -4 + s.repeat(128, 1) * 2.0 ** -10)


def test_act_quant_pow2_exact_on_table_values():
    # restates tests/test_deepseek_v4.py:155-160: table values are fixed
    # points of the power-of-two quant round trip
    tbl = codecs.E4M3_TABLE[1:0x7F][::3].astype(np.float32)
    xs = np.zeros((len(tbl), 128), np.float32)
    xs[:, 0] = 448.0
    xs[:, 1:] = tbl[:, None]
    q, s = quant.act_quant(xs, pow2=True)
    assert np.all(s == 1.0)
    np.testing.assert_array_equal(quant.act_dequant(q, s), xs)


def test_pow2_ceil_matches_frexp():
    rng = np.random.default_rng(1)
    v = np.exp(rng.uniform(-20, 20, 10000)).astype(np.float32)
    v[:8] = np.float32([1, 2, 0.5, 4, 0.25, 3, 1.5, 2 ** -10])
    got = quant.pow2_ceil_f32(v)
    m, e = np.frexp(v.astype(np.float64))
    want = np.where(m > 0.5, 2.0 ** e, 2.0 ** (e - 1))
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_fp8_block_gemm_brute_force():
    rng = np.random.default_rng(2)
    M, N, K = 5, 260, 384
    a = rng.standard_normal((M, K)).astype(np.float32)
    aq, sa = quant.act_quant(a)
    bq = rng.integers(0, 256, (N, K), dtype=np.uint8)
    bq[(bq & 0x7F) == 0x7F] = 0x11
    sb = (rng.random((3, 3)) + 0.5).astype(np.float32)
    got = quant.fp8_block_gemm(aq, sa, bq, sb)
    A = codecs.decode_e4m3fn(aq).astype(np.float64)
    B = codecs.decode_e4m3fn(bq).astype(np.float64)
    want = np.zeros((M, N))
    mag = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            for k in range(K):
                t = A[m, k] * sa[m, k // 128] * B[n, k] * sb[n // 128, k // 128]
                want[m, n] += t
                mag[m, n] += abs(t)
    # fp32 accumulation bound: a few ulps of the sum of |terms|
    assert np.all(np.abs(got - want) <= 8 * 2.0 ** -24 * mag + 1e-30)
    # equivalent to dequantize-then-matmul
    deq = quant.act_dequant(aq, sa) @ codecs.dequant_fp8_block(bq, sb).T
    assert np.all(np.abs(got - deq) <= 16 * 2.0 ** -24 * mag + 1e-30)


def test_fp4_block_gemm_brute_force():
    rng = np.random.default_rng(3)
    M, N, K = 4, 6, 256
    a = rng.standard_normal((M, K)).astype(np.float32)
    aq, sa = quant.act_quant(a, pow2=True)
    packed = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    s = rng.integers(120, 135, (N, K // 32), dtype=np.uint8)
    got = quant.fp4_block_gemm(aq, sa, packed, s)
    A = codecs.decode_e4m3fn(aq).astype(np.float64)
    W = codecs.dequant_fp4_block(packed, s).astype(np.float64)
    want = np.zeros((M, N))
    for m in range(M):
        for k in range(K):
            want[m] += A[m, k] * sa[m, k // 128] * W[:, k]
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-5)


def test_weight_quantizers_roundtrip():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((300, 256)) * 0.02).astype(np.float32)
    q, s = quant.quantize_weight_fp8_block(w)
    assert s.shape == (3, 2)
    deq = codecs.dequant_fp8_block(q, s)
    assert np.abs(deq - w).max() <= np.abs(w).max() * 2 ** -4
    p, e = quant.quantize_weight_mxfp4(w)
    assert p.shape == (300, 128) and e.shape == (300, 8)
    d4 = codecs.dequant_fp4_block(p, e)
    blk = np.abs(w.reshape(300, 8, 32)).max(-1)
    # e2m1 spacing is at most 2 (between 4 and 6) in units of the scale;
    # the scale is < 2*amax/6, so the error is < amax/3
    assert np.all(np.abs(d4 - w).reshape(300, 8, 32).max(-1) <= blk / 3 + 1e-12)
