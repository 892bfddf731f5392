"""GPU parity of the reference-named C-ABI surface (the drop-in boundary):
the restated reference kernel tests (tests/test_qwen4_kernels.py:81-97,
tests/test_fp8_gemm.py:44-68, tests/test_deepseek_cuda.py:18-30) plus the
scale-orientation case the reference's 1x1-scale test cannot see."""
import numpy as np
import pytest

from oracle import codecs, quant

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    from sllm_amd import _lib
    if not _lib.available():
        pytest.fail(f"libsllm_moe.so not loadable: {_lib._lib_error}")


def _silu(x):
    return x / (1.0 + np.exp(-x))


def test_swiglu_axpy_shared_gate():
    from sllm_amd import q4
    rng = np.random.default_rng(34)
    g = rng.standard_normal((3, 6)).astype(np.float32)
    u = rng.standard_normal((3, 6)).astype(np.float32)
    np.testing.assert_allclose(q4.swiglu(g, u), _silu(g) * u, rtol=1e-5, atol=1e-7)
    out = rng.standard_normal((3, 6)).astype(np.float32)
    y = rng.standard_normal((3, 6)).astype(np.float32)
    w = rng.random(3).astype(np.float32)
    np.testing.assert_allclose(q4.axpy_rows(out, y, w), out + w[:, None] * y,
                               rtol=1e-6, atol=1e-7)
    gate = rng.standard_normal(3).astype(np.float32)
    sh = rng.standard_normal((3, 6)).astype(np.float32)
    np.testing.assert_allclose(q4.shared_gate_accum(out, sh, gate),
                               out + (1.0 / (1.0 + np.exp(-gate)))[:, None] * sh,
                               rtol=1e-5, atol=1e-7)


def test_dev_variants_match_host():
    from sllm_amd import q4
    from sllm_amd.runtime import DeviceBuffer, sync, to_device
    rng = np.random.default_rng(35)
    logits = rng.standard_normal((40, 128)).astype(np.float32)
    w_h, ids_h = q4.moe_router(logits, 8)
    w_d, i_d = DeviceBuffer(40 * 8 * 4), DeviceBuffer(40 * 8 * 4)
    lg_d = to_device(logits)
    q4.moe_router_dev(lg_d, w_d, i_d, 40, 128, 8)
    sync()
    np.testing.assert_array_equal(w_d.copy_host().reshape(40, 8), w_h)
    np.testing.assert_array_equal(i_d.copy_host_raw(np.int32, (40, 8)), ids_h)
    g = rng.standard_normal(1000).astype(np.float32)
    u = rng.standard_normal(1000).astype(np.float32)
    o = DeviceBuffer(4000)
    g_d, u_d = to_device(g), to_device(u)
    q4.swiglu_dev(g_d, u_d, o, 1000)
    sync()
    np.testing.assert_array_equal(o.copy_host(), q4.swiglu(g, u))


def test_router_rejects_bad_args():
    from sllm_amd import q4
    with pytest.raises(RuntimeError, match="rc=-1"):
        q4.moe_router(np.zeros((2, 4), np.float32), 5)     # topk > E
    with pytest.raises(RuntimeError, match="rc=-1"):
        q4.moe_router(np.zeros((2, 4096), np.float32), 4)  # E > 2048


def test_fp8_gemm_reference_cases():
    from sllm_amd import fp8
    rng = np.random.default_rng(7)
    M, N, K = 4, 5, 64
    a = rng.standard_normal((M, K)).astype(np.float32) * 0.1
    b8 = codecs.encode_e4m3fn_rne(np.clip(rng.standard_normal((N, K)).astype(np.float32)
                                          * 0.05, -448, 448))
    scale = (rng.standard_normal((1, 1)).astype(np.float32) * 0.5 + 1.0)
    want = codecs.dequant_fp8_block(b8, scale)
    np.testing.assert_allclose(fp8.fp8_gemm(a, b8, scale), a @ want.T, rtol=2e-4, atol=2e-4)


def test_fp8_gemm_scale_orientation():
    """Non-square scale grid: (ceil(N/128), ceil(K/128)) N-block-major, the
    loader's orientation (loaders/fp8.py:98-135)."""
    from sllm_amd import fp8
    rng = np.random.default_rng(8)
    M, N, K = 7, 300, 200
    a = rng.standard_normal((M, K)).astype(np.float32)
    b8 = rng.integers(0, 256, (N, K), dtype=np.uint8)
    b8[(b8 & 0x7F) == 0x7F] = 0x30
    scale = (rng.random((3, 2)) + 0.5).astype(np.float32)
    want = a.astype(np.float64) @ codecs.dequant_fp8_block(b8, scale).astype(np.float64).T
    got = fp8.fp8_gemm(a, b8, scale)
    mag = np.abs(a) @ np.abs(codecs.dequant_fp8_block(b8, scale)).T
    assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-6)
    # other block shapes
    s2 = (rng.random((5, 4)) + 0.5).astype(np.float32)
    got2 = fp8.fp8_gemm(a, b8, s2, 64, 64)
    want2 = a @ codecs.dequant_fp8_block(b8, s2, (64, 64)).T
    np.testing.assert_allclose(got2, want2, rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("M,N,K", [(1, 256, 512), (33, 384, 1024), (64, 128, 128)])
def test_fp8_gemm_decode_shapes(M, N, K):
    """sllm_fp8_gemm at decode sizes with 128 x 128 blocks (M <= 64, N and K
    multiples of 128: the unpacked-weight GEMV path) against the fp64
    product with the dequantized weight."""
    from sllm_amd import fp8
    rng = np.random.default_rng(M + N + K)
    a = rng.standard_normal((M, K)).astype(np.float32)
    b8 = rng.integers(0, 256, (N, K), dtype=np.uint8)
    b8[(b8 & 0x7F) == 0x7F] = 0x30
    scale = (rng.random((N // 128, K // 128)) + 0.5).astype(np.float32)
    wd = codecs.dequant_fp8_block(b8, scale).astype(np.float64)
    want = a.astype(np.float64) @ wd.T
    got = fp8.fp8_gemm(a, b8, scale)
    mag = np.abs(a) @ np.abs(wd).T
    assert np.all(np.abs(got - want) <= 1e-5 * mag + 1e-6)


@pytest.mark.parametrize("rows,K,O", [(1, 2048, 512), (7, 100, 48), (80, 64, 30)])
@pytest.mark.parametrize("post,scale", [(0, 1.0), (1, 2.0), (2, 0.5)])
def test_q4_gemv_rows(rows, K, O, post, scale):
    """sllm_q4_gemv_rows (host) and _dev: A . W^T then silu / sigmoid of
    x / scale (ref kernels/cuda/qwen4.cu:95-136), against fp64; bad sizes
    return -1. Shapes take the GEMV path (rows <= 64, O % 16 == 0) and the
    tiled one."""
    from sllm_amd import q4
    from sllm_amd.runtime import DeviceBuffer, sync, to_device
    rng = np.random.default_rng(rows * K + O + post)
    A = rng.standard_normal((rows, K)).astype(np.float32)
    W = (rng.standard_normal((O, K)) * 0.05).astype(np.float32)
    x = A.astype(np.float64) @ W.astype(np.float64).T
    if post == 1:
        want = (x / scale) / (1 + np.exp(-(x / scale)))
    elif post == 2:
        want = 1 / (1 + np.exp(-(x / scale)))
    else:
        want = x
    np.testing.assert_allclose(q4.gemv_rows(A, W, post, scale), want, rtol=2e-5, atol=2e-5)
    out = DeviceBuffer(rows * O * 4)
    q4.gemv_rows_dev(to_device(A), to_device(W), out, rows, K, O, post, scale)
    sync()
    np.testing.assert_allclose(out.copy_host().reshape(rows, O), want, rtol=2e-5, atol=2e-5)
    with pytest.raises(RuntimeError):
        q4.gemv_rows(np.zeros((0, 4), np.float32), np.zeros((4, 4), np.float32))


def test_silu_mul_f32_and_bf16():
    """sllm_silu_mul: out = silu(g) * u stored as fp32 or bf16 (RNE), with
    an odd element count (ref kernels/cuda/kernels.cu:897-919)."""
    from sllm_amd.runtime import DeviceBuffer, T_BF16, T_F32, silu_mul, sync, to_device
    rng = np.random.default_rng(3)
    n = 1001
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    want = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    gd, ud = to_device(g), to_device(u)
    o32 = DeviceBuffer(n * 4)
    silu_mul(gd, ud, o32, T_F32)
    o16 = DeviceBuffer(n * 2 + 2)
    silu_mul(gd, ud, o16, T_BF16)
    sync()
    np.testing.assert_allclose(o32.copy_host()[:n], want, rtol=1e-5, atol=1e-6)
    got16 = o16.copy_host_raw(np.uint16, (n + 1,))[:n]
    want16 = (codecs.round_bf16(o32.copy_host()[:n]).view(np.uint32) >> 16).astype(np.uint16)
    np.testing.assert_array_equal(got16, want16)


def test_fp4_linear_matches_dequant():
    from sllm_amd import deepseek
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    w = (rng.standard_normal((6, 64)) * 0.1).astype(np.float32)
    packed, s = quant.quantize_weight_mxfp4(w)
    got = deepseek.fp4_moe_linear(x, packed, s)
    want = x @ codecs.dequant_fp4_block(packed, s).T
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    got2 = deepseek.fp4_gemm_dequantized(x, codecs.dequant_fp4_block(packed, s))
    np.testing.assert_allclose(got2, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("M,N,K", [(1, 256, 512), (40, 128, 1024), (64, 48, 96)])
def test_fp4_linear_decode_shapes(M, N, K):
    """Packed MXFP4 linear at decode sizes (M <= 64, 32-column scale blocks:
    the unpacked-weight GEMV path), including e8m0 scale codes 0 (-> 0)
    and 255 (-> NaN, a NaN row), against the fp64 product."""
    from sllm_amd import deepseek
    rng = np.random.default_rng(M * N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
    packed, s = quant.quantize_weight_mxfp4(w)
    s = s.copy()
    s[3, 0] = 0
    s[5, 1] = 255
    got = deepseek.fp4_moe_linear(x, packed, s)
    wd = codecs.dequant_fp4_block(packed, s).astype(np.float64)
    want = x.astype(np.float64) @ wd.T
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    mag = np.abs(x) @ np.abs(np.nan_to_num(wd)).T
    assert np.all(np.abs(got - want)[ok] <= (1e-5 * mag + 1e-6)[ok])


def test_gemm_ex_f32_and_bf16():
    from sllm_amd.runtime import DeviceBuffer, T_BF16, T_F32, gemm_ex, sync, to_bf16, to_device, to_device_raw
    rng = np.random.default_rng(9)
    m, n, k = 1, 300, 257
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    c = DeviceBuffer(m * n * 4)
    a_d, w_d = to_device(a), to_device(w)
    gemm_ex(a_d, w_d, c, m, n, k, T_F32)
    sync()
    np.testing.assert_allclose(c.copy_host().reshape(m, n), a @ w.T, rtol=1e-4, atol=1e-4)
    ab_d, wb_d = to_device_raw(to_bf16(a)), to_device_raw(to_bf16(w))
    gemm_ex(ab_d, wb_d, c, m, n, k, T_BF16)
    sync()
    ab, wb = codecs.round_bf16(a), codecs.round_bf16(w)
    np.testing.assert_allclose(c.copy_host().reshape(m, n), ab @ wb.T, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("atype,m,n,k", [(0, 1, 4096, 2048), (0, 33, 160, 100),
                                         (0, 64, 48, 4), (1, 5, 64, 264), (1, 64, 32, 8)])
def test_gemm_ex_gemv_shapes(atype, m, n, k):
    """gemm_ex at m <= 64 outside the MFMA kernels' shapes (fp32 operands;
    bf16 with k % 128 != 0): the unpacked-weight GEMV, against fp64."""
    from sllm_amd.runtime import DeviceBuffer, T_BF16, T_F32, gemm_ex, sync, to_bf16, to_device, to_device_raw
    rng = np.random.default_rng(m * n + k + atype)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    c = DeviceBuffer(m * n * 4)
    if atype == 1:
        a, w = codecs.round_bf16(a), codecs.round_bf16(w)
        gemm_ex(to_device_raw(to_bf16(a)), to_device_raw(to_bf16(w)), c, m, n, k, T_BF16)
    else:
        gemm_ex(to_device(a), to_device(w), c, m, n, k, T_F32)
    sync()
    want = a.astype(np.float64) @ w.astype(np.float64).T
    mag = np.abs(a) @ np.abs(w).T
    got = c.copy_host().reshape(m, n)
    assert np.all(np.abs(got - want) <= 2e-6 * mag + 1e-6)


@pytest.mark.parametrize("m,n,k", [(1, 1000, 2048), (17, 300, 256), (64, 77, 128),
                                   (65, 200, 384), (300, 129, 1024)])
def test_gemm_ex_bf16_mfma_shapes(m, n, k):
    """bf16 gemm_ex with k % 128 == 0 (the MFMA router kernels: the K-split
    small-batch kernel for m <= 64, the 64 x 128 tiles above; ragged n and
    m): against the fp64 product of the bf16-rounded operands. bf16 products
    are exact in fp32, so only the fp32 accumulation order differs."""
    from sllm_amd.runtime import DeviceBuffer, T_BF16, gemm_ex, sync, to_bf16, to_device_raw
    rng = np.random.default_rng(m * n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.standard_normal((n, k)).astype(np.float32)
    c = DeviceBuffer(m * n * 4)
    gemm_ex(to_device_raw(to_bf16(a)), to_device_raw(to_bf16(w)), c, m, n, k, T_BF16)
    sync()
    want = (codecs.round_bf16(a).astype(np.float64)
            @ codecs.round_bf16(w).astype(np.float64).T)
    got = c.copy_host().reshape(m, n)
    err = np.abs(got - want).max() / np.sqrt(k)
    print(f"gemm_ex bf16 {m}x{n}x{k}: max |err| / sqrt(k) {err:.2e}")
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-4 * np.sqrt(k))


def test_buf_copy_exact_with_tail():
    """sllm_buf_copy (the calibration copy kernel): byte-exact over a size
    with a non-multiple-of-16 tail and over an empty copy."""
    from sllm_amd.runtime import DeviceBuffer, copy, sync
    rng = np.random.default_rng(5)
    n = (1 << 20) + 13
    src_h = rng.integers(0, 256, n, dtype=np.uint8)
    src = DeviceBuffer(n)
    src.upload_raw(src_h)
    dst = DeviceBuffer(n)
    copy(dst, src, n)
    copy(dst, src, 0)
    sync()
    np.testing.assert_array_equal(dst.copy_host_raw(np.uint8, (n,)), src_h)
