"""Activation quantization and block-scaled GEMM semantics (oracle side).

Restates the upstream DeepSeek-V4 tilelang kernels that define where the
quantized MoE layer rounds (the reference's numpy oracles do not quantize
activations at all, ref/deepseek_v4.py:9-15):

- act_quant (ref/hf_sources/dsv4/kernel.py:40-125): per row and per
  128-column block, amax = max(|x|, 1e-4); the scale is
  s = amax * fp32(1/448), or with a ue8m0 scale format the power of two
  2^ceil(log2(amax * fp32(1/448))) (fast_round_scale, :22-37); the stored
  value is e4m3(clamp(x / s, -448, 448)) with round-to-nearest-even.
- fp8_gemm (:203-273): for every 128-wide K block, the fp8 x fp8 partial
  product is formed and accumulated as acc += partial * sa[m, kb] *
  sb[n // 128, kb] in fp32.
- fp4_gemm (:441-536): the same with a per-32 E8M0 weight scale:
  acc += partial32 * sa[m, kb // 4] * sb[n, kb].

Pinned by tests/test_oracle_quant.py: the invariants |q| <= 448,
dequantization error <= half an e4m3 step times s, exactness of
power-of-two scales, the reference's own QAT identities
(tests/test_deepseek_v4.py:148-185 restated), and brute-force fp64 dot
products for the GEMMs on tiny shapes.
"""

from __future__ import annotations

import numpy as np

from . import codecs

INV_448 = np.float32(1.0 / 448.0)
AMAX_FLOOR = np.float32(1e-4)


def pow2_ceil_f32(v) -> np.ndarray:
    """2^ceil(log2(v)) for positive normal fp32 v, from the IEEE bits
    (exponent, plus one when any mantissa bit is set), as
    ref/hf_sources/dsv4/kernel.py:22-37 computes it."""
    v = np.asarray(v, dtype=np.float32)
    bits = v.view(np.uint32)
    e = ((bits >> 23) & 0xFF).astype(np.int64) - 127
    e = e + ((bits & 0x7FFFFF) != 0)
    return np.ldexp(np.float32(1.0), e.astype(np.int32)).astype(np.float32)


def act_quant(x, block: int = 128, pow2: bool = False):
    """x (M, K) float32 -> (q uint8 (M, K) e4m3 codes, s float32 (M, K/block)).

    Arithmetic per element is single-precision IEEE, in this order:
    amax = max(max|x_blk|, 1e-4); s = amax * fp32(1/448) (rounded to fp32)
    [or its power-of-two ceiling]; q = rne_e4m3(clamp(x / s, +-448)).
    """
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    if k % block:
        raise ValueError(f"act_quant: K={k} not a multiple of {block}")
    xb = x.reshape(m, k // block, block)
    amax = np.maximum(np.abs(xb).max(-1), AMAX_FLOOR).astype(np.float32)
    s = (amax * INV_448).astype(np.float32)
    if pow2:
        s = pow2_ceil_f32(s)
    y = (xb / s[..., None]).astype(np.float32)
    y = np.clip(y, -codecs.E4M3_MAX, codecs.E4M3_MAX).astype(np.float32)
    q = codecs.encode_e4m3fn_rne(y).reshape(m, k)
    return q, s


def act_dequant(q, s, block: int = 128) -> np.ndarray:
    """Inverse view of act_quant: e4m3(q) * s per block (float32)."""
    q = np.asarray(q, dtype=np.uint8)
    m, k = q.shape
    v = codecs.decode_e4m3fn(q).reshape(m, k // block, block)
    return (v * np.asarray(s, np.float32)[..., None]).reshape(m, k)


def fp8_block_gemm(aq, sa, bq, sb, block: int = 128) -> np.ndarray:
    """C (M, N) = sum over K blocks of (e4m3(aq) @ e4m3(bq)^T)_kb * sa * sb.

    aq (M, K) e4m3 codes, sa (M, K/128) fp32; bq (N, K) e4m3 codes,
    sb (ceil(N/128), K/128) fp32. Accumulation follows fp8_gemm at
    ref/hf_sources/dsv4/kernel.py:244-257: an fp32 partial per K block,
    scaled and added to an fp32 accumulator.
    """
    a = codecs.decode_e4m3fn(aq)
    b = codecs.decode_e4m3fn(bq)
    m, k = a.shape
    n = b.shape[0]
    nkb = k // block
    sa = np.asarray(sa, np.float32)
    sb = np.asarray(sb, np.float32)
    sbn = sb[np.arange(n) // block]                     # (N, nkb)
    acc = np.zeros((m, n), np.float32)
    for kb in range(nkb):
        sl = slice(kb * block, (kb + 1) * block)
        part = (a[:, sl] @ b[:, sl].T).astype(np.float32)
        acc += part * (sa[:, kb:kb + 1] * sbn[None, :, kb])
    return acc


def fp4_block_gemm(aq, sa, bpacked, sb_u8, act_block: int = 128,
                   w_block: int = 32) -> np.ndarray:
    """C (M, N) = A_fp8 (M, K) @ B_fp4 (N, K)^T with a per-128 activation
    scale and a per-32 E8M0 weight scale (ref/hf_sources/dsv4/kernel.py:
    441-536): an fp32 partial per 32-wide K block, scaled by
    sa[m, kb // 4] * 2^(sb[n, kb] - 127) and accumulated in fp32."""
    a = codecs.decode_e4m3fn(aq)
    b = codecs.decode_fp4_packed(bpacked)
    wsc = codecs.decode_ue8m0(sb_u8)                     # (N, K/32)
    m, k = a.shape
    n = b.shape[0]
    sa = np.asarray(sa, np.float32)
    acc = np.zeros((m, n), np.float32)
    ratio = act_block // w_block
    for kb in range(k // w_block):
        sl = slice(kb * w_block, (kb + 1) * w_block)
        part = (a[:, sl] @ b[:, sl].T).astype(np.float32)
        acc += part * (sa[:, kb // ratio:kb // ratio + 1] * wsc[None, :, kb])
    return acc


def quantize_weight_fp8_block(w, block: int = 128, pow2: bool = False):
    """Synthetic-weight helper: W (N, K) fp32 -> (q e4m3 (N, K),
    s fp32 (ceil(N/128), ceil(K/128))) with s = amax/448 per 128x128 block
    (or its power-of-two ceiling, the ue8m0 checkpoint convention), q =
    rne_e4m3(clamp(W / s)). Dequantization is codecs.dequant_fp8_block."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    nb, kb = -(-n // block), -(-k // block)
    pad = np.zeros((nb * block, kb * block), np.float32)
    pad[:n, :k] = w
    blk = pad.reshape(nb, block, kb, block)
    amax = np.maximum(np.abs(blk).max(axis=(1, 3)), AMAX_FLOOR).astype(np.float32)
    s = (amax * INV_448).astype(np.float32)
    if pow2:
        s = pow2_ceil_f32(s)
    y = (blk / s[:, None, :, None]).astype(np.float32)
    y = np.clip(y, -codecs.E4M3_MAX, codecs.E4M3_MAX)
    q = codecs.encode_e4m3fn_rne(y).reshape(nb * block, kb * block)[:n, :k]
    return np.ascontiguousarray(q), s


def quantize_weight_mxfp4(w, block: int = 32):
    """Synthetic-weight helper: W (N, K) fp32 -> (packed (N, K/2) uint8,
    scale (N, K/32) e8m0 bytes) with s = 2^ceil(log2(amax/6)) per 32 along
    K, as ref/deepseek_v4.py:175-189 (_fp4_rt) chooses it, and RNE nibbles."""
    w = np.asarray(w, np.float32)
    n, k = w.shape
    if k % block:
        raise ValueError("K must be a multiple of 32")
    wb = w.reshape(n, k // block, block)
    amax = np.maximum(np.abs(wb).max(-1), np.float32(1e-30)).astype(np.float32)
    s = pow2_ceil_f32((amax * np.float32(1.0 / 6.0)).astype(np.float32))
    y = np.clip((wb / s[..., None]).astype(np.float32), -6.0, 6.0)
    nib = codecs.encode_e2m1_rne(y).reshape(n, k)
    e = np.round(np.log2(s.astype(np.float64))).astype(np.int64) + 127
    return codecs.pack_fp4(nib), e.astype(np.uint8)
