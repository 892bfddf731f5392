"""Byte codecs for the MoE weight and activation formats (oracle side).

Formats (OCP 8-bit/4-bit floating point, as the reference's loader defines
them in loaders/fp8.py:1-16):

- E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits. Exponent field 0 is
  subnormal (m * 2^-9). Exponent 15 is finite for mantissa 0..6 (256..448);
  0x7F / 0xFF are the only NaNs; there is no infinity.
- BF16: the upper half of an IEEE fp32.
- E8M0 (ue8m0): an exponent-only byte, 2^(u-127). The loader maps 0x00 to 0.0
  and 0xFF to NaN (loaders/fp8.py:145-156).
- E2M1FN (fp4): magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6} with the sign in bit 3.
  Two values share a byte; the low nibble is the even K index
  (loaders/fp8.py:177-200).

Every decoder here is pinned by tests/test_oracle_codecs.py against the
reference's own known answers (tests/test_loaders.py:57-70,
tests/test_loaders_deepseek.py:18-69, tests/test_deepseek_v4.py:148-185) and,
for the full byte range, against torch's float8_e4m3fn / float8_e8m0fnu
conversions (independent library routines). The round-to-nearest-even
encoders are pinned against torch's float -> float8_e4m3fn cast and against
brute-force nearest-value search.
"""

from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0
E2M1_MAX = 6.0


def _e4m3_table() -> np.ndarray:
    """Value of each of the 256 E4M3FN codes (loaders/fp8.py:34-55)."""
    codes = np.arange(256, dtype=np.int64)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    exp = (codes >> 3) & 0xF
    man = codes & 0x7
    mag = np.where(exp == 0, man * 2.0 ** -9,
                   (1.0 + man / 8.0) * np.exp2(exp.astype(np.float64) - 7.0))
    val = sign * mag
    val[(exp == 15) & (man == 7)] = np.nan
    return val.astype(np.float32)


E4M3_TABLE = _e4m3_table()

# E2M1FN value of each nibble (loaders/fp8.py:139-142).
FP4_TABLE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                      -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
                     dtype=np.float32)


def decode_e4m3fn(u8) -> np.ndarray:
    """E4M3FN bytes -> float32 (loaders/fp8.py:34-55)."""
    return E4M3_TABLE[np.asarray(u8, dtype=np.uint8)]


def encode_e4m3fn_rne(x) -> np.ndarray:
    """float32 -> E4M3FN byte, round to nearest, ties to even.

    Inputs must already lie in [-448, 448] (every caller clamps first, as
    the upstream act_quant does at ref/hf_sources/dsv4/kernel.py:83-92); a
    value outside raises. NaN maps to 0x7F. Exact: the significand is
    rounded with np.rint after scaling by a power of two.
    """
    x = np.asarray(x, dtype=np.float32)
    if np.any(np.abs(x) > E4M3_MAX):
        raise ValueError("encode_e4m3fn_rne: |x| > 448 (clamp first)")
    a = np.abs(x).astype(np.float64)
    sign = np.signbit(x).astype(np.uint8) << 7
    # frexp: a = f * 2^e with f in [0.5, 1); the normal range of E4M3 is
    # 2^-6 <= a, i.e. e >= -5.
    f, e = np.frexp(a)
    normal = a >= 2.0 ** -6
    # normal: mantissa steps of 2^(e-1-3); subnormal: fixed step 2^-9
    step_exp = np.where(normal, e - 4, -9)
    q = np.rint(np.ldexp(a, -step_exp))           # integer multiple of step
    # q counts steps: for normals it is in [8, 16] (16 = carry to next binade)
    exp_field = np.where(normal, e + 6, 0)        # stored exponent for f>=.5
    carry = normal & (q >= 16)
    exp_field = np.where(carry, exp_field + 1, exp_field)
    q = np.where(carry, q / 2, q)
    man = np.where(normal, q - 8, q)
    # subnormal that rounded up to 8 steps is the smallest normal (0x08)
    sub_carry = (~normal) & (man >= 8)
    exp_field = np.where(sub_carry, 1, exp_field)
    man = np.where(sub_carry, 0, man)
    code = (exp_field.astype(np.int64) << 3) | man.astype(np.int64)
    code = sign.astype(np.int64) | code
    code = np.where(np.isnan(x), 0x7F, code)
    return code.astype(np.uint8)


def decode_bf16(u16) -> np.ndarray:
    """BF16 bit patterns -> float32 (loaders/fp8.py:58-64)."""
    u16 = np.asarray(u16, dtype=np.uint16)
    return (u16.astype(np.uint32) << 16).view(np.float32)


def encode_bf16_rne(x) -> np.ndarray:
    """float32 -> BF16 bit patterns, round to nearest even.

    Same rounding as the reference's kernels/_sllm_cuda.py:to_bf16
    (:283-287). Pinned against torch's float32 -> bfloat16 cast.
    """
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def round_bf16(x) -> np.ndarray:
    """float32 rounded to the nearest bf16 value, returned as float32."""
    return decode_bf16(encode_bf16_rne(x))


def decode_ue8m0(u8) -> np.ndarray:
    """E8M0 bytes -> float32: 2^(u-127); 0x00 -> 0.0, 0xFF -> NaN
    (loaders/fp8.py:145-156)."""
    u8 = np.asarray(u8, dtype=np.uint8)
    # 0xFF (NaN below) is kept out of the exponent: 2^128 overflows float32
    out = np.exp2(np.minimum(u8, 0xFE).astype(np.float64) - 127.0).astype(np.float32)
    out = np.where(u8 == 0x00, np.float32(0.0), out)
    out = np.where(u8 == 0xFF, np.float32(np.nan), out)
    return out.astype(np.float32)


def _fp4_pair_table() -> np.ndarray:
    # byte b -> the two float32 values (low nibble, high nibble), as one
    # 8-byte word so a single gather decodes a byte
    b = np.arange(256)
    pair = np.stack([FP4_TABLE[b & 0x0F], FP4_TABLE[b >> 4]], axis=1)
    return np.ascontiguousarray(pair.astype(np.float32)).view(np.uint64).reshape(256)


_FP4_PAIRS = None


def decode_fp4_packed(packed) -> np.ndarray:
    """(N, K/2) packed E2M1 bytes -> (N, K) float32, low nibble = even k."""
    global _FP4_PAIRS
    if _FP4_PAIRS is None:
        _FP4_PAIRS = _fp4_pair_table()
    p = np.asarray(packed, dtype=np.uint8)
    out = _FP4_PAIRS[p].view(np.float32)
    return out.reshape(p.shape[:-1] + (p.shape[-1] * 2,))


def encode_e2m1_rne(x) -> np.ndarray:
    """float32 in [-6, 6] -> E2M1 nibble (0..15), nearest value, ties to the
    even code (the rounding of hardware float conversions). Used only to
    build synthetic FP4 weights; the layer consumes whatever bytes it is
    given."""
    x = np.asarray(x, dtype=np.float32)
    if np.any(np.abs(x) > E2M1_MAX):
        raise ValueError("encode_e2m1_rne: |x| > 6 (clamp first)")
    a = np.abs(x).astype(np.float64)
    mags = FP4_TABLE[:8].astype(np.float64)
    d = np.abs(a[..., None] - mags)                  # (..., 8)
    best = d.min(-1, keepdims=True)
    cand = d == best
    # ties: prefer the even code among the (at most two) nearest codes
    even = (np.arange(8) % 2 == 0)
    pick = np.where(cand & even, 1, 0) * 2 + np.where(cand, 1, 0)
    code = np.argmax(pick, axis=-1).astype(np.uint8)
    sign = np.signbit(x).astype(np.uint8) << 3
    return (code | sign).astype(np.uint8)


def pack_fp4(nibbles) -> np.ndarray:
    """(N, K) nibbles -> (N, K/2) bytes, low nibble = even k."""
    n = np.asarray(nibbles, dtype=np.uint8)
    return (n[..., 0::2] | (n[..., 1::2] << 4)).astype(np.uint8)


def dequant_fp8_block(q, scale, block=(128, 128)) -> np.ndarray:
    """W[i, j] = e4m3(q[i, j]) * scale[i // bh, j // bw]
    (loaders/fp8.py:98-135; scale shape (ceil(N/bh), ceil(K/bw)), N-block
    major, the orientation of the loader and of the upstream fp8_gemm)."""
    q = np.asarray(q, dtype=np.uint8)
    scale = np.asarray(scale, dtype=np.float32)
    bh, bw = block
    n, k = q.shape[-2:]
    want = ((n + bh - 1) // bh, (k + bw - 1) // bw)
    if scale.shape[-2:] != want:
        raise ValueError(f"scale shape {scale.shape} != {want} for {q.shape}")
    rows = np.arange(n) // bh
    cols = np.arange(k) // bw
    return decode_e4m3fn(q) * scale[..., rows[:, None], cols[None, :]]


def dequant_fp4_block(packed, scale_u8, block_w: int = 32) -> np.ndarray:
    """W[i, j] = e2m1(packed)[i, j] * 2^(s[i, j // 32] - 127)
    (loaders/fp8.py:177-200)."""
    w = decode_fp4_packed(packed)
    s = decode_ue8m0(scale_u8)
    k = w.shape[-1]
    if s.shape[-1] != (k + block_w - 1) // block_w or s.shape[-2] != w.shape[-2]:
        raise ValueError(f"fp4 scale shape {s.shape} does not fit {w.shape}")
    cols = np.arange(k) // block_w
    # a product past float32's range is inf, as in the loader's float32
    # product (e.g. 6 * 2^127); no warning for it
    with np.errstate(over="ignore"):
        return w * s[..., cols]
