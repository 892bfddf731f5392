"""Pins oracle.codecs: the reference's known answers and library routines.

Known answers restated from the reference's tests:
tests/test_loaders.py:57-70 (E4M3), tests/test_loaders_deepseek.py:18-69
(E8M0, FP4 nibble order), tests/test_deepseek_v4.py:148-185 (table extremes,
E2M1 magnitudes). Full byte ranges and RNE encoders are checked against the
golden vectors tests/golden/codecs.npz written from torch's float8/bfloat16
conversions (tests/golden/make_golden.py).
"""
import os

import numpy as np
import pytest

from oracle import codecs

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "codecs.npz"))


def test_e4m3_known_values():
    cases = {0x00: 0.0, 0x01: 2.0 ** -9, 0x07: 7 * 2.0 ** -9, 0x08: 2.0 ** -6,
             0x38: 1.0, 0x3A: 1.25, 0x3C: 1.5, 0x68: 64.0, 0x78: 256.0,
             0x7E: 448.0}
    for byte, want in cases.items():
        assert codecs.decode_e4m3fn(np.uint8(byte)) == want, hex(byte)
    assert np.isnan(codecs.decode_e4m3fn(np.uint8(0x7F)))
    assert np.isnan(codecs.decode_e4m3fn(np.uint8(0xFF)))
    neg0 = codecs.decode_e4m3fn(np.uint8(0x80))
    assert neg0 == 0.0 and np.signbit(neg0)
    assert codecs.decode_e4m3fn(np.uint8(0xB8)) == -1.0


def test_e4m3_all_bytes_match_library():
    got = codecs.decode_e4m3fn(np.arange(256, dtype=np.uint8))
    want = GOLD["e4m3_all"]
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    fin = got[ok]
    assert fin.max() == 448.0 and np.abs(fin[fin != 0]).min() == 2.0 ** -9


def test_e4m3_encode_matches_library_rne():
    x, want = GOLD["enc_x"], GOLD["enc_e4m3"]
    got = codecs.encode_e4m3fn_rne(x)
    assert np.array_equal(got, want)


def test_e4m3_encode_is_nearest_by_brute_force():
    rng = np.random.default_rng(5)
    x = np.clip(rng.standard_normal(20000).astype(np.float32) * 40, -448, 448)
    code = codecs.encode_e4m3fn_rne(x)
    tbl = codecs.E4M3_TABLE.astype(np.float64)
    fin = ~np.isnan(tbl)
    d = np.abs(x[:, None].astype(np.float64) - np.where(fin, tbl, np.inf)[None])
    best = d.min(1)
    assert np.array_equal(d[np.arange(x.size), code], best)


def test_e4m3_encode_rejects_unclamped():
    with pytest.raises(ValueError):
        codecs.encode_e4m3fn_rne(np.float32([449.0]))


def test_e4m3_roundtrip_of_every_finite_code():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    vals = codecs.decode_e4m3fn(codes)
    assert np.array_equal(codecs.encode_e4m3fn_rne(vals), codes)


def test_bf16_rne_matches_library():
    got = codecs.encode_bf16_rne(GOLD["bf16_x"])
    assert np.array_equal(got, GOLD["bf16_bits"])
    assert codecs.decode_bf16(np.uint16(0x3FC0)) == 1.5


def test_e8m0_values():
    v = codecs.decode_ue8m0(np.array([127, 128, 126, 129, 0, 255], np.uint8))
    np.testing.assert_array_equal(v[:4], [1.0, 2.0, 0.5, 4.0])
    assert v[4] == 0.0 and np.isnan(v[5])
    x = np.arange(1, 255, dtype=np.uint8)
    got = codecs.decode_ue8m0(x)
    np.testing.assert_array_equal(got, GOLD["e8m0_all"][1:255])


def test_fp4_table_and_nibble_order():
    mags = codecs.FP4_TABLE[1:8].tolist()
    assert mags == [0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    rng = np.random.default_rng(2)
    N, K = 5, 200
    packed = rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    s = rng.integers(1, 255, size=(N, (K + 31) // 32), dtype=np.uint8)
    got = codecs.dequant_fp4_block(packed, s)
    want = np.empty((N, K), np.float32)
    for i in range(N):
        k = 0
        for j in range(K // 2):
            b = int(packed[i, j])
            for nib in (b & 0x0F, (b >> 4) & 0x0F):
                with np.errstate(over="ignore"):  # 6 * 2^127 is inf in float32
                    want[i, k] = codecs.FP4_TABLE[nib] * 2.0 ** (int(s[i, k // 32]) - 127)
                k += 1
    np.testing.assert_array_equal(got, want)


def test_e2m1_encode_nearest_even():
    x = np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.75, 6.0, 0.3])
    nib = codecs.encode_e2m1_rne(x)
    vals = codecs.FP4_TABLE[nib]
    np.testing.assert_array_equal(vals, [0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0,
                                         -1.0, 6.0, 0.5])


def test_fp8_block_dequant_matches_loop():
    rng = np.random.default_rng(1)
    q = rng.integers(0, 255, size=(260, 400), dtype=np.uint8)
    q[q == 127] = 126
    s = rng.random((3, 4), dtype=np.float32) + 0.1
    got = codecs.dequant_fp8_block(q, s)
    want = np.empty_like(got)
    for i in range(260):
        for j in range(400):
            want[i, j] = codecs.E4M3_TABLE[q[i, j]] * s[i // 128, j // 128]
    np.testing.assert_array_equal(got, want)
    with pytest.raises(ValueError):
        codecs.dequant_fp8_block(q, s[:2])
