"""Pins sllm_amd.loader's safetensors reader and writer against the
safetensors library itself (files written by either side read by the
other, F8 / BF16 dtypes through torch's float8 / bfloat16), the header
checks, and the scale decoding against the oracle codecs (whose E8M0 and
BF16 decoders are pinned to the reference loader tests)."""
import json
import os
import struct

import numpy as np
import pytest

from oracle import codecs
from sllm_amd import loader

torch = pytest.importorskip("torch")
st_torch = pytest.importorskip("safetensors.torch")
safetensors = pytest.importorskip("safetensors")

TORCH_TAGS = {"F32": torch.float32, "BF16": torch.bfloat16,
              "F8_E4M3": torch.float8_e4m3fn, "I32": torch.int32,
              "U8": torch.uint8, "I8": torch.int8, "F16": torch.float16}
if hasattr(torch, "float8_e8m0fnu"):
    TORCH_TAGS["F8_E8M0"] = torch.float8_e8m0fnu


def _tensors(rng):
    out = {}
    for i, (tag, dt) in enumerate(TORCH_TAGS.items()):
        shape = (3 + i, 5)
        raw = rng.integers(0, 256, int(np.prod(shape)) * loader.DTYPES[tag][1],
                           dtype=np.uint8)
        if tag == "F8_E8M0":
            raw[raw == 255] = 127  # keep NaN codes out of a byte comparison
        out[f"t.{tag.lower()}"] = (tag, shape, raw)
    return out


def _as_torch(tag, shape, raw):
    return torch.frombuffer(bytearray(raw.tobytes()), dtype=torch.uint8) \
        .view(TORCH_TAGS[tag]).reshape(shape)


def test_reads_files_written_by_safetensors(tmp_path):
    rng = np.random.default_rng(0)
    ts = _tensors(rng)
    p = str(tmp_path / "a.safetensors")
    st_torch.save_file({n: _as_torch(*v) for n, v in ts.items()}, p,
                       metadata={"format": "pt"})
    ck = loader.Checkpoint(p)
    for n, (tag, shape, raw) in ts.items():
        assert ck.spec(n) == (tag, shape)
        np.testing.assert_array_equal(ck.bytes(n), raw)


def test_written_files_read_by_safetensors(tmp_path):
    rng = np.random.default_rng(1)
    ts = _tensors(rng)
    p = str(tmp_path / "b.safetensors")
    loader.write_safetensors(p, ts)
    with safetensors.safe_open(p, framework="pt") as f:
        assert set(f.keys()) == set(ts)
        for n, (tag, shape, raw) in ts.items():
            t = f.get_tensor(n)
            assert t.dtype == TORCH_TAGS[tag] and tuple(t.shape) == shape
            got = t.contiguous().view(torch.uint8).reshape(-1).numpy()
            np.testing.assert_array_equal(got, raw)


def test_shards_and_missing_names(tmp_path):
    a, b = str(tmp_path / "s0.safetensors"), str(tmp_path / "s1.safetensors")
    loader.write_safetensors(a, {"x": ("F32", (2,), np.float32([1, 2]))})
    loader.write_safetensors(b, {"y": ("I32", (1,), np.int32([7]))})
    ck = loader.Checkpoint([a, b])
    np.testing.assert_array_equal(ck.array("x"), [1.0, 2.0])
    np.testing.assert_array_equal(ck.array("y"), [7])
    with pytest.raises(loader.CheckpointError):
        ck.bytes("z")


def _raw_file(path, header: dict, data: bytes, hlen=None):
    h = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h) if hlen is None else hlen))
        f.write(h)
        f.write(data)


@pytest.mark.parametrize("case", ["short", "cap", "truncated", "json", "dtype",
                                  "span", "offsets"])
def test_header_checks(tmp_path, case):
    p = str(tmp_path / "bad.safetensors")
    good = {"w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}
    if case == "short":
        open(p, "wb").write(b"\x01\x00")
    elif case == "cap":
        _raw_file(p, good, bytes(8), hlen=1 << 40)
    elif case == "truncated":
        _raw_file(p, good, b"", hlen=10_000)
    elif case == "json":
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", 4) + b"{{{{")
    elif case == "dtype":
        _raw_file(p, {"w": {"dtype": "F7", "shape": [2], "data_offsets": [0, 8]}}, bytes(8))
    elif case == "span":
        _raw_file(p, {"w": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, bytes(8))
    else:
        _raw_file(p, {"w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}, bytes(4))
    with pytest.raises(loader.CheckpointError):
        loader.Checkpoint(p)


def test_scale_decoding_matches_codecs(tmp_path):
    e8 = np.arange(256, dtype=np.uint8).reshape(16, 16)
    rng = np.random.default_rng(3)
    f32 = rng.standard_normal((4, 8)).astype(np.float32)
    bits = codecs.encode_bf16_rne(f32)
    p = str(tmp_path / "s.safetensors")
    loader.write_safetensors(p, {"e8": ("F8_E8M0", e8.shape, e8),
                                 "bf": ("BF16", bits.shape, bits),
                                 "f": ("F32", f32.shape, f32)})
    ck = loader.Checkpoint(p)
    got = loader.scale_f32(ck, "e8")
    want = codecs.decode_ue8m0(e8)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
    np.testing.assert_array_equal(loader.scale_f32(ck, "bf"), codecs.decode_bf16(bits))
    np.testing.assert_array_equal(loader.scale_f32(ck, "f"), f32)


@pytest.mark.parametrize("bad", [16, -1, 1000])
def test_hash_table_out_of_range_is_refused(tmp_path, bad):
    """A hash layer's tid2eid entry outside [0, E) raises before any weight
    reaches the device (ref/deepseek_v4.py:558 raises IndexError for ids >= E;
    the kernels would silently drop the slot)."""
    from sllm_amd.moe import check_tid2eid
    E, k = 16, 4
    rng = np.random.default_rng(5)
    t = np.stack([rng.permutation(E)[:k] for _ in range(30)]).astype(np.int32)
    np.testing.assert_array_equal(check_tid2eid(t, E, k), t)
    t[7, 2] = bad
    with pytest.raises(IndexError, match=r"tid2eid\[7, 2\]"):
        check_tid2eid(t, E, k)
    with pytest.raises(ValueError):
        check_tid2eid(t[:, :3], E, k)
    # through the loader: the table is read and checked first, so a CPU-only
    # process gets the IndexError (not a device error)
    p = str(tmp_path / "h.safetensors")
    H = 256
    loader.write_safetensors(p, {
        "ffn.gate.weight": ("F32", (E, H), np.zeros((E, H), np.float32)),
        "ffn.gate.tid2eid": ("I32", t.shape, t)})
    with pytest.raises(IndexError):
        loader.load_deepseek_moe(loader.Checkpoint(p), "", top_k=k, hash_layer=True)
