"""Checkpoint tensors straight to the device, in their on-disk formats.

The reference reads safetensors on the host and dequantizes FP8 / FP4
expert weights to float there (loaders/safetensors_reader.py,
loaders/fp8.py:98-228; kernels/q4_device_decode.py:118-122 then uploads
bf16/fp32). Here the expert weights stay in their stored formats end to
end. Each tensor's bytes go from the memory-mapped file into a stacked
device buffer:
- F8_E4M3 codes (Qwen experts, DeepSeek shared experts);
- packed E2M1 bytes and their F8_E8M0 block scales (DeepSeek routed
  experts).
The layer kernels consume these formats directly. Only the small per-block
scales of the FP8 weights are decoded on the host, to the fp32 the kernels
take:
- BF16 or F32 `weight_scale_inv` (Qwen);
- F8_E8M0 powers of two (DeepSeek shared experts).

File format (safetensors): an 8-byte little-endian header length, a UTF-8
JSON header {name: {"dtype", "shape", "data_offsets": [begin, end)}} (plus
an optional "__metadata__" entry), then the data; offsets are relative to
the start of the data.

Tensor names follow the reference checkpoints:
- Qwen (ref/qwen4_exp_pipeline.py:29-32, _moe_w :266-278):
  `{prefix}.gate.weight`, `{prefix}.experts.{e}.{gate,up,down}_proj.weight`
  [+ `.weight_scale_inv`], `{prefix}.shared_expert.{gate,up,down}_proj.*`,
  `{prefix}.shared_expert_gate.weight`.
- DeepSeek (ref/deepseek_v4.py:1023-1058; upstream convert.py:102 renames
  weight_scale_inv -> scale): `{prefix}ffn.gate.weight`, `ffn.gate.bias`,
  `ffn.experts.{e}.w{1,3,2}.{weight,scale}`,
  `ffn.shared_experts.w{1,3,2}.{weight,scale}`, and `tid2eid` for hash
  layers (`{prefix}ffn.gate.tid2eid`, else a global `tid2eid`).
"""

from __future__ import annotations

import json
import mmap
import os
import struct
from ctypes import c_void_p
from typing import Iterable

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, to_bf16, to_device_raw

# safetensors dtype tag -> (numpy dtype of the stored bytes, itemsize)
DTYPES = {
    "F64": (np.float64, 8), "F32": (np.float32, 4), "F16": (np.float16, 2),
    "BF16": (np.uint16, 2), "F8_E4M3": (np.uint8, 1), "F8_E5M2": (np.uint8, 1),
    "F8_E8M0": (np.uint8, 1), "I64": (np.int64, 8), "I32": (np.int32, 4),
    "I16": (np.int16, 2), "I8": (np.int8, 1), "U64": (np.uint64, 8),
    "U32": (np.uint32, 4), "U16": (np.uint16, 2), "U8": (np.uint8, 1),
    "BOOL": (np.bool_, 1),
}
HEADER_CAP = 1 << 28  # a corrupt length must not drive a huge read


class CheckpointError(ValueError):
    pass


class SafetensorsFile:
    """One safetensors file, memory-mapped; tensors are zero-copy views of
    their stored bytes."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            head = f.read(8)
            if len(head) < 8:
                raise CheckpointError(f"{path}: shorter than the header length")
            (hlen,) = struct.unpack("<Q", head)
            if hlen > HEADER_CAP:
                raise CheckpointError(f"{path}: header length {hlen} over the cap")
            raw = f.read(hlen)
            if len(raw) != hlen:
                raise CheckpointError(f"{path}: truncated header")
            size = os.fstat(f.fileno()).st_size
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else None
        try:
            doc = json.loads(raw.decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as exc:
            raise CheckpointError(f"{path}: header is not UTF-8 JSON ({exc})") from None
        if not isinstance(doc, dict):
            raise CheckpointError(f"{path}: header is not a JSON object")
        self.data_start = 8 + hlen
        data_len = size - self.data_start
        self.specs = {}
        for name, info in doc.items():
            if name == "__metadata__":
                continue
            try:
                dtype, shape, (b, e) = info["dtype"], tuple(int(d) for d in info["shape"]), info["data_offsets"]
            except (KeyError, TypeError, ValueError):
                raise CheckpointError(f"{path}: malformed entry {name!r}") from None
            if dtype not in DTYPES:
                raise CheckpointError(f"{path}: {name!r} has unknown dtype {dtype!r}")
            if any(d < 0 for d in shape) or not (0 <= b <= e <= data_len):
                raise CheckpointError(f"{path}: {name!r} has bad shape or offsets")
            if int(np.prod(shape, dtype=np.int64)) * DTYPES[dtype][1] != e - b:
                raise CheckpointError(f"{path}: {name!r}: shape {shape} does not "
                                      f"match its {e - b} bytes")
            self.specs[name] = (dtype, shape, b, e)

    def bytes(self, name: str) -> np.ndarray:
        """The tensor's stored bytes (uint8, zero-copy)."""
        dtype, shape, b, e = self.specs[name]
        if e == b:
            return np.zeros(0, np.uint8)
        return np.frombuffer(self._map, np.uint8, e - b, self.data_start + b)

    def array(self, name: str) -> np.ndarray:
        """The tensor as its stored dtype (BF16 as uint16 bits, F8 as uint8)."""
        dtype, shape, _, _ = self.specs[name]
        return self.bytes(name).view(DTYPES[dtype][0]).reshape(shape)


class Checkpoint:
    """A set of safetensors shards addressed by tensor name."""

    def __init__(self, paths: Iterable[str] | str):
        if isinstance(paths, (str, os.PathLike)):
            paths = [paths]
        self.files = [SafetensorsFile(str(p)) for p in paths]
        self._where = {}
        for f in self.files:
            for n in f.specs:
                self._where[n] = f

    def has(self, name: str) -> bool:
        return name in self._where

    def spec(self, name: str):
        if name not in self._where:
            raise CheckpointError(f"no tensor {name!r}")
        dtype, shape, _, _ = self._where[name].specs[name]
        return dtype, shape

    def bytes(self, name: str) -> np.ndarray:
        self.spec(name)
        return self._where[name].bytes(name)

    def array(self, name: str) -> np.ndarray:
        self.spec(name)
        return self._where[name].array(name)


def write_safetensors(path: str, tensors: dict) -> None:
    """Writes {name: (dtype tag, shape, array of that size)} in the
    safetensors format (used for tests and the bench's synthetic
    checkpoints)."""
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, arr) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        if len(b) != int(np.prod(shape, dtype=np.int64)) * DTYPES[dtype][1]:
            raise ValueError(f"{name}: {len(b)} bytes do not match {dtype} {shape}")
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode("utf-8")
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


# ---------------------------------------------------------------------------
# decoding of the (small) scale tensors to the kernels' fp32
# ---------------------------------------------------------------------------

def scale_f32(ckpt: Checkpoint, name: str) -> np.ndarray:
    """A block-scale tensor as fp32: BF16 bits shifted into the high half,
    F32 as stored, F8_E8M0 as 2^(u - 127) with 0x00 -> 0 and 0xFF -> NaN
    (loaders/fp8.py:145-156 conventions)."""
    dtype, _ = ckpt.spec(name)
    a = ckpt.array(name)
    if dtype == "BF16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    if dtype == "F32":
        return np.array(a, np.float32)
    if dtype == "F8_E8M0":
        u = a.astype(np.uint32)
        out = (np.clip(u, 1, 254) << 23).view(np.float32).copy()
        out[u == 0] = 0.0
        out[u == 255] = np.nan
        return out
    raise CheckpointError(f"{name!r}: {dtype} is not a scale format")


def _bf16_bits(ckpt: Checkpoint, name: str) -> np.ndarray:
    dtype, _ = ckpt.spec(name)
    if dtype == "BF16":
        return np.array(ckpt.array(name))
    if dtype in ("F32", "F16"):
        return to_bf16(ckpt.array(name).astype(np.float32))
    raise CheckpointError(f"{name!r}: expected BF16/F32/F16, got {dtype}")


def _stack(ckpt: Checkpoint, names, dtypes, shape) -> DeviceBuffer:
    """One device buffer holding the named tensors back to back, each copied
    from its mapped bytes (no host staging of the whole stack)."""
    for n in names:
        d, s = ckpt.spec(n)
        if d not in dtypes or tuple(s) != tuple(shape):
            raise CheckpointError(f"{n!r}: {d} {s}, expected one of {dtypes} {shape}")
    per = ckpt.bytes(names[0]).nbytes
    buf = DeviceBuffer(max(per * len(names), 4))
    L = _lib.lib()
    for i, n in enumerate(names):
        src = ckpt.bytes(n)
        _lib.check(L.sllm_buf_h2d_raw(c_void_p(buf.ptr + i * per),
                                      src.ctypes.data_as(c_void_p), per),
                   "sllm_buf_h2d_raw")
    return buf


def _cdiv(a, b):
    return -(-a // b)


# ---------------------------------------------------------------------------
# layers
# ---------------------------------------------------------------------------

def load_qwen_moe(ckpt: Checkpoint, prefix: str, top_k: int, eps: float = 1e-20,
                  packed: bool = True):
    """A QwenMoE from an FP8 checkpoint's MoE block at `prefix` (for example
    "model.language_model.layers.3.mlp"): F8_E4M3 expert weights with their
    128x128 `weight_scale_inv` blocks, bf16 router and shared-expert gate."""
    from .moe import QwenMoE
    E, H = ckpt.spec(f"{prefix}.gate.weight")[1]
    I = ckpt.spec(f"{prefix}.experts.0.gate_proj.weight")[1][0]
    ex = lambda e, m: f"{prefix}.experts.{e}.{m}_proj.weight"  # noqa: E731
    b = {"router_w": to_device_raw(_bf16_bits(ckpt, f"{prefix}.gate.weight"))}
    for key, m, shape in (("wg", "gate", (I, H)), ("wu", "up", (I, H)),
                          ("wd", "down", (H, I))):
        b[key] = _stack(ckpt, [ex(e, m) for e in range(E)], ("F8_E4M3",), shape)
        b[key + "_s"] = to_device_raw(np.stack(
            [scale_f32(ckpt, ex(e, m) + "_scale_inv") for e in range(E)]))
        want = (E, _cdiv(shape[0], 128), _cdiv(shape[1], 128))
        if b[key + "_s"].nbytes != 4 * int(np.prod(want)):
            raise CheckpointError(f"{prefix}.experts.*.{m}_proj scales are not {want[1:]}")
    Is = 0
    sp = f"{prefix}.shared_expert"
    if ckpt.has(f"{sp}.gate_proj.weight"):
        Is = ckpt.spec(f"{sp}.gate_proj.weight")[1][0]
        for key, m, shape in (("sg", "gate", (Is, H)), ("su", "up", (Is, H)),
                              ("sd", "down", (H, Is))):
            n = f"{sp}.{m}_proj.weight"
            b[key] = _stack(ckpt, [n], ("F8_E4M3",), shape)
            b[key + "_s"] = to_device_raw(scale_f32(ckpt, n + "_scale_inv"))
        b["sgl"] = to_device_raw(_bf16_bits(ckpt, f"{prefix}.shared_expert_gate.weight").reshape(-1))
    return QwenMoE.from_device(b, E=E, I=I, H=H, Is=Is, top_k=top_k, eps=eps,
                               packed=packed)


def load_dense_mlp(ckpt: Checkpoint, prefix: str, packed: bool = True):
    """A dense FP8 SwiGLU MLP at `prefix` (`{prefix}.{gate,up,down}_proj.weight`
    F8_E4M3 + `weight_scale_inv`) as a one-expert, top-1 QwenMoE with a zero
    router (the form sllm_amd.decode.DenseSwiGLU runs)."""
    from .moe import QwenMoE
    I, H = ckpt.spec(f"{prefix}.gate_proj.weight")[1]
    b = {"router_w": to_device_raw(np.zeros(H, np.uint16))}
    for key, m, shape in (("wg", "gate", (I, H)), ("wu", "up", (I, H)),
                          ("wd", "down", (H, I))):
        n = f"{prefix}.{m}_proj.weight"
        b[key] = _stack(ckpt, [n], ("F8_E4M3",), shape)
        s = scale_f32(ckpt, n + "_scale_inv")
        if s.shape != (_cdiv(shape[0], 128), _cdiv(shape[1], 128)):
            raise CheckpointError(f"{n}_scale_inv is {s.shape}, not 128x128 blocks")
        b[key + "_s"] = to_device_raw(np.ascontiguousarray(s, np.float32))
    return QwenMoE.from_device(b, E=1, I=I, H=H, Is=0, top_k=1, packed=packed)


def load_deepseek_moe(ckpt: Checkpoint, prefix: str, top_k: int, n_group=1,
                      topk_group=1, scoring="sigmoid", route_scale=1.0,
                      swiglu_limit=0.0, packed: bool = True,
                      hash_layer: bool = False):
    """A DeepseekMoE from a converted DeepSeek checkpoint's layer at `prefix`
    (for example "layers.3."): routed experts as packed E2M1 (I8/U8
    (N, K/2)) with F8_E8M0 (N, K/32) scales, shared experts as F8_E4M3 with
    F8_E8M0 128x128 scales; optional `ffn.gate.bias`. A hash layer
    (hash_layer, the first n_hash_layers) also loads its token-id table."""
    from .moe import DeepseekMoE, check_tid2eid
    g = f"{prefix}ffn.gate"
    E, H = ckpt.spec(f"{g}.weight")[1]
    tid2eid = None
    if hash_layer:  # checked before any weight is uploaded
        for n in (f"{g}.tid2eid", "tid2eid"):
            if ckpt.has(n):
                tid2eid = check_tid2eid(np.array(ckpt.array(n)), E, top_k)
                break
        if tid2eid is None:
            raise CheckpointError(f"{prefix}: hash layer without a tid2eid table")
    ep = lambda e, w: f"{prefix}ffn.experts.{e}.{w}"  # noqa: E731
    I = ckpt.spec(ep(0, "w1.weight"))[1][0]
    fp4 = ("I8", "U8")
    b = {"router_w": to_device_raw(_bf16_bits(ckpt, f"{g}.weight")),
         "bias": (to_device_raw(np.array(ckpt.array(f"{g}.bias"), np.float32))
                  if ckpt.has(f"{g}.bias") else None)}
    for w, (N, K) in (("w1", (I, H)), ("w3", (I, H)), ("w2", (H, I))):
        b[w] = _stack(ckpt, [ep(e, f"{w}.weight") for e in range(E)], fp4, (N, K // 2))
        b[w + "_s"] = _stack(ckpt, [ep(e, f"{w}.scale") for e in range(E)],
                             ("F8_E8M0", "U8"), (N, K // 32))
    Is = 0
    sp = f"{prefix}ffn.shared_experts"
    if ckpt.has(f"{sp}.w1.weight"):
        Is = ckpt.spec(f"{sp}.w1.weight")[1][0]
        for w, key, shape in (("w1", "s1", (Is, H)), ("w3", "s3", (Is, H)),
                              ("w2", "s2", (H, Is))):
            b[key] = _stack(ckpt, [f"{sp}.{w}.weight"], ("F8_E4M3",), shape)
            b[key + "_s"] = to_device_raw(scale_f32(ckpt, f"{sp}.{w}.scale"))
    return DeepseekMoE.from_device(
        b, E=E, I=I, H=H, Is=Is, top_k=top_k, n_group=n_group,
        topk_group=topk_group, scoring=scoring, route_scale=route_scale,
        swiglu_limit=swiglu_limit, packed=packed, tid2eid=tid2eid)
