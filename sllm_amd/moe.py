"""Fused MoE layer entry points over libsllm_moe.so.

The layer the reference computes in numpy (ref/qwen4_exp.py:153-184
moe_block_forward; ref/deepseek_v4.py:1070-1087 Block.moe with the upstream
combine of ref/hf_sources/dsv4/model.py:684-699) and, on the device, as a
host loop of per-expert cuBLAS GEMVs (kernels/q4_device_decode.py:316-339).

Two levels:
- `qwen_forward_dev` / `deepseek_forward_dev`: device pointers in, device
  pointers out, stream-ordered, no allocation (caller-owned workspace).
  Buffers may be DeviceBuffer / DeviceView objects, torch tensors or raw
  addresses.
- `QwenMoE` / `DeepseekMoE`: device-resident weights uploaded once from host
  arrays, with `forward(x)` taking and returning numpy arrays -- the drop-in
  for `moe_block_forward` and for `Q4DeviceDecodeState._moe`.
"""

from __future__ import annotations

import weakref
from ctypes import c_void_p
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from .runtime import DeviceBuffer, ptr, stream_handle, to_bf16, to_device, to_device_raw

MODES = {"auto": 0, "prefill": 1, "decode": 2}
SCORING = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}
# stage order of the optional per-stage events (include/sllm_moe.h)
STAGES = ("router_gemm", "route", "permute", "act_quant", "expert_up",
          "expert_down", "shared_up", "shared_down", "combine")


def _event_array(events):
    """ctypes void*[2 * len(STAGES)] from a list of runtime.Event (or None)."""
    if events is None:
        return None
    if len(events) != 2 * len(STAGES):
        raise ValueError(f"need {2 * len(STAGES)} events")
    import ctypes
    arr = (ctypes.c_void_p * len(events))(*[e._ev for e in events])
    return arr


def _mode(m) -> int:
    return MODES[m] if isinstance(m, str) else int(m)


# ---------------------------------------------------------------------------
# Qwen-style layer
# ---------------------------------------------------------------------------

def _qwen_args(T, H, E, I, Is, topk, mode, out_f32, wdtype, eps, x, logits,
               weights, out, debug, workspace, workspace_bytes, stream):
    a = _lib.QwenArgs()
    a.T, a.H, a.E, a.I, a.Is, a.topk = T, H, E, I, Is, topk
    a.mode = _mode(mode)
    a.out_f32 = int(bool(out_f32))
    a.logits_given = int(logits is not None)
    a.wdtype = int(wdtype)
    a.renorm_eps = float(eps)
    a.x = ptr(x)
    a.logits = ptr(logits)
    w = weights
    a.router_w = ptr(w.get("router_w"))
    a.router_bias = ptr(w.get("router_bias"))
    for k in ("wg", "wg_s", "wu", "wu_s", "wd", "wd_s", "sg", "sg_s", "su",
              "su_s", "sd", "sd_s", "sgl", "wgu_packed", "wd_packed",
              "sgu_packed", "sd_packed"):
        setattr(a, k, ptr(w.get(k)))
    a.out = ptr(out)
    debug = debug or {}
    for k in ("logits_out", "w_out", "ids_out", "counts_out", "sorted_out",
              "inv_pos_out"):
        setattr(a, k, ptr(debug.get(k)))
    a.workspace = ptr(workspace)
    a.workspace_bytes = int(workspace_bytes or 0)
    a.stream = stream_handle(stream)
    return a


def qwen_workspace_bytes(T, H, E, I, Is, topk, mode="auto", has_shared=True,
                         logits_given=False, wdtype=0) -> int:
    """Workspace size for one qwen_forward_dev call of these shapes."""
    w = {"su": 1} if has_shared else {}
    a = _qwen_args(T, H, E, I, Is, topk, mode, False, wdtype, 1e-20, None,
                   1 if logits_given else None, w, None, None, None, 0, None)
    n = _lib.lib().sllm_moe_qwen_workspace_bytes(a)
    if n < 0:
        raise RuntimeError(_lib.last_error())
    return int(n)


def stream_status(stream=None) -> None:
    """Raises RuntimeError (rc -2) if a streamed expert GEMM left work items
    undone since the last check (synchronizes ``stream``)."""
    _lib.check(_lib.lib().sllm_moe_stream_status(stream_handle(stream)),
               "sllm_moe_stream_status")


def qwen_forward_dev(x, out, weights: dict, *, T, H, E, I, topk, Is=0,
                     mode="auto", out_f32=False, wdtype=0, eps=1e-20,
                     logits=None, workspace=None, workspace_bytes=None,
                     stream=None, debug=None, stage_events=None) -> None:
    """One Qwen-style MoE layer on device buffers (see include/sllm_moe.h
    sllm_moe_qwen_args for shapes). `weights` maps router_w, wg, wg_s, wu,
    wu_s, wd, wd_s [, sg, sg_s, su, su_s, sd, sd_s, sgl] to device buffers;
    `debug` may map logits_out / w_out / ids_out / counts_out / sorted_out /
    inv_pos_out."""
    if workspace_bytes is None:
        workspace_bytes = getattr(workspace, "nbytes", None)
        if workspace_bytes is None and hasattr(workspace, "numel"):
            workspace_bytes = workspace.numel() * workspace.element_size()
    a = _qwen_args(T, H, E, I, Is, topk, mode, out_f32, wdtype, eps, x, logits,
                   weights, out, debug, workspace, workspace_bytes, stream)
    evs = _event_array(stage_events)
    if evs is not None:
        import ctypes
        a.stage_events = ctypes.cast(evs, ctypes.c_void_p)
    _lib.check(_lib.lib().sllm_moe_qwen_forward(a), "sllm_moe_qwen_forward")


def qwen_forward_noalloc(x, out, weights: dict, *, T, H, E, I, topk, Is=0,
                         mode="auto", out_f32=False, wdtype=0, eps=1e-20,
                         logits=None, stream=None, debug=None) -> None:
    """qwen_forward_dev on the library's per-device scratch instead of a
    workspace (sllm_moe_qwen_forward_noalloc: no device allocation; calls
    whose workspace exceeds noalloc_max_bytes() raise with rc -2; calls that
    overlap on one device race on the scratch)."""
    a = _qwen_args(T, H, E, I, Is, topk, mode, out_f32, wdtype, eps, x, logits,
                   weights, out, debug, None, 0, stream)
    _lib.check(_lib.lib().sllm_moe_qwen_forward_noalloc(a),
               "sllm_moe_qwen_forward_noalloc")


def noalloc_max_bytes() -> int:
    """Size of the per-device scratch of qwen_forward_noalloc."""
    return int(_lib.lib().sllm_moe_qwen_forward_noalloc_max_bytes())


def _graph_free(h):
    try:
        _lib.lib().sllm_moe_graph_free(c_void_p(h))
    except Exception:
        pass


class LayerGraph:
    """One qwen_forward_dev call captured as a HIP graph
    (sllm_moe_qwen_graph_new). `launch()` replays it on the current contents
    of the buffers it was captured with; the graph keeps references to them.
    For decode batches a replay costs one launch instead of the layer's
    kernel launches and their gaps."""

    def __init__(self, x, out, weights: dict, *, T, H, E, I, topk, Is=0,
                 mode="auto", out_f32=False, wdtype=0, eps=1e-20, logits=None,
                 workspace=None, workspace_bytes=None, debug=None):
        if workspace_bytes is None:
            workspace_bytes = getattr(workspace, "nbytes", None)
            if workspace_bytes is None and hasattr(workspace, "numel"):
                workspace_bytes = workspace.numel() * workspace.element_size()
        a = _qwen_args(T, H, E, I, Is, topk, mode, out_f32, wdtype, eps, x,
                       logits, weights, out, debug, workspace, workspace_bytes,
                       None)
        h = _lib.lib().sllm_moe_qwen_graph_new(a)
        if not h:
            raise RuntimeError("sllm_moe_qwen_graph_new: " + _lib.last_error())
        self._keep = (x, out, weights, logits, workspace, debug)
        self._h = h
        self._fin = weakref.finalize(self, _graph_free, h)

    def launch(self, stream=None) -> None:
        if not self._fin.alive:
            raise RuntimeError("LayerGraph: launch after free")
        _lib.check(_lib.lib().sllm_moe_graph_launch(c_void_p(self._h),
                                                    stream_handle(stream)),
                   "sllm_moe_graph_launch")

    def free(self) -> None:
        """Destroys the graph (work already launched is unaffected)."""
        self._fin()
        self._keep = None


# ---------------------------------------------------------------------------
# DeepSeek-style layer
# ---------------------------------------------------------------------------

def _ds_args(T, H, E, I, Is, topk, mode, out_f32, n_group, topk_group,
             scoring, route_scale, swiglu_limit, x, logits, weights, out,
             debug, workspace, workspace_bytes, stream, token_ids=None,
             vocab=0):
    a = _lib.DeepseekArgs()
    a.T, a.H, a.E, a.I, a.Is, a.topk = T, H, E, I, Is, topk
    a.mode = _mode(mode)
    a.out_f32 = int(bool(out_f32))
    a.logits_given = int(logits is not None)
    a.n_group, a.topk_group = int(n_group), int(topk_group)
    a.scoring = SCORING[scoring] if isinstance(scoring, str) else int(scoring)
    a.route_scale = float(route_scale)
    a.swiglu_limit = float(swiglu_limit)
    a.x = ptr(x)
    a.logits = ptr(logits)
    w = weights
    for k in ("router_w", "bias", "w1", "w1_s", "w3", "w3_s", "w2", "w2_s",
              "s1", "s1_s", "s3", "s3_s", "s2", "s2_s", "w13_packed",
              "w13_s_packed", "w2_packed", "w2_s_packed", "s13_packed",
              "s2_packed"):
        setattr(a, k, ptr(w.get(k)))
    a.out = ptr(out)
    debug = debug or {}
    for k in ("logits_out", "w_out", "ids_out", "counts_out", "sorted_out",
              "inv_pos_out"):
        setattr(a, k, ptr(debug.get(k)))
    a.workspace = ptr(workspace)
    a.workspace_bytes = int(workspace_bytes or 0)
    a.stream = stream_handle(stream)
    # hash layers: weights["tid2eid"] (vocab, topk) int32 + per-call token ids
    a.tid2eid = ptr(w.get("tid2eid"))
    a.token_ids = ptr(token_ids)
    a.vocab = int(vocab)
    return a


def deepseek_workspace_bytes(T, H, E, I, Is, topk, mode="auto",
                             has_shared=True, logits_given=False) -> int:
    w = {"s1": 1} if has_shared else {}
    a = _ds_args(T, H, E, I, Is, topk, mode, False, 1, 1, 1, 1.0, 0.0, None,
                 1 if logits_given else None, w, None, None, None, 0, None)
    n = _lib.lib().sllm_moe_ds_workspace_bytes(a)
    if n < 0:
        raise RuntimeError(_lib.last_error())
    return int(n)


def deepseek_forward_dev(x, out, weights: dict, *, T, H, E, I, topk, Is=0,
                         mode="auto", out_f32=False, n_group=1, topk_group=1,
                         scoring="sigmoid", route_scale=1.0, swiglu_limit=0.0,
                         logits=None, workspace=None, workspace_bytes=None,
                         stream=None, debug=None, stage_events=None,
                         token_ids=None, vocab=0) -> None:
    """One DeepSeek-style MoE layer on device buffers (shapes in
    include/sllm_moe.h sllm_moe_ds_args). `weights` maps router_w, bias, w1,
    w1_s, w3, w3_s, w2, w2_s [, s1, s1_s, s3, s3_s, s2, s2_s] [, tid2eid];
    a hash layer (weights["tid2eid"], vocab rows) also takes the tokens' ids
    `token_ids` (T int32 device buffer)."""
    if workspace_bytes is None:
        workspace_bytes = getattr(workspace, "nbytes", None)
        if workspace_bytes is None and hasattr(workspace, "numel"):
            workspace_bytes = workspace.numel() * workspace.element_size()
    if weights.get("tid2eid") is not None and token_ids is None:
        raise ValueError("a hash layer needs token_ids")
    a = _ds_args(T, H, E, I, Is, topk, mode, out_f32, n_group, topk_group,
                 scoring, route_scale, swiglu_limit, x, logits, weights, out,
                 debug, workspace, workspace_bytes, stream, token_ids, vocab)
    evs = _event_array(stage_events)
    if evs is not None:
        import ctypes
        a.stage_events = ctypes.cast(evs, ctypes.c_void_p)
    _lib.check(_lib.lib().sllm_moe_ds_forward(a), "sllm_moe_ds_forward")


# ---------------------------------------------------------------------------
# weight packing (streaming layout of the prefill GEMMs)
# ---------------------------------------------------------------------------

def pack_weights(fp4, up, w0, w1, E, N, K, s0=None, s1=None, stream=None):
    """Repack device weights into the streaming layout; returns
    (packed DeviceBuffer, packed-scales DeviceBuffer or None)."""
    L = _lib.lib()
    nb = L.sllm_moe_packed_bytes(int(fp4), int(up), E, N, K)
    if nb < 0:
        raise RuntimeError(_lib.last_error())
    out = DeviceBuffer(int(nb))
    outs = None
    if fp4:
        ns = L.sllm_moe_packed_scale_bytes(int(up), E, N, K)
        outs = DeviceBuffer(int(ns))
    _lib.check(L.sllm_moe_pack_weights(int(fp4), int(up), ptr(w0), ptr(w1),
                                       ptr(s0), ptr(s1), E, N, K, ptr(out),
                                       ptr(outs), stream_handle(stream)),
               "sllm_moe_pack_weights")
    return out, outs


# ---------------------------------------------------------------------------
# device-resident layers with numpy in / out
# ---------------------------------------------------------------------------

def _up(arr, raw=True):
    if arr is None:
        return None
    return to_device_raw(np.ascontiguousarray(arr)) if raw else to_device(arr)


@dataclass
class _Resident:
    bufs: dict = field(default_factory=dict)

    def get(self, k):
        return self.bufs.get(k)


# Granularity of the fused layer's shapes (sllm_moe_qwen_forward): hidden a
# multiple of 256 (the down projection's column slabs), intermediates of
# 128 (the gate/up slabs and the 128-wide K steps).
H_ALIGN, I_ALIGN = 256, 128


def _round_up(n: int, m: int) -> int:
    return -(-int(n) // m) * m


def _bias_buffer(bias, E):
    if bias is None:
        return None
    b = np.ascontiguousarray(bias, np.float32).reshape(-1)
    if b.size != E:
        raise ValueError(f"router_bias must hold E={E} values, got {b.size}")
    return _up(b)


def _pad_to(a, shape, fill=0):
    """a zero-padded (or `fill`-padded) at the end of each axis to `shape`."""
    a = np.asarray(a)
    if tuple(a.shape) == tuple(shape):
        return a
    out = np.full(shape, fill, a.dtype)
    out[tuple(slice(0, n) for n in a.shape)] = a
    return out


class QwenMoE:
    """Qwen-style layer with device-resident weights.

    FP8 weights: e4m3 codes (uint8) with fp32 block scales, reference
    orientation (out, in): wg/wu (E, I, H), wd (E, H, I), scales
    (E, ceil(out/128), ceil(in/128)); shared sg/su (Is, H), sd (H, Is).
    bf16 weights (wdtype=1): float arrays (rounded to bf16), no scales.
    router_w (E, H) and sgl (1, H) are rounded to bf16. router_bias (E,)
    fp32, optional: a per-expert bias added to the router logits before the
    softmax top-k (the skewed-load configuration's routing bias).

    Shapes whose hidden size is not a multiple of 256, or whose
    intermediate sizes are not multiples of 128 (the reference's tiny dev
    model: hidden 16, intermediate 8), are zero-padded up to them once, at
    upload: padded columns of x and of the weights add exact zeros to every
    dot product (the router's logits, the shared gate), padded intermediate
    columns give gate = up = 0 and so h = silu(0) * 0 = 0, and padded output
    columns are dropped. FP8 codes pad with code 0 (+0.0) and their block
    scales with 1.0, which multiplies only those zero codes; the per-1x128
    activation quantization of prefill sees the same maximum in every block
    that holds real values. Outputs equal those of the unpadded arithmetic.
    """

    def __init__(self, router_w, wg, wu, wd, wg_s=None, wu_s=None, wd_s=None,
                 sg=None, su=None, sd=None, sg_s=None, su_s=None, sd_s=None,
                 sgl=None, top_k=8, eps=1e-20, packed=True, router_bias=None):
        wdtype = 0 if wg_s is not None else 1
        E, I, H = np.asarray(wg).shape
        Is = 0 if su is None else np.asarray(su).shape[0]
        Hp, Ip = _round_up(H, H_ALIGN), _round_up(I, I_ALIGN)
        Isp = _round_up(Is, I_ALIGN)
        self.wdtype = wdtype
        if self.wdtype == 0:
            def cast(a, shape):
                return _pad_to(np.ascontiguousarray(a, np.uint8), shape)
        else:
            def cast(a, shape):
                return _pad_to(to_bf16(a), shape)

        def scales(a, n, k):
            return _pad_to(np.asarray(a, np.float32),
                           (*np.shape(a)[:-2], -(-n // 128), -(-k // 128)), 1.0)
        b = {"router_w": _up(_pad_to(to_bf16(router_w), (E, Hp))),
             "router_bias": _bias_buffer(router_bias, E),
             "wg": _up(cast(wg, (E, Ip, Hp))), "wu": _up(cast(wu, (E, Ip, Hp))),
             "wd": _up(cast(wd, (E, Hp, Ip)))}
        if self.wdtype == 0:
            b.update(wg_s=_up(scales(wg_s, Ip, Hp)),
                     wu_s=_up(scales(wu_s, Ip, Hp)),
                     wd_s=_up(scales(wd_s, Hp, Ip)))
        if su is not None:
            b.update(sg=_up(cast(sg, (Isp, Hp))), su=_up(cast(su, (Isp, Hp))),
                     sd=_up(cast(sd, (Hp, Isp))),
                     sgl=_up(_pad_to(to_bf16(np.asarray(sgl).reshape(-1)), (Hp,))))
            if self.wdtype == 0:
                b.update(sg_s=_up(scales(sg_s, Isp, Hp)),
                         su_s=_up(scales(su_s, Isp, Hp)),
                         sd_s=_up(scales(sd_s, Hp, Isp)))
        self._finish(b, E, Ip, Hp, Isp, top_k, eps, wdtype, packed)
        self.H_in = int(H)

    @classmethod
    def from_device(cls, bufs, *, E, I, H, Is, top_k=8, eps=1e-20, packed=True):
        """FP8 weights already resident on the device (for example from
        sllm_amd.loader): the buffers of __init__'s layout -- router_w (bf16
        bits), wg/wu/wd e4m3 codes with fp32 wg_s/wu_s/wd_s block scales,
        optional shared sg/su/sd (+ scales) and sgl. Streaming-layout
        buffers already in `bufs` (wgu_packed, wd_packed, sgu_packed,
        sd_packed) are used as they are instead of packed again."""
        self = cls.__new__(cls)
        self._finish(dict(bufs), E, I, H, Is, top_k, eps, 0, packed)
        return self

    def _finish(self, b, E, I, H, Is, top_k, eps, wdtype, packed):
        self.wdtype = wdtype
        self.E, self.I, self.H, self.Is = int(E), int(I), int(H), int(Is)
        self.H_in = self.H  # the caller's hidden size (H when not padded)
        self.top_k = int(top_k)
        self.eps = float(eps)
        if packed and wdtype == 0 and "wgu_packed" not in b:
            b["wgu_packed"], _ = pack_weights(0, 1, b["wg"], b["wu"], E, I, H)
            b["wd_packed"], _ = pack_weights(0, 0, b["wd"], None, E, H, I)
            if Is:
                b["sgu_packed"], _ = pack_weights(0, 1, b["sg"], b["su"], 1, Is, H)
                b["sd_packed"], _ = pack_weights(0, 0, b["sd"], None, 1, H, Is)
        self._w = b
        self._ws = None

    def _workspace(self, T, mode, logits_given):
        n = qwen_workspace_bytes(T, self.H, self.E, self.I, self.Is, self.top_k,
                                 mode, self.Is > 0, logits_given, self.wdtype)
        if self._ws is None or self._ws.nbytes < n:
            self._ws = DeviceBuffer(n)
        return self._ws

    def forward(self, x, logits=None, mode="auto", return_routing=False):
        """x (T, H) float (rounded to bf16) -> out (T, H) float32."""
        x = np.asarray(x, np.float32)
        if x.ndim != 2 or x.shape[1] != self.H_in:
            raise ValueError(f"x must be (T, {self.H_in}), got {x.shape}")
        T = x.shape[0]
        xb = _up(_pad_to(to_bf16(x), (T, self.H)))
        lg = _up(np.asarray(logits, np.float32)) if logits is not None else None
        out = DeviceBuffer(T * self.H * 4)
        dbg = {}
        if return_routing:
            dbg = {"logits_out": DeviceBuffer(T * self.E * 4),
                   "w_out": DeviceBuffer(T * self.top_k * 4),
                   "ids_out": DeviceBuffer(T * self.top_k * 4),
                   "counts_out": DeviceBuffer(self.E * 4)}
        ws = self._workspace(T, mode, logits is not None)
        qwen_forward_dev(xb, out, self._w, T=T, H=self.H, E=self.E, I=self.I,
                         Is=self.Is, topk=self.top_k, mode=mode, out_f32=True,
                         wdtype=self.wdtype, eps=self.eps, logits=lg,
                         workspace=ws, debug=dbg)
        y = out.copy_host().reshape(T, self.H)[:, :self.H_in]
        stream_status()
        if not return_routing:
            return np.ascontiguousarray(y)
        r = {"logits": dbg["logits_out"].copy_host().reshape(T, self.E),
             "w": dbg["w_out"].copy_host().reshape(T, self.top_k),
             "ids": dbg["ids_out"].copy_host_raw(np.int32, (T, self.top_k)),
             "counts": dbg["counts_out"].copy_host_raw(np.int32, (self.E,))}
        return np.ascontiguousarray(y), r


def check_tid2eid(table, E: int, top_k: int) -> np.ndarray:
    """A hash layer's expert table as (vocab, top_k) int32, every entry an
    expert id in [0, E). The reference's take_along_axis
    (ref/deepseek_v4.py:558) raises IndexError for ids >= E; the kernels
    would drop such slots from the output, so they are refused here."""
    t = np.asarray(table)
    if t.ndim != 2 or t.shape[1] != top_k or t.shape[0] < 1:
        raise ValueError(f"tid2eid must be (vocab >= 1, top_k={top_k}), got {t.shape}")
    if not np.issubdtype(t.dtype, np.integer):
        raise TypeError(f"tid2eid must hold integer expert ids, got {t.dtype}")
    bad = (t < 0) | (t >= E)
    if bad.any():
        r, c = np.argwhere(bad)[0]
        raise IndexError(f"tid2eid[{r}, {c}] = {t[r, c]} is not an expert id in [0, {E})")
    return np.ascontiguousarray(t, np.int32)


class DeepseekMoE:
    """DeepSeek-style layer with device-resident weights: routed MXFP4
    (w1/w3 (E, I, H/2) packed + (E, I, H/32) e8m0; w2 (E, H, I/2) + (E, H,
    I/32)), optional FP8 shared expert with power-of-two fp32 block scales."""

    def __init__(self, router_w, bias, w1, w1_s, w3, w3_s, w2, w2_s, s1=None,
                 s1_s=None, s3=None, s3_s=None, s2=None, s2_s=None, top_k=8,
                 n_group=1, topk_group=1, scoring="sigmoid", route_scale=1.0,
                 swiglu_limit=0.0, packed=True, tid2eid=None):
        E, I = np.asarray(w1).shape[:2]
        H = np.asarray(w2).shape[1]
        Is = 0 if s1 is None else np.asarray(s1).shape[0]
        if tid2eid is not None:  # before any upload
            tid2eid = check_tid2eid(tid2eid, E, top_k)
        b = {"router_w": _up(to_bf16(router_w)),
             "bias": _up(np.asarray(bias, np.float32)) if bias is not None else None}
        for k, v in (("w1", w1), ("w1_s", w1_s), ("w3", w3), ("w3_s", w3_s),
                     ("w2", w2), ("w2_s", w2_s)):
            b[k] = _up(np.ascontiguousarray(v, np.uint8))
        if s1 is not None:
            for k, v in (("s1", s1), ("s3", s3), ("s2", s2)):
                b[k] = _up(np.ascontiguousarray(v, np.uint8))
            for k, v in (("s1_s", s1_s), ("s3_s", s3_s), ("s2_s", s2_s)):
                b[k] = _up(np.asarray(v, np.float32))
        self._finish(b, E, I, H, Is, top_k, n_group, topk_group, scoring,
                     route_scale, swiglu_limit, packed, tid2eid)

    @classmethod
    def from_device(cls, bufs, *, E, I, H, Is, top_k=8, n_group=1,
                    topk_group=1, scoring="sigmoid", route_scale=1.0,
                    swiglu_limit=0.0, packed=True, tid2eid=None):
        """Weights already resident on the device (for example from
        sllm_amd.loader): the buffers of __init__'s layout -- router_w (bf16
        bits), bias (fp32 or None), packed e2m1 w1/w3/w2 with raw e8m0
        w1_s/w3_s/w2_s, optional shared s1/s3/s2 e4m3 with fp32 scales."""
        self = cls.__new__(cls)
        self._finish(dict(bufs), E, I, H, Is, top_k, n_group, topk_group,
                     scoring, route_scale, swiglu_limit, packed, tid2eid)
        return self

    def _finish(self, b, E, I, H, Is, top_k, n_group, topk_group, scoring,
                route_scale, swiglu_limit, packed, tid2eid):
        self.E, self.I, self.H, self.Is = int(E), int(I), int(H), int(Is)
        self.top_k, self.n_group, self.topk_group = int(top_k), int(n_group), int(topk_group)
        self.scoring, self.route_scale = scoring, float(route_scale)
        self.swiglu_limit = float(swiglu_limit)
        if packed:
            b["w13_packed"], b["w13_s_packed"] = pack_weights(
                1, 1, b["w1"], b["w3"], E, I, H, b["w1_s"], b["w3_s"])
            b["w2_packed"], b["w2_s_packed"] = pack_weights(
                1, 0, b["w2"], None, E, H, I, b["w2_s"])
            if Is:
                b["s13_packed"], _ = pack_weights(0, 1, b["s1"], b["s3"], 1, Is, H)
                b["s2_packed"], _ = pack_weights(0, 0, b["s2"], None, 1, H, Is)
        # hash layer (ref/deepseek_v4.py:545-552): experts from the token-id
        # table instead of the biased top-k
        self.vocab = 0
        if tid2eid is not None:
            t = np.ascontiguousarray(tid2eid, np.int32)
            check_tid2eid(t, self.E, self.top_k)
            self.vocab = t.shape[0]
            b["tid2eid"] = _up(t)
        self._w = b
        self._ws = None

    def forward(self, x, logits=None, mode="auto", return_routing=False,
                token_ids=None):
        x = np.asarray(x, np.float32)
        T = x.shape[0]
        tok = None
        if self.vocab:
            if token_ids is None:
                raise ValueError("a hash layer needs token_ids")
            tok = _up(np.asarray(token_ids).reshape(T).astype(np.int32))
        n = deepseek_workspace_bytes(T, self.H, self.E, self.I, self.Is,
                                     self.top_k, mode, self.Is > 0,
                                     logits is not None)
        if self._ws is None or self._ws.nbytes < n:
            self._ws = DeviceBuffer(n)
        xb = _up(to_bf16(x))
        lg = _up(np.asarray(logits, np.float32)) if logits is not None else None
        out = DeviceBuffer(T * self.H * 4)
        dbg = {}
        if return_routing:
            dbg = {"logits_out": DeviceBuffer(T * self.E * 4),
                   "w_out": DeviceBuffer(T * self.top_k * 4),
                   "ids_out": DeviceBuffer(T * self.top_k * 4),
                   "counts_out": DeviceBuffer(self.E * 4)}
        deepseek_forward_dev(xb, out, self._w, T=T, H=self.H, E=self.E,
                             I=self.I, Is=self.Is, topk=self.top_k, mode=mode,
                             out_f32=True, n_group=self.n_group,
                             topk_group=self.topk_group, scoring=self.scoring,
                             route_scale=self.route_scale,
                             swiglu_limit=self.swiglu_limit, logits=lg,
                             workspace=self._ws, debug=dbg, token_ids=tok,
                             vocab=self.vocab)
        y = out.copy_host().reshape(T, self.H)
        stream_status()
        if not return_routing:
            return y
        r = {"logits": dbg["logits_out"].copy_host().reshape(T, self.E),
             "w": dbg["w_out"].copy_host().reshape(T, self.top_k),
             "ids": dbg["ids_out"].copy_host_raw(np.int32, (T, self.top_k)),
             "counts": dbg["counts_out"].copy_host_raw(np.int32, (self.E,))}
        return y, r


# Device layers of moe_block_forward, most recently used last. An entry is
# reused when the call passes the same router weight object (the caller's
# checkpoint tensor: ref/qwen4_exp_pipeline.py:262-275 stacks the experts
# anew on every call but passes the router tensor as stored) and weights
# whose shapes, dtypes and strided samples match; it is dropped when that
# router object is freed, or as the least recently used past BLOCK_CACHE_MAX.
BLOCK_CACHE_MAX = 64
_block_cache: "dict[tuple, tuple]" = {}


def _sample_key(a):
    if a is None:
        return None
    a = np.asarray(a)
    flat = a.reshape(-1)
    step = max(1, flat.size // 4096)
    return (a.shape, a.dtype.str,
            hash(np.ascontiguousarray(flat[::step][:4096]).tobytes()))


def clear_block_cache() -> None:
    """Frees every device layer moe_block_forward holds (call after editing
    a weight array in place: such edits are not detected)."""
    _block_cache.clear()


def moe_block_forward(x, router_w, expert_gate, expert_up, expert_down,
                      shared_gate_w, shared_gate_linear_w, shared_up_w,
                      shared_down_w, top_k, eps=1e-20):
    """Device twin of ref/qwen4_exp.py:153-184 moe_block_forward with the
    same signature: weights are float arrays used at bf16 precision (the
    bf16 GEMV path, fp32 activations). Returns (n, H) float32.

    The device layer (weights uploaded once) is kept between calls with the
    same weights (see BLOCK_CACHE_MAX); any hidden and intermediate sizes
    are accepted (QwenMoE pads them exactly)."""
    has_sh = shared_up_w is not None
    key = (id(router_w), int(top_k), float(eps), _sample_key(router_w),
           _sample_key(expert_gate), _sample_key(expert_up),
           _sample_key(expert_down),
           *((_sample_key(shared_gate_w), _sample_key(shared_gate_linear_w),
              _sample_key(shared_up_w), _sample_key(shared_down_w))
             if has_sh else ()))
    hit = _block_cache.pop(key, None)
    if hit is not None and hit[0]() is not router_w:
        hit = None  # the router object died and its id was reused
    if hit is None:
        layer = QwenMoE(router_w, expert_gate, expert_up, expert_down,
                        sg=shared_gate_w if has_sh else None,
                        su=shared_up_w, sd=shared_down_w,
                        sgl=shared_gate_linear_w if has_sh else None,
                        top_k=top_k, eps=eps)
        try:
            ref = weakref.ref(router_w, lambda _r, k=key: _block_cache.pop(k, None))
        except TypeError:  # not weak-referenceable: used for this call only
            return layer.forward(x)
        hit = (ref, layer)
    _block_cache[key] = hit
    while len(_block_cache) > BLOCK_CACHE_MAX:
        _block_cache.pop(next(iter(_block_cache)))
    return hit[1].forward(x)
