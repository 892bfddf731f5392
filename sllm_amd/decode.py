"""Drop-ins for the MLP blocks of the reference's device decode loops.

`kernels/q4_device_decode.Q4DeviceDecodeState._moe(x, i)` (:316-339)
computes a token's MoE block from host-side routing: the router GEMM on the
device, qe.moe_route on the host, then 3 k + 5 device GEMVs, each a host
round trip. `DeviceMoEStack.moe(x, i)` has the same contract -- x (n, H)
float in, (n, H) float32 out -- and runs layer i as one stream-ordered call
of the fused MoE layer (router, routing, permutation, expert and shared
GEMVs, combine; all on the device, one upload and one download).

`kernels/hybrid_device_decode.py:308-311` runs the hybrid family's dense
MLP as three GEMMs with a host SwiGLU between them. `DenseSwiGLU` computes
down(silu(gate x) * up x) as the same fused layer with one expert and top-1
routing on zero logits: softmax over one logit is exactly 1 and the
renormalisation 1 / (1 + 1e-20) rounds to 1 in fp32, so every route weight
is exactly 1; the layer recognises this case and runs only the expert
launches (gate/up, down, slice sum) over the rows in token order.

Both keep their staging buffers, workspace and argument blocks between
calls, so a decode step allocates nothing after its first call at a given
batch size. With graphs=True the host-array calls capture each (layer,
batch size) layer call as a HIP graph on first use and replay it after
that; on ROCm 7.2 a replay of the layer's 5-6 launches measured slower than
issuing them (B=1 hook call 67 vs 59 us), so launches are the default.
`moe_dev` / `forward_dev` take device buffers for callers that keep the
hidden state on the device.

Weights come from the reference's float weight dict (the names of
Q4DeviceWeightTable, q4_device_decode.py:112-122, and of the hybrid table's
`{p}.mlp.{gate,up,down}_proj`), used at bf16 precision like that table's
bf16 upload, or from an FP8 checkpoint through sllm_amd.loader, kept in the
stored e4m3 + 128x128 block-scale format.
"""

from __future__ import annotations

from ctypes import c_float, c_void_p

import numpy as np

from . import _lib
from .moe import QwenMoE, _graph_free, _qwen_args, qwen_workspace_bytes
from .runtime import DeviceBuffer, memset, ptr, stream_handle, sync

TEXT_PREFIX = "model.language_model"


class _Pinned:
    """Page-locked host staging (sllm_host_new)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = _lib.lib().sllm_host_new(self.nbytes)
        if not self.ptr:
            raise RuntimeError("sllm_host_new failed: " + _lib.last_error())

    def __del__(self):
        try:
            if self.ptr:
                _lib.lib().sllm_host_free(c_void_p(self.ptr))
                self.ptr = None
        except Exception:
            pass


class _Graph:
    """Owner of one captured layer call (sllm_moe_qwen_graph_new)."""

    def __init__(self, a):
        h = _lib.lib().sllm_moe_qwen_graph_new(a)
        if not h:
            raise RuntimeError("sllm_moe_qwen_graph_new: " + _lib.last_error())
        self.h = h

    def launch(self):
        _lib.check(_lib.lib().sllm_moe_graph_launch(c_void_p(self.h), None),
                   "sllm_moe_graph_launch")

    def __del__(self):
        if getattr(self, "h", None):
            _graph_free(self.h)
            self.h = None


class _Runner:
    """Calls the fused layer for a QwenMoE at decode sizes, reusing the
    device input staging, the output buffer, the workspace, the argument
    block of each (layer, n) and page-locked host staging: a host call is
    one host bf16 rounding, an upload, the layer (a graph replay when
    `graphs`) and a download, ordered on one stream with one wait."""

    def __init__(self, graphs: bool = False):
        self._x = self._out = self._ws = self._zl = None
        self._hx = self._hy = None
        self._args = {}
        self._graphs = {}
        self.graphs = graphs

    def _pin(self, name, nbytes):
        b = getattr(self, name)
        if b is None or b.nbytes < nbytes:
            b = _Pinned(max(int(nbytes), 64))
            setattr(self, name, b)
        return b

    def _grow(self, name, nbytes):
        b = getattr(self, name)
        if b is None or b.nbytes < nbytes:
            self._graphs.clear()  # graphs and argument blocks hold old pointers
            self._args.clear()
            b = DeviceBuffer(max(int(nbytes), 4))
            setattr(self, name, b)
        return b

    def args(self, layer: QwenMoE, n: int, zero_logits: bool, x=None, out=None,
             out_f32=True, stream=None):
        """The argument block for layer at n tokens; x / out default to the
        runner's own staging buffers."""
        own = x is None
        key = (id(layer), n, own, zero_logits, out_f32)
        a = self._args.get(key)
        if a is None:
            if own:
                self._grow("_x", n * layer.H * 2)
                self._grow("_out", n * layer.H * 4)
            if zero_logits and (self._zl is None or self._zl.nbytes < n * layer.E * 4):
                self._grow("_zl", n * layer.E * 4)
                memset(self._zl, 0, self._zl.nbytes)
                sync()  # ordered before calls on any stream
            self._grow("_ws", qwen_workspace_bytes(
                n, layer.H, layer.E, layer.I, layer.Is, layer.top_k, "decode",
                layer.Is > 0, zero_logits, layer.wdtype))
            a = _qwen_args(n, layer.H, layer.E, layer.I, layer.Is, layer.top_k,
                           "decode", out_f32, layer.wdtype, layer.eps,
                           self._x if own else None,
                           self._zl if zero_logits else None, layer._w,
                           self._out if own else None, None, self._ws,
                           self._ws.nbytes, None)
            a._keep = layer  # the key holds the layer's id: keep it alive
            self._args[key] = a
        if not own:
            a.x, a.out = ptr(x), ptr(out)
            a.stream = stream_handle(stream)
        return a

    def run_host(self, layer: QwenMoE, x, zero_logits=False) -> np.ndarray:
        x = np.asarray(x, np.float32)
        if x.ndim != 2 or x.shape[1] != layer.H:
            raise ValueError(f"x must be (n, {layer.H}), got {x.shape}")
        n, cnt = x.shape[0], x.size
        x = np.ascontiguousarray(x)
        a = self.args(layer, n, zero_logits)
        hx, hy = self._pin("_hx", cnt * 2), self._pin("_hy", cnt * 4)
        L = _lib.lib()
        _lib.check(L.sllm_host_f32_to_bf16(c_void_p(hx.ptr), x.ctypes.data_as(c_void_p),
                                           cnt), "sllm_host_f32_to_bf16")
        _lib.check(L.sllm_copy_async(c_void_p(self._x.ptr), c_void_p(hx.ptr),
                                     cnt * 2, None), "sllm_copy_async")
        if self.graphs:
            key = (id(layer), n, zero_logits)
            g = self._graphs.get(key)
            if g is None:
                g = self._graphs[key] = _Graph(a)
            g.launch()
        else:
            _lib.check(L.sllm_moe_qwen_forward(a), "sllm_moe_qwen_forward")
        _lib.check(L.sllm_copy_async(c_void_p(hy.ptr), c_void_p(self._out.ptr),
                                     cnt * 4, None), "sllm_copy_async")
        _lib.check(L.sllm_stream_sync(None), "sllm_stream_sync")
        return np.ctypeslib.as_array((c_float * cnt).from_address(hy.ptr)) \
            .reshape(n, layer.H).copy()

    def run_dev(self, layer: QwenMoE, x, out, n, zero_logits=False,
                out_f32=True, stream=None) -> None:
        a = self.args(layer, n, zero_logits, x=x, out=out, out_f32=out_f32,
                      stream=stream)
        _lib.check(_lib.lib().sllm_moe_qwen_forward(a), "sllm_moe_qwen_forward")


def _f32(a):
    return np.asarray(a, np.float32)


class DeviceMoEStack:
    """One fused device MoE layer per decoder layer, indexed like the
    reference's `_moe(x, i)`."""

    def __init__(self, layers, graphs: bool = False):
        self.layers = list(layers)
        self._run = _Runner(graphs)

    @classmethod
    def from_weights(cls, weights: dict, n_layers: int, top_k: int,
                     prefix: str = TEXT_PREFIX, eps: float = 1e-20):
        """From the reference's float weight dict (bf16 precision)."""
        out = []
        for i in range(n_layers):
            p = f"{prefix}.layers.{i}.mlp"
            E = 0
            while f"{p}.experts.{E}.gate_proj.weight" in weights:
                E += 1
            if E == 0:
                raise KeyError(f"no experts under {p}")

            def stack(m):
                return np.stack([_f32(weights[f"{p}.experts.{e}.{m}_proj.weight"])
                                 for e in range(E)])
            sp = f"{p}.shared_expert"
            sh = f"{sp}.gate_proj.weight" in weights
            shared = {}
            if sh:
                shared = dict(sg=_f32(weights[f"{sp}.gate_proj.weight"]),
                              su=_f32(weights[f"{sp}.up_proj.weight"]),
                              sd=_f32(weights[f"{sp}.down_proj.weight"]),
                              sgl=_f32(weights[f"{p}.shared_expert_gate.weight"]))
            out.append(QwenMoE(_f32(weights[f"{p}.gate.weight"]), stack("gate"),
                               stack("up"), stack("down"), top_k=top_k, eps=eps,
                               **shared))
        return cls(out)

    @classmethod
    def from_checkpoint(cls, ckpt, n_layers: int, top_k: int,
                        prefix: str = TEXT_PREFIX, eps: float = 1e-20):
        """From an FP8 checkpoint (sllm_amd.loader.Checkpoint)."""
        from .loader import load_qwen_moe
        return cls([load_qwen_moe(ckpt, f"{prefix}.layers.{i}.mlp", top_k, eps)
                    for i in range(n_layers)])

    def moe(self, x, i: int) -> np.ndarray:
        """Q4DeviceDecodeState._moe's contract: x (n, H) -> (n, H) float32."""
        return self._run.run_host(self.layers[i], x)

    def moe_dev(self, x, out, i: int, n: int, out_f32: bool = True,
                stream=None) -> None:
        """Layer i on device buffers: x bf16 (n, H), out (n, H) fp32 (or bf16
        when out_f32 is False), ordered on `stream`."""
        self._run.run_dev(self.layers[i], x, out, n, out_f32=out_f32,
                          stream=stream)


class DenseSwiGLU:
    """A dense SwiGLU MLP, down(silu(gate x) * up x), on the fused layer
    (one expert, top-1 on zero logits, no shared expert)."""

    def __init__(self, layer: QwenMoE, graphs: bool = False):
        if layer.E != 1 or layer.top_k != 1 or layer.Is:
            raise ValueError("DenseSwiGLU needs a one-expert, top-1 layer "
                             "without a shared expert")
        self.layer = layer
        self.H, self.I = layer.H, layer.I
        self._run = _Runner(graphs)

    @classmethod
    def from_arrays(cls, gate_w, up_w, down_w):
        """Float gate/up (I, H) and down (H, I), used at bf16 precision."""
        gate_w, up_w, down_w = _f32(gate_w), _f32(up_w), _f32(down_w)
        H = gate_w.shape[1]
        return cls(QwenMoE(np.zeros((1, H), np.float32), gate_w[None],
                           up_w[None], down_w[None], top_k=1))

    @classmethod
    def from_weights(cls, weights: dict, layer: int, prefix: str = TEXT_PREFIX):
        """Layer `layer`'s `{prefix}.layers.{layer}.mlp.*_proj.weight` from
        the reference's float weight dict."""
        p = f"{prefix}.layers.{layer}.mlp"
        return cls.from_arrays(weights[f"{p}.gate_proj.weight"],
                               weights[f"{p}.up_proj.weight"],
                               weights[f"{p}.down_proj.weight"])

    @classmethod
    def from_checkpoint(cls, ckpt, prefix: str):
        """FP8 gate/up/down_proj (+ weight_scale_inv) at `prefix`, for
        example "model.language_model.layers.0.mlp"."""
        from .loader import load_dense_mlp
        return cls(load_dense_mlp(ckpt, prefix))

    def __call__(self, x) -> np.ndarray:
        """x (n, H) -> (n, H) float32."""
        return self._run.run_host(self.layer, x, zero_logits=True)

    def forward_dev(self, x, out, n: int, out_f32: bool = True,
                    stream=None) -> None:
        self._run.run_dev(self.layer, x, out, n, zero_logits=True,
                          out_f32=out_f32, stream=stream)
