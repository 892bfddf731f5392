#!/usr/bin/env python3
"""Benchmark of the MI355X MoE layer on the BASELINE configs.

One "step" is one full Qwen-style FP8 MoE layer (router GEMM, softmax top-10,
permute, activation quant, grouped gate/up + SwiGLU + re-quant, grouped down,
shared expert with sigmoid gate, combine) over the C2 workload: 4096 tokens,
hidden 2048, 512 routed experts, top-10, intermediate 512, one shared expert
(intermediate 512). Inputs and weights are resident in HBM before the timed
region; weights are synthetic N(0, 0.02) quantized to e4m3 with fp32 128x128
block scales, activations bf16 N(0, 1).

Timing: HIP events on the stream the layer is launched on, K steps after W
warm-up steps, bracketed by device synchronisation. The default W (100) is
long enough for the GPU's clocks to settle after idle (~40 ms of
uninterrupted work), so the default K steps time the steady state of
back-to-back layer calls. Then, outside the headline
number: a per-stage event breakdown (the roofline of the dominant kernel),
the C3 decode batches (B = 1, 8, 32, 64; per-call events, L2/MALL flushed with
a 512 MiB fill between calls), and the CPU baseline (the numpy restatement of
the quantized layer on this host).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
Prints ONE JSON line. Other legs, each printing its own line instead:
--config c4 / c5 (the DeepSeek MXFP4 and skewed-routing prefill configs),
--device-decode (the decode drop-ins: the MoE hook with host arrays and a
dense SwiGLU MLP), --loader (FP8 checkpoint to device), --copy-calib MIB
(the byte-counter calibration copy).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = ("MoE layer tokens/s @4096-tok prefill; decode-layer µs @32 tok; "
          "% roofline")
PEAK_HBM_GBPS = 8000.0          # MI355X HBM3E
PEAK_FP8_TFLOPS = 5033.0        # MI355X dense FP8 MFMA (no sparsity)

C2 = dict(T=4096, H=2048, E=512, I=512, Is=512, k=10)
# DeepSeek-style MXFP4 prefill (routed e2m1 + e8m0/32, FP8 ue8m0-scaled shared
# expert, sigmoid scoring with selection bias, group-limited top-k)
C4 = dict(T=8192, H=7168, E=256, I=2048, Is=2048, k=8, n_group=8,
          topk_group=4, route_scale=2.5, swiglu_limit=10.0)
# C2 shapes at 16384 tokens with Zipf-skewed routing
C5 = dict(C2, T=16384)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# --------------------------------------------------------------------------
# synthetic C2 layer on the device
# --------------------------------------------------------------------------
class DeviceLayer:
    def __init__(self, cfg, seed=0):
        import numpy as np
        from sllm_amd import _lib
        from sllm_amd.runtime import (DeviceBuffer, fill_normal, sync, to_bf16,
                                      to_device_raw)
        self.cfg = cfg
        T, H, E, I, Is = cfg["T"], cfg["H"], cfg["E"], cfg["I"], cfg["Is"]
        L = _lib.lib()
        self.w = {}
        tmp = DeviceBuffer(max(E * I * H, Is * H) * 4)
        sub = [0]

        def q8(name, rows, cols):
            n = rows * cols
            fill_normal(tmp, n, seed * 1000 + sub[0], 0.02)
            sub[0] += 1
            q = DeviceBuffer(n)
            s = DeviceBuffer((rows // 128) * (cols // 128) * 4)
            _lib.check(L.sllm_quantize_weight_fp8(tmp.ptr, rows, cols, 0, q.ptr,
                                                  s.ptr, None), "quantize")
            self.w[name], self.w[name + "_s"] = q, s

        q8("wg", E * I, H)
        q8("wu", E * I, H)
        q8("wd", E * H, I)
        q8("sg", Is, H)
        q8("su", Is, H)
        q8("sd", H, Is)
        sync()
        tmp.free()
        # streaming layout of the prefill GEMMs (one-time repack)
        from sllm_amd.moe import pack_weights
        w = self.w
        w["wgu_packed"], _ = pack_weights(0, 1, w["wg"], w["wu"], E, I, H)
        w["wd_packed"], _ = pack_weights(0, 0, w["wd"], None, E, H, I)
        w["sgu_packed"], _ = pack_weights(0, 1, w["sg"], w["su"], 1, Is, H)
        w["sd_packed"], _ = pack_weights(0, 0, w["sd"], None, 1, H, Is)
        sync()
        rng = np.random.default_rng(seed)
        self.router_w_host = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        self.w["router_w"] = to_device_raw(to_bf16(self.router_w_host))
        self.sgl_host = (rng.standard_normal(H) * 0.02).astype(np.float32)
        self.w["sgl"] = to_device_raw(to_bf16(self.sgl_host))
        self.rng = rng

    def host_expert(self, name, e, rows, cols):
        """Host copy (q, s) of expert e of stacked weight `name`."""
        import numpy as np
        from sllm_amd import _lib
        q = np.empty((rows, cols), np.uint8)
        s = np.empty((rows // 128, cols // 128), np.float32)
        L = _lib.lib()
        qb, sb = self.w[name], self.w[name + "_s"]
        _lib.check(L.sllm_buf_d2h_raw(q.ctypes.data, qb.ptr + e * rows * cols, q.nbytes))
        _lib.check(L.sllm_buf_d2h_raw(s.ctypes.data, sb.ptr + e * s.nbytes, s.nbytes))
        return q, s


def layer_call(layer, x, out, ws, T, mode, debug=None, stage_events=None):
    from sllm_amd.moe import qwen_forward_dev
    c = layer.cfg
    qwen_forward_dev(x, out, layer.w, T=T, H=c["H"], E=c["E"], I=c["I"],
                     Is=c["Is"], topk=c["k"], mode=mode, out_f32=False,
                     workspace=ws, debug=debug, stage_events=stage_events)


class DeviceLayerDS:
    """Synthetic C4 layer on the device: routed N(0, 0.02) weights quantized
    to MXFP4 (e2m1 + e8m0 per 32, s = 2^ceil(log2(amax/6))), shared expert
    FP8 with power-of-two 128x128 scales, router bf16 N(0, 0.02), selection
    bias N(0, 0.01); all packed into the streaming layout."""

    def __init__(self, cfg, seed=0):
        import numpy as np
        from sllm_amd import _lib
        from sllm_amd.moe import pack_weights
        from sllm_amd.runtime import (DeviceBuffer, fill_normal, sync, to_bf16,
                                      to_device_raw)
        self.cfg = cfg
        H, E, I, Is = cfg["H"], cfg["E"], cfg["I"], cfg["Is"]
        L = _lib.lib()
        tmp = DeviceBuffer(E * I * H * 4)
        w = {}
        sub = [0]

        def q4(rows, cols):
            n = rows * cols
            fill_normal(tmp, n, seed * 1000 + 500 + sub[0], 0.02)
            sub[0] += 1
            q, sc = DeviceBuffer(n // 2), DeviceBuffer(n // 32)
            _lib.check(L.sllm_quantize_weight_mxfp4(tmp.ptr, rows, cols, q.ptr,
                                                    sc.ptr, None), "quantize")
            return q, sc

        def q8(rows, cols):
            n = rows * cols
            fill_normal(tmp, n, seed * 1000 + 500 + sub[0], 0.02)
            sub[0] += 1
            q, sc = DeviceBuffer(n), DeviceBuffer((rows // 128) * (cols // 128) * 4)
            _lib.check(L.sllm_quantize_weight_fp8(tmp.ptr, rows, cols, 1, q.ptr,
                                                  sc.ptr, None), "quantize")
            return q, sc

        w1, w1s = q4(E * I, H)
        w3, w3s = q4(E * I, H)
        w2, w2s = q4(E * H, I)
        w["w13_packed"], w["w13_s_packed"] = pack_weights(1, 1, w1, w3, E, I, H, w1s, w3s)
        w["w2_packed"], w["w2_s_packed"] = pack_weights(1, 0, w2, None, E, H, I, w2s)
        sync()
        w["w1"], w["w3"], w["w2"] = w1, w3, w2
        w["w1_s"], w["w3_s"], w["w2_s"] = w1s, w3s, w2s
        s1, w["s1_s"] = q8(Is, H)
        s3, w["s3_s"] = q8(Is, H)
        s2, w["s2_s"] = q8(H, Is)
        w["s13_packed"], _ = pack_weights(0, 1, s1, s3, 1, Is, H)
        w["s2_packed"], _ = pack_weights(0, 0, s2, None, 1, H, Is)
        w["s1"], w["s3"], w["s2"] = s1, s3, s2
        sync()
        tmp.free()
        rng = np.random.default_rng(seed)
        w["router_w"] = to_device_raw(to_bf16((rng.standard_normal((E, H)) * 0.02)
                                              .astype(np.float32)))
        w["bias"] = to_device_raw((rng.standard_normal(E) * 0.01).astype(np.float32))
        self.w = w
        self.rng = rng


def c4_inputs(layer):
    """The C4 activations: N(0, 1) rows from the layer's rng (drawn right
    after the router weights and bias), as float32; uploaded as bf16
    (rounded to nearest even, so the layer sees to_bf16_values of them)."""
    c = layer.cfg
    return layer.rng.standard_normal((c["T"], c["H"])).astype("float32")


def ds_call(layer, x, out, ws, T, mode, debug=None, stage_events=None):
    from sllm_amd.moe import deepseek_forward_dev
    c = layer.cfg
    deepseek_forward_dev(x, out, layer.w, T=T, H=c["H"], E=c["E"], I=c["I"],
                         Is=c["Is"], topk=c["k"], mode=mode, out_f32=False,
                         n_group=c["n_group"], topk_group=c["topk_group"],
                         scoring="sigmoid", route_scale=c["route_scale"],
                         swiglu_limit=c["swiglu_limit"], workspace=ws,
                         debug=debug, stage_events=stage_events)


def _time_layer(call, steps, warmup):
    from sllm_amd.runtime import Event, sync
    for _ in range(warmup):
        call()
    sync()
    e0, e1 = Event(), Event()
    e0.record()
    for _ in range(steps):
        call()
    e1.record()
    e1.synchronize()
    return e0.elapsed_ms(e1) / steps


def _stage_times(call_with_events, nstages, reps=10):
    from sllm_amd.moe import STAGES
    from sllm_amd.runtime import Event
    evs = [Event() for _ in range(2 * nstages)]
    per = {s: [] for s in STAGES}
    for _ in range(reps):
        call_with_events(evs)
        for e in evs:  # stages a call skips are recorded at its end
            e.synchronize()
        for i, s in enumerate(STAGES):
            per[s].append(evs[2 * i].elapsed_ms(evs[2 * i + 1]))
    return {s: round(statistics.median(v), 4) for s, v in per.items()}


def run_c4(args):
    """C4 prefill: one JSON line for this configuration."""
    print(json.dumps(c4_result(args)), flush=True)
    return 0


def c4_result(args):
    """C4 prefill (DeepSeek MXFP4) timed like the headline: layer ms and
    tokens/s, roofline fractions, per-stage ms, touched experts."""
    import numpy as np
    from sllm_amd.moe import STAGES, deepseek_workspace_bytes
    from sllm_amd.runtime import DeviceBuffer, sync, to_bf16, to_device_raw
    c = dict(C4)
    T, H, E, I, Is, k = c["T"], c["H"], c["E"], c["I"], c["Is"], c["k"]
    t0 = time.perf_counter()
    layer = DeviceLayerDS(c, seed=args.seed)
    xh = c4_inputs(layer)
    x = to_device_raw(to_bf16(xh))
    out = DeviceBuffer(T * H * 2)
    ws = DeviceBuffer(deepseek_workspace_bytes(T, H, E, I, Is, k, "prefill"))
    cnt = DeviceBuffer(E * 4)
    ds_call(layer, x, out, ws, T, "prefill", debug={"counts_out": cnt})
    sync()
    touched = int((cnt.copy_host_raw(np.int32, (E,)) > 0).sum())
    log(f"C4 setup {time.perf_counter() - t0:.1f}s, touched {touched}")
    ms = _time_layer(lambda: ds_call(layer, x, out, ws, T, "prefill"),
                     args.steps, args.warmup)
    st = _stage_times(lambda ev: ds_call(layer, x, out, ws, T, "prefill",
                                         stage_events=ev), len(STAGES))
    routing_us = _c4_routing_us(c, layer.rng)
    flops = 6 * H * I * T * k + 6 * H * Is * T
    wbytes = touched * 3 * H * I // 2 + touched * 3 * H * I // 32
    bytes_ = wbytes + 3 * H * Is + E * H * 2 + 2 * T * H * 2
    up_bytes = touched * (2 * I * H // 2 + 2 * I * H // 32) + T * H + T * k * I
    up_flops = 4 * H * I * T * k
    t_up = st["expert_up"] / 1e3
    res = {"metric": "C4 MoE layer tokens/s (prefill)", "value": round(T / (ms / 1e3), 1),
           "unit": "tokens/s", "ms_per_step": round(ms, 4), "steps": args.steps,
           "config": {"workload": "C4 DeepSeek-style MXFP4 MoE layer, prefill", **c},
           "layer": {"flops": flops, "bytes": bytes_,
                     "mfma_frac_fp8_rate": round(flops / (ms / 1e3) / (PEAK_FP8_TFLOPS * 1e12), 4),
                     "hbm_frac": round(bytes_ / (ms / 1e3) / (PEAK_HBM_GBPS * 1e9), 4),
                     "stage_ms": st, "touched_experts": touched},
           "expert_up": {"algorithmic_bytes": up_bytes, "ms": st["expert_up"],
                         "GBps": round(up_bytes / t_up / 1e9, 1),
                         "TFLOPs": round(up_flops / t_up / 1e12, 1),
                         "mfma_frac_fp8_rate": round(up_flops / t_up / (PEAK_FP8_TFLOPS * 1e12), 4)},
           "routing_us": routing_us}
    if not args.no_decode:
        res["decode"] = c4_decode(layer, xh, (1, 8, 32), args.decode_iters)
    del layer
    sync()
    return res


def c4_decode(layer, xh, batches, iters):
    """The C4 layer in decode mode at each batch size B (its first B tokens),
    per call between HIP events with a 512 MiB fill before each timed call
    (L2 and MALL flushed), as the C3 decode leg: us, touched experts, the
    algorithmic bytes (touched experts' MXFP4 weights and e8m0 scales, the
    FP8 shared expert and its scales, the bf16 router) and their rate."""
    import numpy as np
    from sllm_amd.moe import deepseek_workspace_bytes
    from sllm_amd.runtime import DeviceBuffer, Event, memset, sync, to_bf16, to_device_raw
    c = layer.cfg
    H, E, I, Is, k = c["H"], c["E"], c["I"], c["Is"], c["k"]
    flush = DeviceBuffer(512 << 20)
    a0, a1 = Event(), Event()
    out = {}
    for B in batches:
        xb = to_device_raw(to_bf16(xh[:B]))
        ob = DeviceBuffer(B * H * 2)
        wsb = DeviceBuffer(deepseek_workspace_bytes(B, H, E, I, Is, k, "decode"))
        cb = DeviceBuffer(E * 4)
        ds_call(layer, xb, ob, wsb, B, "decode", debug={"counts_out": cb})
        sync()
        tb = int((cb.copy_host_raw(np.int32, (E,)) > 0).sum())
        t = []
        for it in range(iters + 3):
            memset(flush, it & 0xFF, flush.nbytes)
            a0.record()
            ds_call(layer, xb, ob, wsb, B, "decode")
            a1.record()
            a1.synchronize()
            if it >= 3:
                t.append(a0.elapsed_ms(a1) * 1e3)
        us = statistics.median(t)
        nb = (tb * (3 * H * I // 2 + 3 * H * I // 32) + 3 * H * Is +
              3 * (H // 128) * (Is // 128) * 4 + E * H * 2)
        out[str(B)] = {"us": round(us, 2), "touched_experts": tb, "bytes": nb,
                       "GBps": round(nb / (us * 1e-6) / 1e9, 1),
                       "hbm_frac": round(nb / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
        log(f"C4 decode B={B}: {us:.1f} us, touched {tb}, "
            f"{nb / (us * 1e-6) / 1e9:.1f} GB/s")
    return out


def run_loader(args):
    """Checkpoint to device at C2 size: a synthetic Qwen FP8 MoE layer in the
    reference checkpoint naming (per-expert F8_E4M3 weights, BF16
    weight_scale_inv, BF16 router and gate) written to a temporary
    safetensors file, then timed through sllm_amd.loader (open + upload of
    the stored bytes + the one-time repack into the streaming layout). The
    file is read once before the timed load so that it sits in the page
    cache: the number is host-to-device, not disk, throughput."""
    import shutil
    import tempfile
    import numpy as np
    from sllm_amd import loader
    from sllm_amd.runtime import sync
    c = dict(C2)
    H, E, I, Is = c["H"], c["E"], c["I"], c["Is"]
    rng = np.random.default_rng(args.seed)
    pre = "model.language_model.layers.0.mlp"
    bf = lambda a: np.asarray(a, np.float32).view(np.uint32).__rshift__(16).astype(np.uint16)  # noqa: E731
    t = {f"{pre}.gate.weight": ("BF16", (E, H), bf(rng.standard_normal((E, H)) * 0.02))}
    codes = lambda n, k: rng.integers(0, 0x7E, (n, k), dtype=np.uint8)  # finite e4m3  # noqa: E731
    scl = lambda n, k: bf(rng.uniform(1e-5, 1e-4, (-(-n // 128), -(-k // 128))))  # noqa: E731
    for e in range(E):
        for m, (n, k) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            nm = f"{pre}.experts.{e}.{m}_proj.weight"
            t[nm] = ("F8_E4M3", (n, k), codes(n, k))
            t[nm + "_scale_inv"] = ("BF16", (-(-n // 128), -(-k // 128)), scl(n, k))
    for m, (n, k) in (("gate", (Is, H)), ("up", (Is, H)), ("down", (H, Is))):
        nm = f"{pre}.shared_expert.{m}_proj.weight"
        t[nm] = ("F8_E4M3", (n, k), codes(n, k))
        t[nm + "_scale_inv"] = ("BF16", (-(-n // 128), -(-k // 128)), scl(n, k))
    t[f"{pre}.shared_expert_gate.weight"] = ("BF16", (1, H), bf(rng.standard_normal((1, H)) * 0.02))
    d = tempfile.mkdtemp(prefix="sllm_ckpt_")
    try:
        path = os.path.join(d, "c2.safetensors")
        loader.write_safetensors(path, t)
        nbytes = os.path.getsize(path)
        del t
        with open(path, "rb") as f:  # warm the page cache
            while f.read(64 << 20):
                pass
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            layer = loader.load_qwen_moe(loader.Checkpoint(path), pre, c["k"])
            sync()
            times.append(time.perf_counter() - t0)
            del layer
        best = min(times)
        print(json.dumps({"metric": "C2 FP8 checkpoint to device (stored formats, no host dequant)",
                          "bytes": nbytes, "seconds": round(best, 4),
                          "GB_per_s": round(nbytes / best / 1e9, 2),
                          "includes": "open + per-tensor upload + streaming repack",
                          "runs": len(times)}), flush=True)
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return 0


# the hybrid family's dense MLP (recipes/schema.py:146 and :357 defaults)
DENSE = dict(H=5120, I=17408)


def run_device_decode(args):
    """The device-decode drop-ins (sllm_amd.decode) at decode batch sizes.
    MoE: the C2/C3 layer behind DeviceMoEStack; `hook_us` is the wall time
    of one `moe(x, i)` call with host arrays (the contract of the reference's
    Q4DeviceDecodeState._moe: bf16 conversion, upload, the fused layer,
    download), `hook_us_graph` the same with the layer replayed as a HIP
    graph, `device_us` the layer on device buffers (moe_dev) between HIP
    events. Dense: a DENSE-shaped FP8 SwiGLU MLP behind DenseSwiGLU,
    device time and HBM rate of its weight stream. L2 and MALL are flushed
    with a 512 MiB fill before every timed call."""
    import numpy as np
    from sllm_amd import _lib
    from sllm_amd.decode import DenseSwiGLU, DeviceMoEStack
    from sllm_amd.moe import QwenMoE
    from sllm_amd.runtime import (DeviceBuffer, Event, fill_normal, memset,
                                  sync, to_bf16, to_device_raw)
    c = dict(C2)
    H, E, I, Is, k = c["H"], c["E"], c["I"], c["Is"], c["k"]
    rng = np.random.default_rng(args.seed)
    flush = DeviceBuffer(512 << 20)
    iters = args.decode_iters

    def dev_us(call):
        a0, a1 = Event(), Event()
        times = []
        for it in range(iters + 3):
            memset(flush, it & 0xFF, flush.nbytes)
            a0.record()
            call()
            a1.record()
            a1.synchronize()
            if it >= 3:
                times.append(a0.elapsed_ms(a1) * 1e3)
        return statistics.median(times)

    def host_us(call):
        times = []
        for it in range(iters + 3):
            memset(flush, it & 0xFF, flush.nbytes)
            sync()
            t0 = time.perf_counter()
            call()
            if it >= 3:
                times.append((time.perf_counter() - t0) * 1e6)
        return statistics.median(times)

    base = DeviceLayer(c, seed=args.seed)
    w = {n: base.w[n] for n in ("router_w", "wg", "wg_s", "wu", "wu_s", "wd",
                                "wd_s", "sg", "sg_s", "su", "su_s", "sd", "sd_s",
                                "sgl", "wgu_packed", "wd_packed", "sgu_packed",
                                "sd_packed")}
    stack = DeviceMoEStack([QwenMoE.from_device(w, E=E, I=I, H=H, Is=Is, top_k=k)])
    graphed = DeviceMoEStack(stack.layers, graphs=True)
    moe = {}
    for B in (1, 8, 32):
        x = to_bf16_values(rng.standard_normal((B, H)).astype(np.float32))
        xd = to_device_raw(to_bf16(x))
        od = DeviceBuffer(B * H * 4)
        moe[str(B)] = {"hook_us": round(host_us(lambda: stack.moe(x, 0)), 1),
                       "hook_us_graph": round(host_us(lambda: graphed.moe(x, 0)), 1),
                       "device_us": round(dev_us(lambda: stack.moe_dev(xd, od, 0, B)), 1)}
        log(f"moe hook B={B}: {moe[str(B)]}")
    del stack, graphed, base, w
    sync()

    Hd, Id = DENSE["H"], DENSE["I"]
    L = _lib.lib()
    tmp = DeviceBuffer(Id * Hd * 4)
    b = {"router_w": to_device_raw(np.zeros(Hd, np.uint16))}
    for j, (key, n, kk) in enumerate((("wg", Id, Hd), ("wu", Id, Hd), ("wd", Hd, Id))):
        fill_normal(tmp, n * kk, args.seed * 1000 + 700 + j, 0.02)
        b[key] = DeviceBuffer(n * kk)
        b[key + "_s"] = DeviceBuffer((n // 128) * (kk // 128) * 4)
        _lib.check(L.sllm_quantize_weight_fp8(tmp.ptr, n, kk, 0, b[key].ptr,
                                              b[key + "_s"].ptr, None), "quantize")
    sync()
    tmp.free()
    mlp = DenseSwiGLU(QwenMoE.from_device(b, E=1, I=Id, H=Hd, Is=0, top_k=1))
    wbytes = 3 * Hd * Id + 3 * (Id // 128) * (Hd // 128) * 4
    dense = {}
    for B in (1, 8, 32):
        x = to_bf16_values(rng.standard_normal((B, Hd)).astype(np.float32))
        xd = to_device_raw(to_bf16(x))
        od = DeviceBuffer(B * Hd * 4)
        us = dev_us(lambda: mlp.forward_dev(xd, od, B))
        nb = wbytes + B * Hd * 2 + B * Hd * 4
        dense[str(B)] = {"device_us": round(us, 1), "bytes": nb,
                         "GBps": round(nb / (us * 1e-6) / 1e9, 1),
                         "hbm_frac": round(nb / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
        if B == 1:
            dense[str(B)]["hook_us"] = round(host_us(lambda: mlp(x)), 1)
        log(f"dense B={B}: {dense[str(B)]}")
    print(json.dumps({"metric": "device-decode drop-ins: per-call µs",
                      "moe": {"config": "C3 (C2 shapes, FP8)", "batches": moe},
                      "dense_mlp": {"config": {"hidden": Hd, "intermediate": Id,
                                               "weights": "e4m3 + fp32 128x128 block scales"},
                                    "batches": dense}}), flush=True)
    return 0


def _c4_routing_us(c, rng, reps=20):
    """The two DeepSeek routing kernels alone at C4 shape (synthetic fp32
    logits N(0,1)): group-limited sigmoid top-k with bias, and a hash layer
    (a seeded (vocab, k) token-id table of uniform expert ids; vocab 129280
    as DeepSeek-V3/V4)."""
    import numpy as np
    from sllm_amd import _lib
    from sllm_amd.runtime import DeviceBuffer, Event, sync, to_device_raw
    T, E, k = c["T"], c["E"], c["k"]
    V = 129280
    L = _lib.lib()
    lg = to_device_raw(rng.standard_normal((T, E)).astype(np.float32))
    bias = to_device_raw((rng.standard_normal(E) * 0.01).astype(np.float32))
    table = to_device_raw(rng.integers(0, E, (V, k)).astype(np.int32))
    tok = to_device_raw(rng.integers(0, V, T).astype(np.int32))
    w, ids = DeviceBuffer(T * k * 4), DeviceBuffer(T * k * 4)
    calls = {
        "grouped_topk": lambda: L.sllm_moe_route_grouped(
            lg.ptr, bias.ptr, w.ptr, ids.ptr, T, E, k, c["n_group"],
            c["topk_group"], 1, np.float32(c["route_scale"]), None),
        "hash": lambda: L.sllm_moe_route_hash(
            lg.ptr, tok.ptr, table.ptr, V, w.ptr, ids.ptr, T, E, k, 1,
            np.float32(c["route_scale"]), None),
    }
    out = {}
    for name, call in calls.items():
        _lib.check(call(), name)
        sync()
        e0, e1 = Event(), Event()
        e0.record()
        for _ in range(reps):
            call()
        e1.record()
        e1.synchronize()
        out[name] = round(e0.elapsed_ms(e1) / reps * 1e3, 2)
    return out


def c2_inputs(layer):
    """The C2 / C3 activations: bf16 N(0, 1) rows from the layer's rng (drawn
    right after the weights, as the headline run does)."""
    c = layer.cfg
    return to_bf16_values(layer.rng.standard_normal((c["T"], c["H"])).astype("float32"))


C5_EMPTY_FRAC = 20   # the lowest-ranked E / 20 experts receive no tokens


def c5_inputs(layer):
    """C5 activations and the skewed routing bias: x as c2_inputs; the
    router logits x . router_w^T get the per-expert bias
    b_e = -beta ln(rank_e) with ranks a seeded permutation of 1..E and beta
    calibrated (bisection on the first 2048 tokens' host logits) so that
    the top 10% of experts receive 60% of the assignments; the E / 20
    experts of the lowest ranks get a further -64 (a softmax weight below
    1e-27 of the others), so that they receive no tokens. The layer adds
    the bias to the logits its router GEMM computes (router_bias). Returns
    (x, bias (E,) float32, beta) on the host."""
    import numpy as np
    c = layer.cfg
    E, k = c["E"], c["k"]
    xh = c2_inputs(layer)
    rwh = to_bf16_values(layer.router_w_host)
    logits0 = (xh[:2048] @ rwh.T).astype(np.float32)
    rank = layer.rng.permutation(E) + 1
    off = np.where(rank > E - E // C5_EMPTY_FRAC, 64.0, 0.0)
    top = E // 10

    def share(beta):
        lg = logits0 - beta * np.log(rank)[None, :] - off[None, :]
        ids = np.argpartition(-lg, k, axis=1)[:, :k]
        cnt = np.bincount(ids.ravel(), minlength=E)
        return np.sort(cnt)[::-1][:top].sum() / cnt.sum()

    lo, hi = 0.0, 10.0
    for _ in range(40):
        mid = 0.5 * (lo + hi)
        lo, hi = (mid, hi) if share(mid) < 0.6 else (lo, mid)
    beta = 0.5 * (lo + hi)
    bias = (-beta * np.log(rank) - off).astype(np.float32)
    return xh, bias, beta


def run_c5(args):
    print(json.dumps(c5_result(args)), flush=True)
    return 0


def c5_result(args):
    """C5: C2 shapes at T=16384 with Zipf-skewed routing: the whole layer
    from bf16 x, router GEMM included, with the per-expert routing bias
    -beta ln(rank_e) added to its logits (ranks a seeded permutation of
    1..E, beta calibrated so the top 10% of experts take ~60% of the
    assignments)."""
    import numpy as np
    from sllm_amd.moe import STAGES, qwen_workspace_bytes
    from sllm_amd.runtime import DeviceBuffer, sync, to_bf16, to_device_raw
    c = dict(C5)
    T, H, E, I, Is, k = c["T"], c["H"], c["E"], c["I"], c["Is"], c["k"]
    t0 = time.perf_counter()
    layer = DeviceLayer(c, seed=args.seed)
    xh, bias, beta = c5_inputs(layer)
    top = E // 10
    x = to_device_raw(to_bf16(xh))
    wts = dict(layer.w, router_bias=to_device_raw(bias))
    out = DeviceBuffer(T * H * 2)
    ws = DeviceBuffer(qwen_workspace_bytes(T, H, E, I, Is, k, "prefill"))
    from sllm_amd.moe import qwen_forward_dev

    def call(debug=None, ev=None):
        qwen_forward_dev(x, out, wts, T=T, H=H, E=E, I=I, Is=Is, topk=k,
                         mode="prefill", out_f32=False, workspace=ws,
                         debug=debug, stage_events=ev)
    cnt = DeviceBuffer(E * 4)
    call(debug={"counts_out": cnt})
    sync()
    counts = cnt.copy_host_raw(np.int32, (E,))
    touched = int((counts > 0).sum())
    share_top = float(np.sort(counts)[::-1][:top].sum() / counts.sum())
    log(f"C5 setup {time.perf_counter() - t0:.1f}s, beta {beta:.3f}, top-10% share "
        f"{share_top:.3f}, empty experts {E - touched}")
    ms = _time_layer(call, args.steps, args.warmup)
    st = _stage_times(lambda ev: call(ev=ev), len(STAGES))
    flops, bytes_ = prefill_work(c, touched)
    res = {"metric": "C5 MoE layer tokens/s (prefill, skewed routing, router GEMM included)",
           "value": round(T / (ms / 1e3), 1), "unit": "tokens/s",
           "ms_per_step": round(ms, 4), "steps": args.steps,
           "config": {"workload": "C5 Qwen-style FP8 MoE layer, Zipf-skewed prefill", **c,
                      "beta": round(beta, 4), "top10pct_share": round(share_top, 4),
                      "empty_experts": E - touched},
           "layer": {"flops": flops, "bytes": bytes_,
                     "mfma_frac": round(flops / (ms / 1e3) / (PEAK_FP8_TFLOPS * 1e12), 4),
                     "hbm_frac": round(bytes_ / (ms / 1e3) / (PEAK_HBM_GBPS * 1e9), 4),
                     "attainable_frac": round(
                         max(flops / (PEAK_FP8_TFLOPS * 1e12), bytes_ / (PEAK_HBM_GBPS * 1e9))
                         / (ms / 1e3), 4),
                     "stage_ms": st, "touched_experts": touched,
                     "empty_experts": E - touched}}
    del layer
    sync()
    return res


# --------------------------------------------------------------------------
# algorithmic work: FLOPs of the GEMMs, bytes of the weights, scales and rows moved
# --------------------------------------------------------------------------
def prefill_work(c, touched):
    T, H, E, I, Is, k = c["T"], c["H"], c["E"], c["I"], c["Is"], c["k"]
    flops = 6 * H * I * T * k + 6 * H * Is * T
    wbytes = touched * 3 * H * I + touched * 3 * (H // 128) * (I // 128) * 4
    bytes_ = (wbytes + 3 * H * Is + E * H * 2 + H * 2 + 2 * T * H * 2)
    return flops, bytes_


def gemm1_bytes(c, touched):
    """Algorithmic HBM bytes of one routed gate/up launch: each touched
    expert's gate and up weights (e4m3) and scales once, the e4m3
    activations and their scales once, the e4m3 h rows and scales out."""
    T, H, I, k = c["T"], c["H"], c["I"], c["k"]
    N = T * k
    return (touched * (2 * I * H + 2 * (I // 128) * (H // 128) * 4)
            + T * H + T * (H // 128) * 4 + N * I + N * (I // 128) * 4)


def gemm2_bytes(c, touched):
    T, H, I, k = c["T"], c["H"], c["I"], c["k"]
    N = T * k
    return (touched * (H * I + (H // 128) * (I // 128) * 4)
            + N * I + N * (I // 128) * 4 + N * H * 2)


def decode_bytes(c, B, touched):
    H, E, I, Is = c["H"], c["E"], c["I"], c["Is"]
    return (touched * (3 * H * I + 3 * (H // 128) * (I // 128) * 4)
            + 3 * H * Is + E * H * 2 + H * 2 + 2 * B * H * 2)


# --------------------------------------------------------------------------
# CPU baseline: numpy restatement of the quantized layer, bounded sample
# --------------------------------------------------------------------------
def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or the platform's
    processor string where that file is absent."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(layer, x_host):
    """The whole C2 layer on this host's cores: the numpy restatement of the
    quantized layer in expert-grouped form (oracle act_quant, fp32 BLAS),
    router GEMM and softmax top-k, activation quant, all routed experts with
    their tokens, the shared expert and its gate. Weights are dequantized to
    fp32 outside the timed region (6.4 GB for C2). One warm-up,
    then the median of 3 runs; no extrapolation."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import codecs, quant
    c = layer.cfg
    T, H, E, I, Is, k = c["T"], c["H"], c["E"], c["I"], c["Is"], c["k"]
    cores = len(os.sched_getaffinity(0))
    t0 = time.perf_counter()
    deq = [tuple(codecs.dequant_fp8_block(*layer.host_expert(n, e, r, cc))
                 for n, r, cc in (("wg", I, H), ("wu", I, H), ("wd", H, I)))
           for e in range(E)]
    sh = tuple(codecs.dequant_fp8_block(*layer.host_expert(n, 0, r, cc))
               for n, r, cc in (("sg", Is, H), ("su", Is, H), ("sd", H, Is)))
    t_deq = time.perf_counter() - t0
    rw = codecs.round_bf16(layer.router_w_host)
    sgl = codecs.round_bf16(layer.sgl_host)

    def silu(v):
        return v / (1.0 + np.exp(-v))

    def expert(xr, g, u, d):
        h = (silu(xr @ g.T) * (xr @ u.T)).astype(np.float32)
        return quant.act_dequant(*quant.act_quant(h)) @ d.T

    def run():
        t0 = time.perf_counter()
        logits = x_host @ rw.T
        p = np.exp(logits - logits.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        sel = np.argsort(-p, axis=-1, kind="stable")[:, :k]
        w = np.take_along_axis(p, sel, -1)
        w /= w.sum(-1, keepdims=True) + np.float32(1e-20)
        xd = quant.act_dequant(*quant.act_quant(x_host))
        out = np.zeros((T, H), np.float32)
        order = np.argsort(sel.ravel(), kind="stable")
        bounds = np.searchsorted(sel.ravel()[order], np.arange(E + 1))
        for e in range(E):
            a = order[bounds[e]:bounds[e + 1]]
            if a.size:
                t, j = a // k, a % k
                out[t] += w[t, j][:, None] * expert(xd[t], *deq[e])
        gate = 1.0 / (1.0 + np.exp(-(x_host @ sgl)))
        out += gate[:, None] * expert(xd, *sh)
        return time.perf_counter() - t0

    with threadpool_limits(limits=cores):
        run()                                  # warm-up
        runs = [run() for _ in range(3)]
    sec = statistics.median(runs)
    return {
        "value": round(T / sec, 2), "unit": "tokens/s", "cores": cores,
        "cpu_model": cpu_model(), "kind": "port",
        "sample": (f"the whole C2 layer ({T} tokens, all {E} experts, shared "
                   f"expert), numpy restatement of the quantized layer (oracle "
                   f"act_quant + fp32 BLAS on weights dequantized beforehand, "
                   f"{t_deq:.0f} s, untimed); median of 3 after a warm-up; "
                   f"{cores} BLAS threads"),
        "seconds_per_layer": round(sec, 3),
        "runs_s": [round(r, 3) for r in runs],
    }


def cpu_c1_literal_loop():
    """The reference's literal per-token loop (ref/qwen4_exp.py:175-179, as
    oracle.qwen_moe.moe_block_forward) on C1: 64 tokens, H 1024, 16 experts,
    top-4, I 512, bf16-valued fp32 weights, seed 0. Median of 3 after a
    warm-up, single-threaded BLAS (the loop is GEMV-bound)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import codecs
    from oracle import qwen_moe as qm
    rng = np.random.default_rng(0)
    T, H, E, k, I = 64, 1024, 16, 4, 512
    bf = codecs.round_bf16
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    eg = bf((rng.standard_normal((E, I, H)) * 0.02).astype(np.float32))
    eu = bf((rng.standard_normal((E, I, H)) * 0.02).astype(np.float32))
    ed = bf((rng.standard_normal((E, H, I)) * 0.02).astype(np.float32))
    times = []
    with threadpool_limits(limits=1):
        for it in range(4):
            t0 = time.perf_counter()
            qm.moe_block_forward(x, rw, eg, eu, ed, None, None, None, None, k)
            if it:
                times.append(time.perf_counter() - t0)
    ms = statistics.median(times) * 1e3
    return {"config": "C1 (64 tokens, H 1024, E 16, top-4, I 512, bf16 weights)",
            "ms": round(ms, 2), "tokens_per_s": round(T / (ms / 1e3), 1),
            "cores": 1, "cpu_model": cpu_model(), "note": "median of 3 after a warm-up"}


# --------------------------------------------------------------------------
def decode_leg(layer, batches, iters, flush):
    """C3: the C2 layer in decode mode at each batch size B, per call
    between HIP events with a 512 MiB fill before each timed call (L2 and
    MALL flushed); `us` issues the layer's launches, `us_graph` replays the
    same call captured as a HIP graph; B=32 adds a per-stage breakdown."""
    import numpy as np
    from sllm_amd.moe import STAGES, LayerGraph, qwen_workspace_bytes
    from sllm_amd.runtime import DeviceBuffer, Event, memset, sync, to_bf16, to_device_raw
    c = layer.cfg
    H, E, I, Is, k = c["H"], c["E"], c["I"], c["Is"], c["k"]
    decode = {}
    for B in batches:
        xb_host = to_bf16_values(layer.rng.standard_normal((B, H)).astype(np.float32))
        xb = to_device_raw(to_bf16(xb_host))
        ob = DeviceBuffer(B * H * 2)
        wsb = DeviceBuffer(qwen_workspace_bytes(B, H, E, I, Is, k, "decode"))
        cb = DeviceBuffer(E * 4)
        layer_call(layer, xb, ob, wsb, B, "decode", debug={"counts_out": cb})
        sync()
        tb = int((cb.copy_host_raw(np.int32, (E,)) > 0).sum())
        a0, a1 = Event(), Event()

        def timed(run):
            t = []
            for it in range(iters + 3):
                memset(flush, it & 0xFF, flush.nbytes)
                a0.record()
                run()
                a1.record()
                a1.synchronize()
                if it >= 3:
                    t.append(a0.elapsed_ms(a1) * 1e3)
            return statistics.median(t)
        us = timed(lambda: layer_call(layer, xb, ob, wsb, B, "decode"))
        g = LayerGraph(xb, ob, layer.w, T=B, H=H, E=E, I=I, Is=Is, topk=k,
                       mode="decode", out_f32=False, workspace=wsb)
        us_graph = timed(g.launch)
        g.free()
        nb = decode_bytes(c, B, tb)
        decode[str(B)] = {"us": round(us, 2), "us_graph": round(us_graph, 2),
                          "touched_experts": tb,
                          "bytes": nb, "GBps": round(nb / (us * 1e-6) / 1e9, 1),
                          "hbm_frac": round(nb / (us * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)}
        if B == 32:  # per-stage breakdown (flushed like the timed calls)
            evs = [Event() for _ in range(2 * len(STAGES))]
            per = {s_: [] for s_ in STAGES}
            for it in range(10):
                memset(flush, it & 0xFF, flush.nbytes)
                layer_call(layer, xb, ob, wsb, B, "decode", stage_events=evs)
                for e in evs:
                    e.synchronize()
                for i, s_ in enumerate(STAGES):
                    per[s_].append(evs[2 * i].elapsed_ms(evs[2 * i + 1]) * 1e3)
            decode[str(B)]["stage_us"] = {s_: round(statistics.median(v), 2)
                                          for s_, v in per.items()}
        log(f"decode B={B}: {us:.1f} us ({us_graph:.1f} as a graph replay), "
            f"touched {tb}, {decode[str(B)]['GBps']} GB/s")
    return decode


def run_decode_batch(args):
    """One C3 decode batch alone (the C2 layer at B = --decode-batch
    tokens; with --config c4 the C4 layer's first B tokens), one JSON line:
    for profiling the decode kernels."""
    from sllm_amd.runtime import DeviceBuffer
    if args.config == "c4":
        layer = DeviceLayerDS(dict(C4), seed=args.seed)
        d = c4_decode(layer, c4_inputs(layer), (args.decode_batch,),
                      args.decode_iters)
        print(json.dumps({"metric": "C4 decode layer us",
                          "batch": args.decode_batch,
                          **d[str(args.decode_batch)]}), flush=True)
        return 0
    layer = DeviceLayer(dict(C2), seed=args.seed)
    flush = DeviceBuffer(512 << 20)
    d = decode_leg(layer, (args.decode_batch,), args.decode_iters, flush)
    print(json.dumps({"metric": "C3 decode layer us", "batch": args.decode_batch,
                      **d[str(args.decode_batch)]}), flush=True)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # the GPU's clocks take ~40 ms of uninterrupted work to settle after
    # idle (C2 calls: 0.475 ms in the first 10 ms, 0.41 ms from ~40 ms on);
    # 100 warm-up calls are ~45 ms at C2
    ap.add_argument("--warmup", type=int, default=100)
    # clock settle, before (and not counted in) the warm-up calls: layer
    # calls until this much wall time has passed, reported as its own key
    ap.add_argument("--settle-ms", type=float, default=100.0)
    ap.add_argument("--decode-iters", type=int, default=20)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra-configs", action="store_true",
                    help="leave the C4 and C5 legs out of the default line")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--config", choices=("c2", "c4", "c5"), default="c2",
                    help="c2 (default): the headline line; c4 / c5: one line "
                         "for that configuration instead")
    ap.add_argument("--loader", action="store_true",
                    help="only time loading a synthetic C2-shaped FP8 "
                         "checkpoint (safetensors, reference naming) to the "
                         "device and exit")
    ap.add_argument("--decode-batch", type=int, default=0, metavar="B",
                    help="only time the C3 decode layer at B tokens and exit "
                         "(with --config c4: the C4 layer's decode)")
    ap.add_argument("--device-decode", action="store_true",
                    help="only time the device-decode drop-ins (MoE hook and "
                         "dense SwiGLU MLP) at decode batch sizes and exit")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="only run the library's copy kernel over MIB MiB five "
                         "times (the known-size reference for scaling HBM "
                         "byte counters) and exit")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus "
              f"{args.gpus}); the MoE layer's multi-GPU expert-parallel "
              f"sharding is a design note, not a measured path.",
              file=sys.stderr)
        return 2

    import numpy as np

    from sllm_amd import _lib
    from sllm_amd.moe import STAGES, qwen_workspace_bytes
    from sllm_amd.runtime import (DeviceBuffer, Event, memset, sync, to_bf16,
                                  to_device_raw)
    if not _lib.available():
        raise RuntimeError(f"libsllm_moe.so unavailable: {_lib._lib_error}")

    if args.copy_calib:
        from sllm_amd.runtime import copy
        nb = args.copy_calib << 20
        src, dst = DeviceBuffer(nb), DeviceBuffer(nb)
        memset(src, 1, nb)
        for _ in range(5):
            copy(dst, src, nb)
        sync()
        print(json.dumps({"copy_calib_bytes": nb, "launches": 5}))
        return 0
    if args.loader:
        return run_loader(args)
    if args.device_decode:
        return run_device_decode(args)
    if args.decode_batch:
        return run_decode_batch(args)
    if args.config == "c4":
        return run_c4(args)
    if args.config == "c5":
        return run_c5(args)

    c = dict(C2)
    T, H, E, I, Is, k = c["T"], c["H"], c["E"], c["I"], c["Is"], c["k"]
    t_setup = time.perf_counter()
    layer = DeviceLayer(c, seed=args.seed)
    x_host = c2_inputs(layer)
    x = to_device_raw(to_bf16(x_host))
    out = DeviceBuffer(T * H * 2)
    ws = DeviceBuffer(qwen_workspace_bytes(T, H, E, I, Is, k, "prefill"))
    dbg = {"ids_out": DeviceBuffer(T * k * 4), "w_out": DeviceBuffer(T * k * 4),
           "counts_out": DeviceBuffer(E * 4)}
    layer_call(layer, x, out, ws, T, "prefill", debug=dbg)
    sync()
    counts = dbg["counts_out"].copy_host_raw(np.int32, (E,))
    touched = int((counts > 0).sum())
    log(f"setup {time.perf_counter() - t_setup:.1f}s; touched experts {touched}")

    # ---- clock settle (reported as "settle"), then the warm-up calls -----
    settle_calls, s0 = 0, time.perf_counter()
    while (time.perf_counter() - s0) * 1e3 < args.settle_ms:
        for _ in range(16):
            layer_call(layer, x, out, ws, T, "prefill")
        sync()
        settle_calls += 16
    settle = {"calls": settle_calls,
              "ms": round((time.perf_counter() - s0) * 1e3, 1),
              "note": "layer calls before the warm-up so the clocks ramp up; "
                      "not counted in warmup"}

    # ---- headline: K steps of the full layer ---------------------------
    for _ in range(args.warmup):
        layer_call(layer, x, out, ws, T, "prefill")
    sync()
    e0, e1 = Event(), Event()
    w0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        layer_call(layer, x, out, ws, T, "prefill")
    e1.record()
    e1.synchronize()
    wall = time.perf_counter() - w0
    sync()
    ms = e0.elapsed_ms(e1) / args.steps
    tok_s = T / (ms / 1e3)
    log(f"prefill {ms:.3f} ms/layer ({tok_s:.4g} tok/s), wall {wall * 1e3 / args.steps:.3f} ms")

    # ---- per-stage breakdown (roofline of the dominant kernel) ----------
    evs = [Event() for _ in range(2 * len(STAGES))]
    per_stage = {s: [] for s in STAGES}
    for _ in range(max(5, min(args.steps, 20))):
        layer_call(layer, x, out, ws, T, "prefill", stage_events=evs)
        for e in evs:
            e.synchronize()
        for i, s in enumerate(STAGES):
            per_stage[s].append(evs[2 * i].elapsed_ms(evs[2 * i + 1]))
    stage_ms = {s: statistics.median(v) for s, v in per_stage.items()}
    dom = max(("expert_up", "expert_down"), key=lambda s: stage_ms[s])
    dom_bytes = gemm1_bytes(c, touched) if dom == "expert_up" else gemm2_bytes(c, touched)
    dom_gbps = dom_bytes / (stage_ms[dom] / 1e3) / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", f"traffic_{dom}_c2.json")
    if os.path.isfile(tf):
        with open(tf) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    flops, bytes_ = prefill_work(c, touched)
    t_s = ms / 1e3
    layer_info = {
        "ms": round(ms, 4), "flops": flops, "bytes": bytes_,
        "mfma_frac": round(flops / t_s / (PEAK_FP8_TFLOPS * 1e12), 4),
        "hbm_frac": round(bytes_ / t_s / (PEAK_HBM_GBPS * 1e9), 4),
        "attainable_frac": round(max(flops / (PEAK_FP8_TFLOPS * 1e12),
                                     bytes_ / (PEAK_HBM_GBPS * 1e9)) / t_s, 4),
        "stage_ms": {s: round(v, 4) for s, v in stage_ms.items()},
        "touched_experts": touched,
    }

    # ---- the same layer with L2 and MALL flushed before every call -------
    flush = DeviceBuffer(512 << 20)
    fl = []
    a0, a1 = Event(), Event()
    for it in range(13):
        memset(flush, it & 0xFF, flush.nbytes)
        a0.record()
        layer_call(layer, x, out, ws, T, "prefill")
        a1.record()
        a1.synchronize()
        if it >= 3:
            fl.append(a0.elapsed_ms(a1))
    layer_info["ms_flushed"] = round(statistics.median(fl), 4)
    layer_info["flush"] = "512 MiB fill before each of 10 timed calls (median)"
    log(f"prefill with caches flushed: {layer_info['ms_flushed']} ms")

    # ---- decode batches (C3) -------------------------------------------
    decode = {} if args.no_decode else decode_leg(layer, (1, 8, 32, 64),
                                                  args.decode_iters, flush)

    # ---- CPU baseline -----------------------------------------------------
    cpu = c1_loop = None
    if not args.no_cpu:
        tc = time.perf_counter()
        cpu = cpu_baseline(layer, x_host)
        log(f"cpu baseline {cpu['value']} tok/s ({time.perf_counter() - tc:.1f}s)")
        c1_loop = cpu_c1_literal_loop()
        log(f"cpu C1 literal loop {c1_loop['ms']} ms")

    # ---- C4 and C5 (their own layers; the C2 layer is freed first) --------
    extra = {}
    if not args.no_extra_configs:
        del layer, x, out, ws, dbg
        sync()
        for name, fn in (("c4", c4_result), ("c5", c5_result)):
            r = fn(args)
            extra[name] = {"ms": r["ms_per_step"], "tokens_per_s": r["value"],
                           "config": r["config"], "layer": r["layer"]}
            if "expert_up" in r:
                extra[name]["expert_up"] = r["expert_up"]
            if "routing_us" in r:
                extra[name]["routing_us"] = r["routing_us"]
            if "decode" in r:
                extra[name]["decode"] = r["decode"]
            log(f"{name}: {r['ms_per_step']} ms, {r['value']} tok/s")

    res = {
        "metric": METRIC, "value": round(tok_s, 1), "unit": "tokens/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "settle": settle,
        "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp8_e4m3",
        "data": "synthetic (seeded N(0,0.02) weights quantized on device, bf16 N(0,1) activations)",
        "config": {"workload": "C2 Qwen-style FP8 MoE layer, prefill",
                   "tokens": T, "hidden": H, "experts": E, "top_k": k,
                   "intermediate": I, "shared_intermediate": Is,
                   "weights": "e4m3 + fp32 128x128 block scales",
                   "activations": "bf16, e4m3 per 1x128 before each expert GEMM"},
        "roofline": {"bound": "hbm",
                     "kernel": f"moe_stream_kernel<fp8,{0 if dom == 'expert_up' else 1}>",
                     "achieved": round(dom_gbps, 1), "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(dom_gbps / PEAK_HBM_GBPS, 4),
                     "traffic": traffic, "algorithmic_bytes": dom_bytes,
                     "avg_ms": round(stage_ms[dom], 4)},
        "layer": layer_info,
        "decode": decode,
        "decode_us_at_32": decode.get("32", {}).get("us"),
        "cpu_baseline": cpu,
        "cpu_c1_literal_loop": c1_loop,
        **extra,
    }
    print(json.dumps(res), flush=True)
    return 0


def to_bf16_values(a):
    """float32 array rounded to bf16 values (kept as float32)."""
    import numpy as np
    u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


if __name__ == "__main__":
    sys.exit(main())
