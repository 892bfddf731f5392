"""sllm_moe_qwen_forward_noalloc (the layer on the library's per-device
scratch, no workspace argument) against sllm_moe_qwen_forward on the same
inputs: two calls in a row (a prefill call, then a smaller decode call),
each equal bit for bit to the workspace entry point's output and routing
(same kernels, deterministic order); and a call whose workspace would exceed
the scratch is refused with rc -2 before anything runs.
"""
import numpy as np
import pytest

from tests._fixtures import qwen_fp8, qwen_layer

pytestmark = pytest.mark.gpu


def _lib():
    from sllm_amd import _lib as L
    if not L.available():
        pytest.fail(f"libsllm_moe.so not loadable: {L._lib_error}")
    return L


def _noalloc(L, a):
    return L.lib().sllm_moe_qwen_forward_noalloc(a)


def _call(layer, x, T, mode, noalloc):
    """One layer call; returns (out fp32 (T, H), ids (T, k), sorted (T k,))."""
    from sllm_amd.moe import _qwen_args, qwen_workspace_bytes
    from sllm_amd.runtime import DeviceBuffer, sync, to_bf16, to_device_raw
    L = _lib()
    H, E, I, Is, k = layer.H, layer.E, layer.I, layer.Is, layer.top_k
    xd = to_device_raw(to_bf16(x))
    out = DeviceBuffer(T * H * 4)
    dbg = {"ids_out": DeviceBuffer(T * k * 4), "sorted_out": DeviceBuffer(T * k * 4)}
    ws, nb = None, 0
    if not noalloc:
        nb = qwen_workspace_bytes(T, H, E, I, Is, k, mode, Is > 0)
        ws = DeviceBuffer(nb)
    a = _qwen_args(T, H, E, I, Is, k, mode, True, 0, 1e-20, xd, None, layer._w,
                   out, dbg, ws, nb, None)
    rc = _noalloc(L, a) if noalloc else L.lib().sllm_moe_qwen_forward(a)
    L.check(rc, "noalloc layer" if noalloc else "layer")
    sync()
    return (out.copy_host().reshape(T, H), dbg["ids_out"].copy_host_raw(np.int32, (T, k)),
            dbg["sorted_out"].copy_host_raw(np.int32, (T * k,)))


def test_noalloc_matches_workspace_entry_point():
    from sllm_amd.moe import noalloc_max_bytes
    assert noalloc_max_bytes() == 32 << 20
    x, W = qwen_fp8(seed=41, T=200, H=512, E=8, I=256, Is=256)
    layer = qwen_layer(W, 2)
    # first call: prefill, T = 200; second: decode, T = 7 (smaller)
    for T, mode in ((200, "prefill"), (7, "decode")):
        want = _call(layer, x[:T], T, mode, noalloc=False)
        got = _call(layer, x[:T], T, mode, noalloc=True)
        for g, w_ in zip(got, want):
            np.testing.assert_array_equal(g, w_)
        # the workspace entry point itself is oracle-checked in
        # test_gpu_layer.py; here the scratch path must reproduce it exactly
        print(f"noalloc {mode} T={T}: equal to the workspace entry point "
              f"({np.abs(got[0]).max():.3e} max |out|)")
        assert np.isfinite(got[0]).all()


def test_noalloc_refuses_calls_beyond_the_scratch():
    """T = 16384 at H = 512, top-2 needs more than 32 MiB of workspace (the
    y rows alone are 32 MiB): rc -2 and a message, before any launch (the
    buffers are real and sized for the call all the same)."""
    from sllm_amd.moe import _qwen_args, qwen_workspace_bytes
    from sllm_amd.runtime import DeviceBuffer, to_bf16, to_device_raw
    L = _lib()
    x, W = qwen_fp8(seed=42, T=64, H=512, E=8, I=256, Is=256)
    layer = qwen_layer(W, 2)
    T = 16384
    assert qwen_workspace_bytes(T, 512, 8, 256, 256, 2, "prefill") > 32 << 20
    xd = to_device_raw(to_bf16(np.tile(x, (T // 64, 1))))
    out = DeviceBuffer(T * 512 * 4)
    a = _qwen_args(T, 512, 8, 256, 256, 2, "prefill", True, 0, 1e-20, xd, None,
                   layer._w, out, None, None, 0, None)
    assert _noalloc(L, a) == -2
    assert "scratch" in L.last_error()
    # a workspace argument is refused too (the call would not use it)
    ws = DeviceBuffer(1 << 20)
    a = _qwen_args(64, 512, 8, 256, 256, 2, "decode", True, 0, 1e-20, xd, None,
                   layer._w, out, None, ws, ws.nbytes, None)
    assert _noalloc(L, a) == -1
