"""GPU parity of the device-decode drop-ins (sllm_amd.decode).

DeviceMoEStack.moe(x, i) stands in for Q4DeviceDecodeState._moe
(kernels/q4_device_decode.py:316-339): its oracle is the reference's
literal per-token loop (ref/qwen4_exp.py:153-184, oracle.qwen_moe.
moe_block_forward) on the same bf16 weights, and for FP8 checkpoints the
array-built layer, bit for bit. DenseSwiGLU stands in for the hybrid
family's dense MLP (kernels/hybrid_device_decode.py:308-311): its oracle is
swiglu_mlp (ref/qwen4_exp.py:143-150) on the same bf16 weights or on the
dequantized FP8 blocks. The decode path multiplies bf16 x against bf16 (or
exactly widened e4m3 x fp32 scale) weights with fp32 accumulation and an
fp32 intermediate, so the bound is rel-L2 < 1e-4.
"""
import numpy as np
import pytest

from oracle import codecs
from oracle import qwen_moe as qm
from tests._fixtures import (qwen_checkpoint_tensors, qwen_fp8, qwen_layer,
                             rel_l2)

pytestmark = pytest.mark.gpu

bf = codecs.round_bf16
PRE = "model.language_model"


@pytest.fixture(scope="module", autouse=True)
def _lib_loaded():
    from sllm_amd import _lib
    if not _lib.available():
        pytest.fail(f"libsllm_moe.so not loadable: {_lib._lib_error}")


def _weight_dict(rng, n_layers, E, H, I, Is):
    """The reference's float weight dict (bf16-exact values) for n_layers
    MoE blocks, in Q4DeviceWeightTable's names."""
    w = {}
    nrm = lambda *s: bf((rng.standard_normal(s) * 0.02).astype(np.float32))  # noqa: E731
    for i in range(n_layers):
        p = f"{PRE}.layers.{i}.mlp"
        w[f"{p}.gate.weight"] = nrm(E, H)
        for e in range(E):
            w[f"{p}.experts.{e}.gate_proj.weight"] = nrm(I, H)
            w[f"{p}.experts.{e}.up_proj.weight"] = nrm(I, H)
            w[f"{p}.experts.{e}.down_proj.weight"] = nrm(H, I)
        w[f"{p}.shared_expert.gate_proj.weight"] = nrm(Is, H)
        w[f"{p}.shared_expert.up_proj.weight"] = nrm(Is, H)
        w[f"{p}.shared_expert.down_proj.weight"] = nrm(H, Is)
        w[f"{p}.shared_expert_gate.weight"] = nrm(1, H)
    return w


def _ref_moe(w, x, i, E, k):
    p = f"{PRE}.layers.{i}.mlp"
    st = lambda m: np.stack([w[f"{p}.experts.{e}.{m}_proj.weight"]  # noqa: E731
                             for e in range(E)])
    return qm.moe_block_forward(
        x, w[f"{p}.gate.weight"], st("gate"), st("up"), st("down"),
        w[f"{p}.shared_expert.gate_proj.weight"],
        w[f"{p}.shared_expert_gate.weight"],
        w[f"{p}.shared_expert.up_proj.weight"],
        w[f"{p}.shared_expert.down_proj.weight"], k)


def test_moe_stack_matches_reference_loop():
    """Two layers, batch sizes changing between calls (1 -> 5 -> 1): the
    cached staging, workspace and argument blocks must follow."""
    from sllm_amd.decode import DeviceMoEStack
    rng = np.random.default_rng(40)
    E, H, I, Is, k = 16, 512, 256, 256, 4
    w = _weight_dict(rng, 2, E, H, I, Is)
    stack = DeviceMoEStack.from_weights(w, 2, k)
    xs = [bf(rng.standard_normal((n, H)).astype(np.float32)) for n in (1, 5, 1)]
    for x in xs:
        for i in (0, 1):
            got = stack.moe(x, i)
            want = _ref_moe(w, x, i, E, k)
            rel = rel_l2(got, want)
            print(f"layer {i} n {x.shape[0]}: rel-L2 {rel:.2e}")
            assert got.shape == (x.shape[0], H) and got.dtype == np.float32
            assert rel < 1e-4
    np.testing.assert_array_equal(stack.moe(xs[1], 0), stack.moe(xs[1], 0))


def test_moe_stack_dev_matches_host():
    from sllm_amd.decode import DeviceMoEStack
    from sllm_amd.runtime import DeviceBuffer, sync, to_bf16, to_device_raw
    rng = np.random.default_rng(41)
    E, H, I, Is, k, n = 8, 512, 256, 256, 2, 7
    w = _weight_dict(rng, 1, E, H, I, Is)
    stack = DeviceMoEStack.from_weights(w, 1, k)
    x = bf(rng.standard_normal((n, H)).astype(np.float32))
    xd = to_device_raw(to_bf16(x))
    out = DeviceBuffer(n * H * 4)
    stack.moe_dev(xd, out, 0, n)
    sync()
    np.testing.assert_array_equal(out.copy_host().reshape(n, H), stack.moe(x, 0))


def test_moe_stack_from_fp8_checkpoint(tmp_path):
    """Layers loaded from an FP8 checkpoint (two MoE blocks, BF16 scales)
    equal the array-built layers bit for bit."""
    from sllm_amd import loader
    from sllm_amd.decode import DeviceMoEStack
    k, t, Ws = 4, {}, []
    for i in range(2):
        x, W = qwen_fp8(seed=50 + i, T=6, H=512, E=8, I=256, Is=256)
        for a in ("wg_s", "wu_s", "wd_s", "sg_s", "su_s", "sd_s"):
            setattr(W, a, codecs.decode_bf16(codecs.encode_bf16_rne(getattr(W, a))))
        t.update(qwen_checkpoint_tensors(W, f"{PRE}.layers.{i}.mlp"))
        Ws.append(W)
    p = str(tmp_path / "two_layers.safetensors")
    loader.write_safetensors(p, t)
    stack = DeviceMoEStack.from_checkpoint(loader.Checkpoint(p), 2, k)
    for i, W in enumerate(Ws):
        want = qwen_layer(W, k).forward(x, mode="decode")
        np.testing.assert_array_equal(stack.moe(x, i), want)


@pytest.mark.parametrize("n", [1, 3, 16, 17, 32, 50, 64])
def test_dense_swiglu_bf16(n):
    from sllm_amd.decode import DenseSwiGLU
    rng = np.random.default_rng(60 + n)
    H, I = 768, 384
    nrm = lambda *s: bf((rng.standard_normal(s) * 0.02).astype(np.float32))  # noqa: E731
    p = f"{PRE}.layers.3.mlp"
    w = {f"{p}.gate_proj.weight": nrm(I, H), f"{p}.up_proj.weight": nrm(I, H),
         f"{p}.down_proj.weight": nrm(H, I)}
    mlp = DenseSwiGLU.from_weights(w, 3)
    x = bf(rng.standard_normal((n, H)).astype(np.float32))
    got = mlp(x)
    want = qm.swiglu_mlp(x, w[f"{p}.gate_proj.weight"], w[f"{p}.up_proj.weight"],
                         w[f"{p}.down_proj.weight"])
    rel = rel_l2(got, want)
    print(f"dense bf16 n {n}: rel-L2 {rel:.2e}")
    assert rel < 1e-4


def test_dense_swiglu_fp8_checkpoint(tmp_path):
    from sllm_amd import loader
    from sllm_amd.decode import DenseSwiGLU
    from oracle import quant
    rng = np.random.default_rng(70)
    H, I = 1024, 640
    q = {m: quant.quantize_weight_fp8_block(
        (rng.standard_normal(s) * 0.02).astype(np.float32))
         for m, s in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    p = f"{PRE}.layers.0.mlp"
    t = {}
    for m, (codes, sc) in q.items():
        t[f"{p}.{m}_proj.weight"] = ("F8_E4M3", codes.shape, codes)
        t[f"{p}.{m}_proj.weight_scale_inv"] = ("F32", sc.shape, sc)
    path = str(tmp_path / "dense.safetensors")
    loader.write_safetensors(path, t)
    mlp = DenseSwiGLU.from_checkpoint(loader.Checkpoint(path), p)
    deq = {m: codecs.dequant_fp8_block(*v) for m, v in q.items()}
    for n in (1, 9):
        x = bf(rng.standard_normal((n, H)).astype(np.float32))
        rel = rel_l2(mlp(x), qm.swiglu_mlp(x, deq["gate"], deq["up"], deq["down"]))
        print(f"dense fp8 n {n}: rel-L2 {rel:.2e}")
        assert rel < 1e-4


@pytest.mark.parametrize("T,mode", [(1, "decode"), (8, "decode"), (32, "decode"),
                                    (96, "prefill")])
def test_layer_graph_replays_match_eager(T, mode):
    """A captured layer call (sllm_moe_qwen_graph_new) replayed five times,
    with new inputs written into the captured x buffer and eager layer calls
    and synchronizations between the replays: every replay equals the eager
    call on the same input bit for bit (same kernels, same order)."""
    from sllm_amd.moe import LayerGraph, qwen_forward_dev, qwen_workspace_bytes
    from sllm_amd.runtime import DeviceBuffer, sync, to_bf16
    x0, W = qwen_fp8(seed=80 + T, T=T, H=512, E=16, I=256, Is=256)
    k = 4
    layer = qwen_layer(W, k)
    H, E, I, Is = layer.H, layer.E, layer.I, layer.Is
    kw = dict(T=T, H=H, E=E, I=I, Is=Is, topk=k, mode=mode, out_f32=True,
              wdtype=layer.wdtype, eps=layer.eps)
    xg = DeviceBuffer(T * H * 2)
    og = DeviceBuffer(T * H * 4)
    wsg = DeviceBuffer(qwen_workspace_bytes(T, H, E, I, Is, k, mode))
    g = LayerGraph(xg, og, layer._w, workspace=wsg, **kw)
    xe = DeviceBuffer(T * H * 2)
    oe = DeviceBuffer(T * H * 4)
    wse = DeviceBuffer(qwen_workspace_bytes(T, H, E, I, Is, k, mode))
    rng = np.random.default_rng(T)
    for r in range(5):
        x = bf(rng.standard_normal((T, H)).astype(np.float32))
        xg.upload_raw(to_bf16(x))
        xe.upload_raw(to_bf16(x))
        sync()
        g.launch()
        qwen_forward_dev(xe, oe, layer._w, workspace=wse, **kw)
        sync()
        got, want = og.copy_host().reshape(T, H), oe.copy_host().reshape(T, H)
        np.testing.assert_array_equal(got, want, err_msg=f"replay {r}")
        # eager work on the graph's own buffers between replays
        qwen_forward_dev(xg, og, layer._w, workspace=wsg, **kw)
        sync()
    g.free()
    with pytest.raises(RuntimeError):
        g.launch()


def test_moe_stack_graphs_match_eager():
    """DeviceMoEStack with graph replay equals it without (the default), at
    changing batch sizes (1 -> 8 -> 1 -> 3) over two layers."""
    from sllm_amd.decode import DeviceMoEStack
    rng = np.random.default_rng(42)
    E, H, I, Is, k = 16, 512, 256, 256, 4
    w = _weight_dict(rng, 2, E, H, I, Is)
    se = DeviceMoEStack.from_weights(w, 2, k)
    sg = DeviceMoEStack(se.layers, graphs=True)
    for n in (1, 8, 1, 3):
        x = bf(rng.standard_normal((n, H)).astype(np.float32))
        for i in (0, 1):
            np.testing.assert_array_equal(sg.moe(x, i), se.moe(x, i))
