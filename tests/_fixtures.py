"""Synthetic MoE layers for the tests (seeded numpy, oracle quantizers).

Generation follows the BASELINE config recipes: activations bf16 N(0,1),
weights N(0, 0.02) quantized to e4m3 with fp32 128x128 block scales
(amax/448) or to MXFP4 (e2m1 + e8m0 per 32), router weights bf16
N(0, 0.02), DeepSeek selection bias N(0, 0.01).
"""

from __future__ import annotations

import numpy as np

from oracle import codecs, quant
from oracle import deepseek_moe as dm
from oracle import qwen_moe as qm

bf = codecs.round_bf16


def qwen_fp8(seed=0, T=64, H=512, E=8, I=256, Is=256, shared=True,
             x_scale=1.0):
    rng = np.random.default_rng(seed)
    x = bf((rng.standard_normal((T, H)) * x_scale).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.02).astype(np.float32))

    def qw(n, k):
        return quant.quantize_weight_fp8_block(
            (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    g = [qw(I, H) for _ in range(E)]
    u = [qw(I, H) for _ in range(E)]
    d = [qw(H, I) for _ in range(E)]
    W = qm.QwenFp8Weights(
        router_w=rw,
        wg_q=np.stack([a for a, _ in g]), wg_s=np.stack([b for _, b in g]),
        wu_q=np.stack([a for a, _ in u]), wu_s=np.stack([b for _, b in u]),
        wd_q=np.stack([a for a, _ in d]), wd_s=np.stack([b for _, b in d]))
    if shared:
        (W.sg_q, W.sg_s), (W.su_q, W.su_s), (W.sd_q, W.sd_s) = \
            qw(Is, H), qw(Is, H), qw(H, Is)
        W.sgl = bf((rng.standard_normal((1, H)) * 0.02).astype(np.float32))
    return x, W


class _DevRng:
    """Seeded stream of N(0, std^2) device arrays from sllm_fill_normal
    (torch must not touch the GPU here: it bundles another HIP runtime)."""

    def __init__(self, seed):
        self.seed = int(seed) * 1000003
        self.k = 0

    def normal(self, n, std):
        from sllm_amd.runtime import DeviceBuffer, fill_normal
        buf = DeviceBuffer(int(n) * 4)
        fill_normal(buf, n, self.seed + self.k, std)
        self.k += 1
        return buf


def _gpu_fp8(rng, E, N, K, pow2=False):
    """E stacked (N, K) weights ~N(0, 0.02) quantized on the device with
    sllm_quantize_weight_fp8 (bit-exact with oracle.quant, see
    test_gpu_kernels.py) -> host (q (E,N,K) uint8, s (E,N/128,K/128))."""
    from sllm_amd import _lib
    from sllm_amd.runtime import DeviceBuffer
    assert N % 128 == 0
    kb = -(-K // 128)
    w = rng.normal(E * N * K, 0.02)
    q = DeviceBuffer(E * N * K)
    sc = DeviceBuffer(E * N // 128 * kb * 4)
    _lib.check(_lib.lib().sllm_quantize_weight_fp8(w.ptr, E * N, K, int(pow2),
                                                   q.ptr, sc.ptr, None))
    w.free()
    return (q.copy_host_raw(np.uint8, (E, N, K)),
            sc.copy_host_raw(np.float32, (E, N // 128, kb)))


def _gpu_fp4(rng, E, N, K):
    from sllm_amd import _lib
    from sllm_amd.runtime import DeviceBuffer
    w = rng.normal(E * N * K, 0.02)
    p = DeviceBuffer(E * N * K // 2)
    sc = DeviceBuffer(E * N * K // 32)
    _lib.check(_lib.lib().sllm_quantize_weight_mxfp4(w.ptr, E * N, K, p.ptr,
                                                     sc.ptr, None))
    w.free()
    return (p.copy_host_raw(np.uint8, (E, N, K // 2)),
            sc.copy_host_raw(np.uint8, (E, N, K // 32)))


def qwen_fp8_gpu(seed=0, T=64, H=2048, E=128, I=512, Is=512, shared=True):
    """qwen_fp8 with the expert weights generated (sllm_fill_normal) and
    quantized on the GPU: the numpy route takes minutes at C2 geometry."""
    rng = np.random.default_rng(seed)
    dr = _DevRng(seed)
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    g, u, d = _gpu_fp8(dr, E, I, H), _gpu_fp8(dr, E, I, H), _gpu_fp8(dr, E, H, I)
    W = qm.QwenFp8Weights(router_w=rw, wg_q=g[0], wg_s=g[1], wu_q=u[0],
                          wu_s=u[1], wd_q=d[0], wd_s=d[1])
    if shared:
        sg, su, sd = _gpu_fp8(dr, 1, Is, H), _gpu_fp8(dr, 1, Is, H), _gpu_fp8(dr, 1, H, Is)
        W.sg_q, W.sg_s = sg[0][0], sg[1][0]
        W.su_q, W.su_s = su[0][0], su[1][0]
        W.sd_q, W.sd_s = sd[0][0], sd[1][0]
        W.sgl = bf((rng.standard_normal((1, H)) * 0.02).astype(np.float32))
    return x, W


def deepseek_mxfp4_gpu(seed=0, T=64, H=7168, E=32, I=2048, Is=2048, shared=True):
    rng = np.random.default_rng(seed)
    dr = _DevRng(seed)
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    w1, w3, w2 = _gpu_fp4(dr, E, I, H), _gpu_fp4(dr, E, I, H), _gpu_fp4(dr, E, H, I)
    W = dm.DeepseekMxfp4Weights(router_w=rw, bias=bias, w1_p=w1[0], w1_s=w1[1],
                                w3_p=w3[0], w3_s=w3[1], w2_p=w2[0], w2_s=w2[1])
    if shared:
        s1, s3, s2 = (_gpu_fp8(dr, 1, Is, H, True), _gpu_fp8(dr, 1, Is, H, True),
                      _gpu_fp8(dr, 1, H, Is, True))
        W.s1_q, W.s1_s = s1[0][0], s1[1][0]
        W.s3_q, W.s3_s = s3[0][0], s3[1][0]
        W.s2_q, W.s2_s = s2[0][0], s2[1][0]
    return x, W


def qwen_layer(W, top_k, packed=True):
    from sllm_amd.moe import QwenMoE
    kw = {"packed": packed}
    if W.has_shared:
        kw.update(sg=W.sg_q, su=W.su_q, sd=W.sd_q, sg_s=W.sg_s, su_s=W.su_s,
                  sd_s=W.sd_s, sgl=W.sgl)
    return QwenMoE(W.router_w, W.wg_q, W.wu_q, W.wd_q, W.wg_s, W.wu_s,
                   W.wd_s, top_k=top_k, **kw)


def deepseek_mxfp4(seed=0, T=64, H=512, E=16, I=256, Is=256, shared=True):
    rng = np.random.default_rng(seed)
    x = bf(rng.standard_normal((T, H)).astype(np.float32))
    rw = bf((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)

    def q4(n, k):
        return quant.quantize_weight_mxfp4(
            (rng.standard_normal((n, k)) * 0.02).astype(np.float32))

    def q8(n, k):
        return quant.quantize_weight_fp8_block(
            (rng.standard_normal((n, k)) * 0.02).astype(np.float32), pow2=True)
    w1 = [q4(I, H) for _ in range(E)]
    w3 = [q4(I, H) for _ in range(E)]
    w2 = [q4(H, I) for _ in range(E)]
    W = dm.DeepseekMxfp4Weights(
        router_w=rw, bias=bias,
        w1_p=np.stack([a for a, _ in w1]), w1_s=np.stack([b for _, b in w1]),
        w3_p=np.stack([a for a, _ in w3]), w3_s=np.stack([b for _, b in w3]),
        w2_p=np.stack([a for a, _ in w2]), w2_s=np.stack([b for _, b in w2]))
    if shared:
        (W.s1_q, W.s1_s), (W.s3_q, W.s3_s), (W.s2_q, W.s2_s) = \
            q8(Is, H), q8(Is, H), q8(H, Is)
    return x, W


def deepseek_layer(W, top_k, packed=True, **route):
    from sllm_amd.moe import DeepseekMoE
    kw = {"packed": packed}
    if W.has_shared:
        kw.update(s1=W.s1_q, s1_s=W.s1_s, s3=W.s3_q, s3_s=W.s3_s, s2=W.s2_q,
                  s2_s=W.s2_s)
    return DeepseekMoE(W.router_w, W.bias, W.w1_p, W.w1_s, W.w3_p, W.w3_s,
                       W.w2_p, W.w2_s, top_k=top_k, **kw, **route)


def qwen_checkpoint_tensors(W, prefix, scale_tag="BF16"):
    """W in a Qwen FP8 checkpoint's naming under `prefix` (a `.mlp` block):
    per-expert F8_E4M3 weights with `weight_scale_inv` blocks stored as
    `scale_tag` (BF16 or F32), BF16 router and shared-expert gate. Returns
    {name: (dtype tag, shape, array)} for sllm_amd.loader.write_safetensors."""
    def sc(a):
        return (("BF16", a.shape, codecs.encode_bf16_rne(a)) if scale_tag == "BF16"
                else ("F32", a.shape, np.asarray(a, np.float32)))
    t = {f"{prefix}.gate.weight": ("BF16", W.router_w.shape,
                                   codecs.encode_bf16_rne(W.router_w))}
    mats = [("gate", W.wg_q, W.wg_s), ("up", W.wu_q, W.wu_s), ("down", W.wd_q, W.wd_s)]
    for e in range(W.wg_q.shape[0]):
        for m, q, sv in mats:
            n = f"{prefix}.experts.{e}.{m}_proj.weight"
            t[n] = ("F8_E4M3", q[e].shape, q[e])
            t[n + "_scale_inv"] = sc(sv[e])
    if W.has_shared:
        for m, q, sv in [("gate", W.sg_q, W.sg_s), ("up", W.su_q, W.su_s),
                         ("down", W.sd_q, W.sd_s)]:
            n = f"{prefix}.shared_expert.{m}_proj.weight"
            t[n] = ("F8_E4M3", q.shape, q)
            t[n + "_scale_inv"] = sc(sv)
        t[f"{prefix}.shared_expert_gate.weight"] = ("BF16", W.sgl.shape,
                                                    codecs.encode_bf16_rne(W.sgl))
    return t


def qwen_checkpoint(path, W, prefix, scale_tag="BF16"):
    from sllm_amd.loader import write_safetensors
    write_safetensors(path, qwen_checkpoint_tensors(W, prefix, scale_tag))


def check_router_logits(name, xh, rw, got):
    """Device router logits against fp64 x . W_r^T of the same bf16 values
    (ref/qwen4_exp.py:173, kernels/cuda/qwen4.cu:98-113,
    ref/deepseek_v4.py:57-60): within 4 2^-24 sum_h |x_h| |w_h| per logit,
    the bound of an fp32 accumulation of the exact bf16 products in any
    order of chunks of at most 2^21 terms."""
    x64, w64 = np.asarray(xh, np.float64), np.asarray(rw, np.float64)
    want = x64 @ w64.T
    mag = np.abs(x64) @ np.abs(w64).T
    err = np.abs(np.asarray(got, np.float64) - want)
    ratio = float((err / (mag + 1e-300)).max())
    print(f"{name}: router logits vs fp64, max |err| / sum|x||w| = "
          f"{ratio:.3e} (bound 4 * 2^-24 = {4 * 2.0 ** -24:.3e})", flush=True)
    assert np.all(err <= 4 * 2.0 ** -24 * mag + 1e-30)


def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def certified_tie_tokens(ids_dev, ids_ref, p_ref) -> np.ndarray:
    """Tokens whose device and oracle ids differ only where the oracle's
    fp32 probabilities of the two experts are bitwise equal (a rounding tie
    of the probabilities that the device, selecting on the logits, breaks by
    the logit order). Raises on any other mismatch. Returns the sorted token
    indices with at least one such tie."""
    bad = np.argwhere(ids_dev != ids_ref)
    tied = set()
    for t, j in bad:
        a, b = int(ids_dev[t, j]), int(ids_ref[t, j])
        if p_ref[t, a] != p_ref[t, b]:
            raise AssertionError(
                f"routing mismatch at token {t} slot {j}: device {a} "
                f"(p={p_ref[t, a]!r}) vs oracle {b} (p={p_ref[t, b]!r})")
        tied.add(int(t))
    return np.array(sorted(tied), np.int64)


def certified_route_ties(ids_dev, ids_ref, p_ref) -> int:
    """Number of mismatching (token, slot) positions that are certified
    ties (see certified_tie_tokens); raises on any other mismatch."""
    bad = np.argwhere(ids_dev != ids_ref)
    certified_tie_tokens(ids_dev, ids_ref, p_ref)
    return len(bad)


def check_qwen_routing(logits, ids, w, k, eps=1e-20, name="routing"):
    """Device routing (ids, w) against the oracle's moe_route of the same
    fp32 logits: ids bit-exact except certified ties (printed), weights
    rtol 1e-5 on every token without a tie. Returns the tied tokens."""
    from oracle import qwen_moe as qm
    w_ref, ids_ref = qm.moe_route(logits, k, eps)
    tied = certified_tie_tokens(ids, ids_ref.astype(np.int32), qm.softmax_rows(logits))
    print(f"{name}: {len(tied)} tokens with a certified probability tie")
    keep = np.ones(len(ids), bool)
    keep[tied] = False
    np.testing.assert_allclose(w[keep], w_ref[keep], rtol=1e-5, atol=1e-7)
    return tied
