"""CPU checks of the drop-in boundary: the library loads without a GPU and
exports every function include/sllm_moe.h declares; the ctypes signature
table covers the same set; the argument structs match the header."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    src = open(os.path.join(ROOT, "include", "sllm_moe.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b(sllm_\w+)\s*\(", src)
    return sorted(set(names))


def test_header_declares_reference_names():
    names = _header_functions()
    for ref in ("sllm_q4_moe_router", "sllm_q4_moe_router_dev", "sllm_q4_swiglu",
                "sllm_q4_axpy_rows", "sllm_q4_shared_gate_accum", "sllm_fp8_gemm",
                "sllm_fp8_gemm_dev", "sllm_ds_fp4_gemm", "sllm_buf_new",
                "sllm_buf_free", "sllm_buf_h2d", "sllm_buf_h2d_raw", "sllm_buf_d2h",
                "sllm_mem_free_bytes", "sllm_sync", "sllm_device_count",
                "sllm_last_error", "sllm_q4_last_error", "sllm_fp8_last_error",
                "sllm_ds_last_error", "sllm_gemm_ex"):
        assert ref in names, ref


def test_library_exports_every_declared_symbol():
    from sllm_amd import _lib
    if not os.path.isfile(_lib.LIB_PATH):
        pytest.fail("library not built: run python -m sllm_amd.build")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _header_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(_lib.SIGNATURES) == _header_functions()
    assert _lib.available()


def test_struct_layout_matches_header():
    from sllm_amd import _lib
    src = open(os.path.join(ROOT, "include", "sllm_moe.h")).read()
    for cname, py in (("sllm_moe_qwen_args", _lib.QwenArgs),
                      ("sllm_moe_ds_args", _lib.DeepseekArgs)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), src,
                         re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            parts = decl.replace("*", " ").split()
            names = " ".join(parts[1:]).replace(",", " ").split()
            if parts[0] == "const":
                names = " ".join(parts[2:]).replace(",", " ").split()
            fields += names
        assert [f for f, _ in py._fields_] == fields, cname


def test_error_contract_without_gpu():
    from sllm_amd import _lib, q4
    lib = _lib.lib()
    rc = lib.sllm_q4_moe_router(None, None, None, 0, 4, 2)
    assert rc == -1
    assert "bad args" in _lib.last_error()
    with pytest.raises(RuntimeError, match="rc=-1"):
        _lib.check(rc, "q4 kernel")
    assert q4.available()
    # graph entry points: argument errors before any device call
    assert lib.sllm_moe_qwen_graph_new(None) is None
    assert "null args" in _lib.last_error()
    a = _lib.QwenArgs()
    a.T, a.H, a.E, a.I, a.topk = 4, 100, 8, 128, 2
    assert lib.sllm_moe_qwen_graph_new(a) is None
    assert "H % 256" in _lib.last_error()
    assert lib.sllm_moe_graph_launch(None, None) == -1
    assert "null graph" in _lib.last_error()
    assert lib.sllm_moe_graph_free(None) == 0


def test_host_bf16_rounding_matches_python():
    """sllm_host_f32_to_bf16 (host code, no GPU) against runtime.to_bf16 on
    random values and the patterns where rounding carries or wraps."""
    import numpy as np
    from sllm_amd import _lib
    from sllm_amd.runtime import to_bf16
    rng = np.random.default_rng(5)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000,
                        0x7F800001, 0x7F7FFFFF, 0x00000001, 0x3F808000,
                        0x3F818000, 0x3F80FFFF, 0xFFFFFFFF, 0x7FFFFFFF],
                       np.uint32)
    bits = np.concatenate([rng.integers(0, 2**32, 4096, dtype=np.uint64)
                           .astype(np.uint32), special])
    x = bits.view(np.float32)
    got = np.empty(x.size, np.uint16)
    _lib.check(_lib.lib().sllm_host_f32_to_bf16(got.ctypes.data, x.ctypes.data, x.size))
    np.testing.assert_array_equal(got, to_bf16(x))


@pytest.mark.parametrize("inline", ["1", "0"])
def test_decode_workspace_holds_split_router_slices(inline, monkeypatch):
    """Host plan, no GPU: a decode call that computes its own logits splits
    the router GEMM's K over 2 workgroups when its batch is routed by
    many workgroups: by the multi-workgroup routing kernel (17 <= T <= 64
    here), or up to 8 tokens inside the gate/up launch, whose workgroups
    each read the slices. Its workspace then holds 2 partial-logit slices
    of T * E floats and 2 partial gate slices of T floats beyond a call
    given the logits. Batches routed in one fused workgroup (9 <= T <= 16,
    and T <= 8 with SLLM_MOE_ROUTE_INLINE=0) and prefill keep one slice;
    prefill also holds the fused router's partials: per token and
    128-expert tile, a (max, sum) pair and k top-k keys of 8 bytes."""
    from sllm_amd.moe import qwen_workspace_bytes as wsb
    monkeypatch.setenv("SLLM_MOE_ROUTE_INLINE", inline)

    def up256(n):
        return -(-n // 256) * 256
    H, E, I, Is, k = 2048, 512, 512, 512, 10
    for T, mode, split in ((1, "decode", inline == "1"),
                           (8, "decode", inline == "1"), (9, "decode", False),
                           (16, "decode", False),
                           (17, "decode", True), (32, "decode", True),
                           (64, "decode", True), (128, "prefill", False)):
        own = wsb(T, H, E, I, Is, k, mode)
        given = wsb(T, H, E, I, Is, k, mode, logits_given=True)
        want = (up256(2 * T * E * 4) + up256(3 * T * 4) - up256(T * 4)
                if split else up256(T * E * 4))
        if mode == "prefill":
            want += up256(T * (E // 128) * 8 * (1 + k))
        assert own - given == want, T
