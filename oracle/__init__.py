"""CPU oracle for the sLLM mixture-of-experts layer -- TEST INFRASTRUCTURE ONLY.

This package is a numpy restatement of the reference's MoE arithmetic. It is
the checker that the HIP library is compared against; it is never the thing
measured or shipped. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it. The product path
(``sllm_amd``) never imports it and fails loudly when the HIP library is
missing.

Modules and the reference code each one restates (paths relative to the
skfine24/sLLM checkout):

- ``codecs``   loaders/fp8.py:34-200 (E4M3FN / BF16 / E8M0 / E2M1 decoding,
               block dequant) plus round-to-nearest-even encoders.
- ``quant``    ref/hf_sources/dsv4/kernel.py:22-125 (act_quant, including the
               ue8m0 power-of-two scale) and :203-273 / :441-536 (block-scaled
               FP8 and FP4 GEMM accumulation order).
- ``qwen_moe`` ref/qwen4_exp.py:118-184 (softmax top-k routing, SwiGLU
               experts, sigmoid-gated shared expert) and the quantized layer.
- ``deepseek_moe`` ref/deepseek_v4.py:522-570 (sigmoid scoring with
               selection bias, expert_ffn with swiglu_limit) with the
               upstream combine of ref/hf_sources/dsv4/model.py:684-699, and
               the group-limited top-k the reference does not have.
- ``permute``  the stable expert-major permutation
               (np.argsort(ids.ravel(), kind="stable"), bincount as in
               ref/hf_sources/dsv4/model.py:689).

How each function is pinned (golden vectors, closed forms, library
routines, brute force) is stated in its docstring and exercised by
``tests/test_oracle_*.py``.
"""
