"""sllm_amd: MI355X-native (gfx950, HIP) mixture-of-experts layer for sLLM.

Host side is Python + numpy over a ctypes C-ABI (include/sllm_moe.h) to the
HIP library sllm_amd/lib/libsllm_moe.so, matching the reference's binding
style (kernels/_q4_cuda.py, _fp8_cuda.py, _deepseek_cuda.py, _sllm_cuda.py).

Modules:
  runtime   device buffers, sync, gemm_ex      (ref kernels/_sllm_cuda.py)
  q4        moe_router, swiglu, axpy_rows, ... (ref kernels/_q4_cuda.py)
  fp8       fp8_gemm(_dev)                     (ref kernels/_fp8_cuda.py)
  deepseek  fp4_moe_linear                     (ref kernels/_deepseek_cuda.py)
  moe       the fused layers: QwenMoE, DeepseekMoE, *_forward_dev
  build     hipcc build of the library
"""

from . import _lib

available = _lib.available

__all__ = ["available"]
