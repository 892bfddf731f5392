// Activation quantization and synthetic-weight quantizers.
//
// act_quant restates the upstream quantization point that the reference's
// numpy oracles leave out (act_quant.h: the per-row body, also run by the
// prefill softmax routing launch). The shared-expert gate of the Qwen layer,
// sigmoid(x . W_sg) (ref/qwen4_exp.py:180-183), needs one dot product per
// token over the same row, so it is fused here rather than paid as a
// separate pass over x.
#include "act_quant.h"
#include "launch.h"

namespace sllm {

// One wave per row, 4 rows per workgroup. q == nullptr computes only the
// gate (the decode path keeps x in fp32).
__global__ __launch_bounds__(256) void act_quant_kernel(
    const uint16_t* x, int T, int H, int pow2, uint8_t* q, float* s,
    const uint16_t* gate_w, float* gate_out) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  act_quant_row(x, t, H, pow2, q, s, gate_w, gate_out);
}

int launch_act_quant(const uint16_t* x, int T, int H, int pow2, uint8_t* q,
                     float* s, const uint16_t* gate_w, float* gate_out,
                     hipStream_t st) {
  SLLM_REQUIRE(x && ((q && s) || (!q && gate_w)), "act_quant: null pointer");
  SLLM_REQUIRE(T > 0 && H > 0 && H % 128 == 0,
               "act_quant: need T>0 and H %% 128 == 0 (T=%d H=%d)", T, H);
  SLLM_REQUIRE(!gate_w || gate_out, "act_quant: gate_w without gate_out");
  act_quant_kernel<<<ceil_div(T, 4), 256, 0, st>>>(x, T, H, pow2, q, s,
                                                    gate_w, gate_out);
  SLLM_LAUNCHED();
  return 0;
}

// --------------------------------------------------------------------------
// synthetic weight quantizers (data preparation, not the layer)
// --------------------------------------------------------------------------
// FP8 128x128 block: one workgroup per block, s = amax * fp32(1/448)
// (optionally its power-of-two ceiling), q = e4m3(clamp(w / s)).
__global__ __launch_bounds__(256) void quant_w_fp8_kernel(
    const float* __restrict__ w, int N, int K, int pow2,
    uint8_t* __restrict__ q, float* __restrict__ s) {
  __shared__ float red[4];
  const int nb = blockIdx.y, kb = blockIdx.x;
  const int KB = (K + 127) / 128;
  const int tid = threadIdx.x;
  // thread -> (row r = tid/2 .. step 128, 64 columns)
  float amax = 0.f;
  for (int i = tid; i < 128 * 128; i += 256) {
    int r = nb * 128 + i / 128, c = kb * 128 + i % 128;
    if (r < N && c < K) amax = fmaxf(amax, fabsf(w[(size_t)r * K + c]));
  }
  amax = wave_max(amax);
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sc = fmaxf(amax, 1e-4f) * (1.0f / 448.0f);
  if (pow2) sc = pow2_ceil(sc);
  if (tid == 0) s[(size_t)nb * KB + kb] = sc;
  for (int i = tid; i < 128 * 128; i += 256) {
    int r = nb * 128 + i / 128, c = kb * 128 + i % 128;
    if (r < N && c < K) {
      float y = fminf(fmaxf(w[(size_t)r * K + c] / sc, -448.f), 448.f);
      q[(size_t)r * K + c] =
          (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(y, 0.f, 0, false) & 0xFF);
    }
  }
}

// E2M1 nibble of a value already divided by its scale (|a| <= 6), nearest
// with ties to the even code (oracle/codecs.py:encode_e2m1_rne).
__device__ __forceinline__ uint32_t e2m1_rne(float v) {
  float a = fabsf(v);
  uint32_t c;
  if (a <= 0.25f) c = 0;
  else if (a < 0.75f) c = 1;
  else if (a <= 1.25f) c = 2;
  else if (a < 1.75f) c = 3;
  else if (a <= 2.5f) c = 4;
  else if (a < 3.5f) c = 5;
  else if (a <= 5.0f) c = 6;
  else c = 7;
  return c | (__float_as_uint(v) >> 31 << 3);
}

// MXFP4 per 32 along K: one thread per (row, 32-block); s is the power of two
// 2^ceil(log2(amax * fp32(1/6))) as ref/deepseek_v4.py:175-189 chooses it.
__global__ __launch_bounds__(256) void quant_w_mxfp4_kernel(
    const float* __restrict__ w, int N, int K, uint8_t* __restrict__ packed,
    uint8_t* __restrict__ scale) {
  const int KB = K / 32;
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)N * KB) return;
  const int r = (int)(i / KB), kb = (int)(i % KB);
  const float* src = w + (size_t)r * K + kb * 32;
  float v[32];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 32; j += 4) {
    float4 f = *(const float4*)(src + j);
    v[j] = f.x; v[j + 1] = f.y; v[j + 2] = f.z; v[j + 3] = f.w;
  }
#pragma unroll
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(v[j]));
  float sc = pow2_ceil(fmaxf(amax, 1e-30f) * (1.0f / 6.0f));
  uint32_t out[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    float y = fminf(fmaxf(v[j] / sc, -6.f), 6.f);
    out[j / 8] |= e2m1_rne(y) << (4 * (j % 8));
  }
  *(uint4*)(packed + (size_t)r * (K / 2) + kb * 16) =
      make_uint4(out[0], out[1], out[2], out[3]);
  scale[(size_t)r * KB + kb] = (uint8_t)((__float_as_uint(sc) >> 23) & 0xFF);
}

}  // namespace sllm

using namespace sllm;

extern "C" {

int sllm_moe_act_quant(const void* x_bf16, int T, int H, int pow2,
                       void* q_e4m3, float* scale, const void* gate_w_bf16,
                       float* gate_out, void* stream) {
  return launch_act_quant((const uint16_t*)x_bf16, T, H, pow2,
                          (uint8_t*)q_e4m3, scale,
                          (const uint16_t*)gate_w_bf16, gate_out,
                          (hipStream_t)stream);
}

int sllm_quantize_weight_fp8(const float* w, int N, int K, int pow2,
                             void* q_e4m3, float* scale, void* stream) {
  SLLM_REQUIRE(w && q_e4m3 && scale && N > 0 && K > 0,
               "sllm_quantize_weight_fp8: bad args");
  dim3 grid((K + 127) / 128, (N + 127) / 128);
  quant_w_fp8_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(
      w, N, K, pow2, (uint8_t*)q_e4m3, scale);
  SLLM_LAUNCHED();
  return 0;
}

int sllm_quantize_weight_mxfp4(const float* w, int N, int K, void* packed,
                               void* scale_e8m0, void* stream) {
  SLLM_REQUIRE(w && packed && scale_e8m0 && N > 0 && K > 0 && K % 32 == 0,
               "sllm_quantize_weight_mxfp4: bad args (K %% 32 == 0)");
  long n = (long)N * (K / 32);
  quant_w_mxfp4_kernel<<<(unsigned)((n + 255) / 256), 256, 0,
                         (hipStream_t)stream>>>(w, N, K, (uint8_t*)packed,
                                                (uint8_t*)scale_e8m0);
  SLLM_LAUNCHED();
  return 0;
}

}  // extern "C"
