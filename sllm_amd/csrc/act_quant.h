// Per-row activation quantization on one wave, shared by the
// activation-quant launch (quant.hip) and the prefill softmax routing
// launch, which quantizes its token's row as well (router.hip). The
// quantization point restates ref/hf_sources/dsv4/kernel.py:40-125: per
// 128 columns, s = max(amax, 1e-4) * fp32(1/448) (or its power-of-two
// ceiling, :22-37), q = e4m3(clamp(x / s, +-448)) with round-to-nearest-
// even; bit-exact with oracle/quant.py (same fp32 operations in the same
// order: IEEE division, hardware RNE conversion).
#pragma once
#include "common.h"

namespace sllm {

__device__ __forceinline__ float pow2_ceil(float v) {
  uint32_t b = __float_as_uint(v);
  int e = (int)((b >> 23) & 0xFF) - 127 + ((b & 0x7FFFFF) ? 1 : 0);
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// Row t of x (bf16, H a multiple of 128) on the calling wave. Lane group
// g = lane / 16 takes blocks g, g + 4, ...; its 16 lanes load 8 bf16 each
// (16 bytes). The loads of up to four blocks per lane (16 blocks per wave)
// are issued together before any is converted. q == nullptr: only the
// gate. gate_w: also gate_out[t] = sigmoid(x . gate_w) (the Qwen
// shared-expert gate, ref/qwen4_exp.py:180-183), each lane adding its
// blocks in order.
__device__ __forceinline__ void act_quant_row(
    const uint16_t* __restrict__ x, int t, int H, int pow2,
    uint8_t* __restrict__ q, float* __restrict__ s,
    const uint16_t* __restrict__ gate_w, float* __restrict__ gate_out) {
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, li = lane & 15;
  const int nblk = H / 128;
  const uint16_t* row = x + (size_t)t * H;
  float gdot = 0.f;
  for (int b0 = 0; b0 < nblk; b0 += 16) {
    uint4 raw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int blk = b0 + 4 * j + g;
      raw[j] = blk < nblk ? *(const uint4*)(row + blk * 128 + li * 8)
                          : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int blk = b0 + 4 * j + g;
      const bool on = blk < nblk;
      const int col = blk * 128 + li * 8;
      const uint32_t w4[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
      float v[8];
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w4[i] << 16);
        v[2 * i + 1] = __uint_as_float(w4[i] & 0xFFFF0000u);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
      if (gate_w && on) {
        const uint4 gr = *(const uint4*)(gate_w + col);
        const uint32_t g4[4] = {gr.x, gr.y, gr.z, gr.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          gdot += v[2 * i] * __uint_as_float(g4[i] << 16);
          gdot += v[2 * i + 1] * __uint_as_float(g4[i] & 0xFFFF0000u);
        }
      }
#pragma unroll
      for (int o = 8; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 16));
      if (on && q) {
        float sc = fmaxf(amax, 1e-4f) * (1.0f / 448.0f);
        if (pow2) sc = pow2_ceil(sc);
        float y[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] = fminf(fmaxf(v[i] / sc, -448.f), 448.f);
        uint2 packed;
        packed.x = f32x4_to_e4m3(y[0], y[1], y[2], y[3]);
        packed.y = f32x4_to_e4m3(y[4], y[5], y[6], y[7]);
        *(uint2*)(q + (size_t)t * H + col) = packed;
        if (li == 0) s[(size_t)t * nblk + blk] = sc;
      }
    }
  }
  if (gate_w) {
    gdot = wave_sum(gdot);
    if (lane == 0) gate_out[t] = sigmoid_f32(gdot);
  }
}

}  // namespace sllm
