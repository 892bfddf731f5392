// Shared definitions for the sLLM MoE HIP library (gfx950 / MI355X).
//
// Error model (mirrors the reference's C-ABI, kernels/cuda/qwen4.cu:23-34):
// every entry point returns 0 on success, -1 on bad arguments or a runtime
// error, -2 on a capacity bound; the message is kept in a THREAD-LOCAL
// buffer (the reference's buffers are process-global statics) that all the
// *_last_error getters return.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

namespace sllm {

// --------------------------------------------------------------------------
// errors
// --------------------------------------------------------------------------
void set_error(const char* fmt, ...);
const char* last_error();

#define SLLM_HIP(expr)                                                        \
  do {                                                                        \
    hipError_t _e = (expr);                                                   \
    if (_e != hipSuccess) {                                                   \
      ::sllm::set_error("%s:%d %s: %s", __FILE__, __LINE__, #expr,            \
                        hipGetErrorString(_e));                               \
      return -1;                                                              \
    }                                                                         \
  } while (0)

#define SLLM_REQUIRE(cond, ...)                                               \
  do {                                                                        \
    if (!(cond)) {                                                            \
      ::sllm::set_error(__VA_ARGS__);                                         \
      return -1;                                                              \
    }                                                                         \
  } while (0)

// A capacity bound (the reference's rc -2, qwen4.cu:582, 661).
#define SLLM_CAPACITY(cond, ...)                                              \
  do {                                                                        \
    if (!(cond)) {                                                            \
      ::sllm::set_error(__VA_ARGS__);                                         \
      return -2;                                                              \
    }                                                                         \
  } while (0)

// Checks the launch that was just issued.
#define SLLM_LAUNCHED()                                                       \
  do {                                                                        \
    hipError_t _e = hipGetLastError();                                        \
    if (_e != hipSuccess) {                                                   \
      ::sllm::set_error("%s:%d launch failed: %s", __FILE__, __LINE__,        \
                        hipGetErrorString(_e));                               \
      return -1;                                                              \
    }                                                                         \
  } while (0)

constexpr int kWave = 64;

// --------------------------------------------------------------------------
// number formats
// --------------------------------------------------------------------------
// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// fp32 -> bf16 bits, round to nearest even, by the gfx950 conversion
// instruction (v_cvt_pk_bf16_f32; a NaN stays a NaN). pk_bf16 converts two
// values in one instruction, a in the low half.
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));
typedef float f32x2_cvt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(
      uint32_t, __builtin_convertvector((f32x2_cvt){a, b}, bf16x2_cvt));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// One OCP E4M3FN byte (selected by `sel`, 0..3 of a dword) -> fp32, using the
// gfx950 hardware conversion (exact for every finite code).
__device__ __forceinline__ float e4m3_to_f32(uint32_t dword, int sel) {
  switch (sel) {
    case 0: return __builtin_amdgcn_cvt_f32_fp8(dword, 0);
    case 1: return __builtin_amdgcn_cvt_f32_fp8(dword, 1);
    case 2: return __builtin_amdgcn_cvt_f32_fp8(dword, 2);
    default: return __builtin_amdgcn_cvt_f32_fp8(dword, 3);
  }
}

// Four fp32 values (already clamped to +-448) -> four E4M3FN bytes packed
// little-endian in a dword, round to nearest even (v_cvt_pk_fp8_f32).
__device__ __forceinline__ uint32_t f32x4_to_e4m3(float a, float b, float c,
                                                  float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// Order-preserving map of fp32 onto uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t f32_order_key(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// --------------------------------------------------------------------------
// wave64 reductions
// --------------------------------------------------------------------------

// Maxima through DPP lane moves instead of LDS shuffles (a top-k makes
// one such reduction per selected element, so their latency adds up): xor 1
// and xor 2 within quads, half-row and row mirrors (max over 16 lanes in
// every lane of a row), then row_bcast15 / row_bcast31 carry the row maxima
// up so that lane 63 holds the wave's; readlane broadcasts it. Lanes a row
// mask leaves out keep `ident`, the identity of the max.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t ident) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)ident, (int)v, CTRL,
                                               ROW_MASK, 0xF, false);
}

__device__ __forceinline__ float wave_max(float v) {
  const uint32_t ni = __float_as_uint(-INFINITY);
  v = fmaxf(v, __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v), ni)));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v), ni)));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x141>(__float_as_uint(v), ni)));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x140>(__float_as_uint(v), ni)));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x142, 0xA>(__float_as_uint(v), ni)));
  v = fmaxf(v, __uint_as_float(dpp_u32<0x143, 0xC>(__float_as_uint(v), ni)));
  return __uint_as_float(
      (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), 63));
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint64_t dpp_max_u64_step(uint64_t v) {
  const uint64_t w =
      ((uint64_t)dpp_u32<CTRL, ROW_MASK>((uint32_t)(v >> 32), 0u) << 32) |
      dpp_u32<CTRL, ROW_MASK>((uint32_t)v, 0u);
  return w > v ? w : v;
}

// Sum by the same DPP pattern (a fixed order: quads, half rows, rows, then
// rows 0+1 and 2+3, then the two halves), broadcast from lane 63.
__device__ __forceinline__ float wave_sum(float v) {
  v += __uint_as_float(dpp_u32<0xB1>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp_u32<0x4E>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp_u32<0x141>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp_u32<0x140>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp_u32<0x142, 0xA>(__float_as_uint(v), 0u));
  v += __uint_as_float(dpp_u32<0x143, 0xC>(__float_as_uint(v), 0u));
  return __uint_as_float(
      (uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), 63));
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v, 0u));
  v = max(v, dpp_u32<0x4E>(v, 0u));
  v = max(v, dpp_u32<0x141>(v, 0u));
  v = max(v, dpp_u32<0x140>(v, 0u));
  v = max(v, dpp_u32<0x142, 0xA>(v, 0u));
  v = max(v, dpp_u32<0x143, 0xC>(v, 0u));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// keys are >= 0 (0 = no candidate)
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = dpp_max_u64_step<0xB1>(v);
  v = dpp_max_u64_step<0x4E>(v);
  v = dpp_max_u64_step<0x141>(v);
  v = dpp_max_u64_step<0x140>(v);
  v = dpp_max_u64_step<0x142, 0xA>(v);
  v = dpp_max_u64_step<0x143, 0xC>(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}

// Maximum over the wave's four 16-lane rows at each row position (lanes
// l, l ^ 16, l ^ 32, l ^ 48), by gfx950's row-swap permutes: one VALU
// instruction each instead of an LDS shuffle's round trip. Given the same
// value as both operands, v_permlane16_swap returns rows (2i, 2i + 1) as
// (even, even) and (odd, odd), so the maximum of its two results is the
// pair's maximum on both rows; v_permlane32_swap does the same for the row
// pairs (0, 1) and (2, 3).
__device__ __forceinline__ float rows4_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float silu_f32(float x) {
  return x / (1.0f + expf(-x));
}

// SiLU from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, about
// 1 ulp each): x / (1 + 2^(-x log2 e)). Large negative x: the exponential
// overflows to +inf and the result is -0; large positive x: x.
__device__ __forceinline__ float silu_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float sigmoid_f32(float x) {
  return 1.0f / (1.0f + expf(-x));
}

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace sllm
