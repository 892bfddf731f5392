// Decode-regime expert GEMVs: stream only the touched experts' weight bytes.
//
// Replaces the reference's device-decode MoE (kernels/q4_device_decode.py:
// 316-339: one cuBLAS GEMV per expert projection with a host sync each,
// 3k+5 round trips per layer) with two launches over all touched experts.
// Activations stay fp32 (x is bf16, exact in fp32); weights (FP8 128x128
// block, MXFP4, or plain bf16) are dequantized in registers, so this path is the un-quantized-activation
// semantics of the reference's gemm_ex decode (oracle:
// qwen_moe.moe_layer_fp8_dequant / deepseek_moe.moe_block_forward on
// dequantized weights).
//
// Work item = (touched expert, group of output columns). A workgroup of 4
// waves owns 4 weight rows per wave; lane l reads 16-byte chunks
// l, l+64, ... of each row (coalesced 1 KB per wave instruction), converts
// them with the gfx950 fp8/fp4 conversions and accumulates dot products
// against up to 4 activation rows at a time; a wave reduction finishes each
// dot. gemv1 pairs gate row n with up row n in the same wave so SwiGLU is
// applied before anything leaves registers.
#include "launch.h"

namespace sllm {

// WF_F32: fp32 weight rows (sllm_gemm_ex's fp32 GEMV; no scales)
enum WFmt { WF_FP8_BLOCK = 0, WF_MXFP4 = 1, WF_BF16 = 2, WF_F32 = 3 };

typedef float f32x2 __attribute__((ext_vector_type(2)));

template <int WF>
struct ChunkK {  // K values in one 16-byte chunk of a weight row
  static constexpr int value =
      WF == WF_FP8_BLOCK ? 16 : (WF == WF_MXFP4 ? 32 : (WF == WF_F32 ? 4 : 8));
};

// Dequantized chunk of one weight row: KPC values, already scaled.
template <int WF>
__device__ __forceinline__ void load_w_chunk(const uint8_t* row, int k0,
                                             float scale,
                                             float (&w)[ChunkK<WF>::value]) {
  if constexpr (WF == WF_FP8_BLOCK) {
    const uint4 r = *(const uint4*)(row + k0);
    const uint32_t d[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(d[i], false);
      const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(d[i], true);
      w[4 * i] = lo.x * scale;
      w[4 * i + 1] = lo.y * scale;
      w[4 * i + 2] = hi.x * scale;
      w[4 * i + 3] = hi.y * scale;
    }
  } else if constexpr (WF == WF_MXFP4) {
    // e2m1 * 2^(b - 127) is exact in bf16: v_cvt_scalef32_pk_bf16_fp4 makes
    // two values per instruction (it reads only the exponent of its scale
    // operand, so a zero scale zeroes the data instead; a NaN scale gives
    // NaN), then they are widened to fp32
    const uint4 r = *(const uint4*)(row + k0 / 2);
    const uint32_t d[4] = {r.x, r.y, r.z, r.w};
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t di = scale == 0.f ? 0u : d[i];
      const uint32_t p[4] = {
          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(di, scale, 0)),
          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(di, scale, 1)),
          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(di, scale, 2)),
          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(di, scale, 3))};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w[8 * i + 2 * j] = __uint_as_float(p[j] << 16);
        w[8 * i + 2 * j + 1] = __uint_as_float(p[j] & 0xFFFF0000u);
      }
    }
  } else if constexpr (WF == WF_F32) {
    (void)scale;
    const float4 r = *(const float4*)(row + 4 * k0);
    w[0] = r.x; w[1] = r.y; w[2] = r.z; w[3] = r.w;
  } else {
    (void)scale;
    const uint4 r = *(const uint4*)(row + 2 * k0);
    const uint32_t d[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[2 * i] = __uint_as_float(d[i] << 16);
      w[2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
    }
  }
}

template <typename TA, int N>
__device__ __forceinline__ void load_act(const TA* p, float (&a)[N]) {
  if constexpr (sizeof(TA) == 2) {
#pragma unroll
    for (int q = 0; q < N; q += 8) {
      const uint4 r = *(const uint4*)(p + q);
      const uint32_t d[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[q + 2 * i] = __uint_as_float(d[i] << 16);
        a[q + 2 * i + 1] = __uint_as_float(d[i] & 0xFFFF0000u);
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < N; q += 4) {
      const float4 r = *(const float4*)(p + q);
      a[q] = r.x; a[q + 1] = r.y; a[q + 2] = r.z; a[q + 3] = r.w;
    }
  }
}

// Weight scale of (row n, K offset k0) for the chunk.
template <int WF>
__device__ __forceinline__ float w_scale(const void* s, size_t e, int n, int k0,
                                         int N, int K) {
  if constexpr (WF == WF_BF16 || WF == WF_F32) {
    return 1.f;
  } else if constexpr (WF == WF_FP8_BLOCK) {
    const int KB = K / 128, NB = N / 128;
    return ((const float*)s)[(e * NB + n / 128) * KB + k0 / 128];
  } else {
    const uint8_t b = ((const uint8_t*)s)[(e * N + n) * (size_t)(K / 32) + k0 / 32];
    // loader convention (loaders/fp8.py:145-156): 0x00 -> 0, 0xFF -> NaN
    return b == 0 ? 0.f : (b == 255 ? __uint_as_float(0x7FC00000u)
                                    : __uint_as_float((uint32_t)b << 23));
  }
}

// SWIGLU = 1: rows (gate n, gate n+1, up n, up n+1) per wave, output h.
// SWIGLU = 0: rows n..n+3 per wave of one weight, output y * row weight.
template <int WF, typename TA, int SWIGLU>
__global__ __launch_bounds__(256) void moe_gemv_kernel(
    const TA* __restrict__ act, int gather_tokens,
    const int* __restrict__ sorted_idx, int topk, int total_rows,
    const int* __restrict__ tile_info, const int* __restrict__ num_tiles,
    const int* __restrict__ offsets, const uint8_t* __restrict__ w0,
    const void* __restrict__ s0, const uint8_t* __restrict__ w1,
    const void* __restrict__ s1, int N, int K,
    const float* __restrict__ row_w, float limit, float* __restrict__ out) {
  constexpr int KPC = ChunkK<WF>::value;  // K values per 16-byte chunk
  int e, row_begin, rows;
  if (tile_info) {
    const int tile = blockIdx.y;
    if (tile >= *num_tiles) return;
    const int4 d = *(const int4*)(tile_info + 4 * tile);
    e = d.x;
    row_begin = d.y;
    rows = d.z;
  } else {
    e = 0;
    row_begin = 0;
    rows = total_rows;
  }
  if (rows <= 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // weight rows of this wave
  const uint8_t* wrow[4];
  const void* srow[4];
  int nrow[4];
  const size_t rb = WF == WF_FP8_BLOCK ? (size_t)K
                    : (WF == WF_MXFP4 ? (size_t)K / 2
                                      : (WF == WF_F32 ? (size_t)K * 4 : (size_t)K * 2));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (SWIGLU) {
      nrow[i] = blockIdx.x * 8 + wave * 2 + (i & 1);
      const uint8_t* base = i < 2 ? w0 : w1;
      wrow[i] = base + ((size_t)e * N + nrow[i]) * rb;
      srow[i] = i < 2 ? s0 : s1;
    } else {
      nrow[i] = blockIdx.x * 16 + wave * 4 + i;
      wrow[i] = w0 + ((size_t)e * N + nrow[i]) * rb;
      srow[i] = s0;
    }
  }
  const int nch = K / KPC;
  for (int r0 = 0; r0 < rows; r0 += 4) {
    const int nr = min(4, rows - r0);
    const TA* arow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = row_begin + r0 + min(r, nr - 1);
      const int ai = (gather_tokens && sorted_idx) ? sorted_idx[pos] / topk : pos;
      arow[r] = act + (size_t)ai * K;
    }
    float part[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[i][r] = 0.f;
    for (int c = lane; c < nch; c += 64) {
      const int k0 = c * KPC;
      float wv[4][KPC];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        load_w_chunk<WF>(wrow[i], k0,
                         w_scale<WF>(srow[i], e, nrow[i], k0, N, K), wv[i]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (r < nr) {
          float a[KPC];
          load_act<TA, KPC>(arow[r] + k0, a);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float d = 0.f;
#pragma unroll
            for (int q = 0; q < KPC; ++q) d = fmaf(a[q], wv[i][q], d);
            part[i][r] += d;
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[i][r] = wave_sum(part[i][r]);
    // every lane holds the reduced sums; lane q*4+r writes output (q, r)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (lane == q * 4 + r && r < nr && (!SWIGLU || q < 2)) {
          const int pos = row_begin + r0 + r;
          if (SWIGLU) {
            float g = part[q][r], u = part[q + 2][r];
            if (limit > 0.f) {
              u = fminf(fmaxf(u, -limit), limit);
              g = fminf(g, limit);
            }
            out[(size_t)pos * N + nrow[q]] = silu_f32(g) * u;
          } else {
            float w = 1.f;
            if (row_w) w = row_w[sorted_idx ? sorted_idx[pos] : pos];
            out[(size_t)pos * N + nrow[q]] = part[q][r] * w;
          }
        }
      }
    }
  }
}

// Launch helper. act: bf16 (act_bf16=1) or fp32 rows; gather_tokens=1 maps a
// permuted row to its token (sorted_idx / topk).
int launch_gemv(int wf, int swiglu, const void* act, int act_bf16,
                int gather_tokens, const int* sorted_idx, int topk,
                int total_rows, const int* tile_info, const int* num_tiles,
                int max_tiles, const int* offsets, const uint8_t* w0,
                const void* s0, const uint8_t* w1, const void* s1, int N,
                int K, const float* row_w, float limit, float* out,
                hipStream_t st) {
  SLLM_REQUIRE(wf >= 0 && wf <= 3, "gemv: bad weight format %d", wf);
  const int kpc = wf == WF_FP8_BLOCK ? 16 : (wf == WF_MXFP4 ? 32 : (wf == WF_F32 ? 4 : 8));
  SLLM_REQUIRE(K % kpc == 0 && K > 0 && N > 0,
               "gemv: K must be a multiple of %d (K=%d)", kpc, K);
  SLLM_REQUIRE(wf != WF_FP8_BLOCK || (K % 128 == 0 && N % 128 == 0),
               "gemv: fp8 block weights need N, K multiples of 128");
  SLLM_REQUIRE(N % (swiglu ? 8 : 16) == 0, "gemv: N=%d not tileable", N);
  const int tiles = tile_info ? max_tiles : 1;
  if (tiles <= 0 || (!tile_info && total_rows <= 0)) return 0;
  dim3 grid(N / (swiglu ? 8 : 16), tiles);
#define GO(WF_, TA_, SW_)                                                     \
  moe_gemv_kernel<WF_, TA_, SW_><<<grid, 256, 0, st>>>(                       \
      (const TA_*)act, gather_tokens, sorted_idx, topk, total_rows,           \
      tile_info, num_tiles, offsets, w0, s0, w1, s1, N, K, row_w, limit, out)
  if (wf == WF_FP8_BLOCK) {
    if (act_bf16) {
      if (swiglu) GO(WF_FP8_BLOCK, uint16_t, 1); else GO(WF_FP8_BLOCK, uint16_t, 0);
    } else {
      if (swiglu) GO(WF_FP8_BLOCK, float, 1); else GO(WF_FP8_BLOCK, float, 0);
    }
  } else if (wf == WF_BF16) {
    if (act_bf16) {
      if (swiglu) GO(WF_BF16, uint16_t, 1); else GO(WF_BF16, uint16_t, 0);
    } else {
      if (swiglu) GO(WF_BF16, float, 1); else GO(WF_BF16, float, 0);
    }
  } else if (wf == WF_F32) {
    SLLM_REQUIRE(!swiglu && !act_bf16, "gemv: fp32 weights take fp32 rows, no SwiGLU");
    GO(WF_F32, float, 0);
  } else {
    if (act_bf16) {
      if (swiglu) GO(WF_MXFP4, uint16_t, 1); else GO(WF_MXFP4, uint16_t, 0);
    } else {
      if (swiglu) GO(WF_MXFP4, float, 1); else GO(WF_MXFP4, float, 0);
    }
  }
#undef GO
  SLLM_LAUNCHED();
  return 0;
}

}  // namespace sllm
