// Grouped block-scaled expert GEMMs for prefill-sized token counts.
//
// Replaces the per-token expert loop of ref/qwen4_exp.py:175-183, the
// per-expert loop of ref/deepseek_v4.py:1080-1086 and the reference's naive
// one-thread-per-output GEMMs (kernels/cuda/fp8.cu:51-70,
// kernels/cuda/deepseek.cu:46-55) with two grouped GEMMs over the
// expert-major permutation:
//
//   gemm1: h = silu(x W1^T) * (x W3^T) [DeepSeek: clamped by swiglu_limit and
//          times the routing weight, upstream Expert.forward], then h
//          re-quantized to e4m3 per 1x128 (the upstream quantization point
//          before the down projection, ref/hf_sources/dsv4/kernel.py:40-125);
//   gemm2: y = h W2^T [Qwen: times the routing weight / shared gate], bf16
//          rows per (token, slot) for the combine.
//
// B (weight) formats and their arithmetic:
//   BF_FP8_F32S  e4m3 with fp32 128x128 block scales (Qwen). One
//                v_mfma_f32_16x16x128_f8f6f4 per 128-wide K block forms the
//                exact fp8 x fp8 partial; acc += partial * (sa * sb) as in
//                upstream fp8_gemm (kernel.py:244-257). fp32 (non power-of-
//                two) scales cannot ride in the MFMA's e8m0 scale operand.
//   BF_FP8_POW2  e4m3 with power-of-two 128x128 block scales (DeepSeek
//                shared expert): v_mfma_scale_f32_16x16x128_f8f6f4 with the
//                e8m0 exponents of both scales; accumulation stays in the
//                MFMA accumulator for the whole K loop.
//   BF_FP4       MXFP4: e2m1 pairs with an e8m0 scale per 32 along K
//                (DeepSeek routed experts, upstream fp4_gemm kernel.py:
//                441-536), same scaled MFMA with B format e2m1.
// The activation A is always e4m3 with a per-(row, 128) scale; for the two
// MX formats that scale is a power of two (ue8m0 act_quant), so its exponent
// is exact as an e8m0 operand.
//
// Tiling (gfx950, wave64): a workgroup of 4 waves owns one tile of up to 128
// rows of ONE expert (its tokens are contiguous after the permute) and a
// slab of output columns. Each wave owns 4 column subtiles of 16 and all 8
// row subtiles: B (the weights, streamed once from HBM) goes straight from
// global memory into registers with no sharing, and A (the gathered
// activations, 16 KB per K step) is staged once in LDS for all four waves.
// Row subtiles past the expert's row count issue no MFMA. Ragged tiles come
// from the permute's tile table; the grid is the worst case and surplus
// workgroups exit at once. Consecutive column slabs of one row tile are
// mapped onto one XCD so the gathered A rows are reused from its L2.
//
// MFMA lane layout (v_mfma_*_16x16x128_f8f6f4, measured on gfx950 with
// one-hot operands): lane l supplies row (l % 16) of A and column (l % 16)
// of B. An e4m3 operand holds, in lane group g = l / 16, the K values
// [16 g, 16 g + 16) in bytes 0-15 and [64 + 16 g, 64 + 16 g + 16) in bytes
// 16-31; an e2m1 operand holds the contiguous K values [32 g, 32 g + 32)
// (low nibble first); lane group b supplies the e8m0 scale of the K block
// [32 b, 32 b + 32). fp8 x fp8 products only need both operands loaded the
// same way (their scales are uniform over the 128-wide step), so they load
// 32 contiguous bytes; fp8 x fp4 loads the A operand in the split order so
// that it pairs with the contiguous fp4 B operand and its per-32 scales.
// The 16x16 fp32 result holds row 4 (l / 16) + v, column l % 16 in element v.
#include "launch.h"

namespace sllm {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

enum BFmt { BF_FP8_F32S = 0, BF_FP8_POW2 = 1, BF_FP4 = 2 };

constexpr int G_BM = 128;          // rows per tile
constexpr int G_LDS_STRIDE = 144;  // bytes per A row in LDS (128 + 16 pad)

__device__ __forceinline__ uint32_t e8m0_of(float pow2) {
  return (__float_as_uint(pow2) >> 23) & 0xFF;
}

template <int BF>
__device__ __forceinline__ f32x4 mma(const v8i& a, const v8i& b, f32x4 c,
                                     uint32_t sa, uint32_t sb) {
  if constexpr (BF == BF_FP8_F32S) {
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0,
                                                            0, 0, 0);
  } else if constexpr (BF == BF_FP8_POW2) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
        a, b, c, 0, 0, 0, (int)sa, 0, (int)sb);
  } else {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
        a, b, c, 0, 4, 0, (int)sa, 0, (int)sb);
  }
}

// Workgroup index -> logical tile so that consecutive logical tiles land on
// the same XCD (workgroups are dispatched round-robin over the 8 XCDs).
__device__ __forceinline__ int xcd_remap(int L, int total) {
  const int per = total >> 3, rem = total & 7;
  const int xcd = L & 7, slot = L >> 3;
  return xcd < rem ? xcd * (per + 1) + slot
                   : rem * (per + 1) + (xcd - rem) * per + slot;
}

struct TileRows {
  int e, row_begin, rows;
};

// Routed: tile table from the permute. Shared (tile_info == nullptr):
// identity rows, tile i covers rows [128 i, 128 i + 128).
__device__ __forceinline__ bool resolve_tile(int tile, const int* tile_info,
                                             const int* num_tiles,
                                             const int* offsets, int total_rows,
                                             TileRows& tr) {
  if (tile_info) {
    if (tile >= *num_tiles) return false;
    const int4 d = *(const int4*)(tile_info + 4 * tile);
    tr.e = d.x;
    tr.row_begin = d.y;
    tr.rows = min(G_BM, d.z);
  } else {
    tr.e = 0;
    tr.row_begin = tile * G_BM;
    if (tr.row_begin >= total_rows) return false;
    tr.rows = min(G_BM, total_rows - tr.row_begin);
  }
  return tr.rows > 0;
}

struct AFetch {
  uint4 v[4];
};

// Cooperative A-tile fetch: thread -> (row tid/2, 64 bytes at half*64).
__device__ __forceinline__ void fetch_a(const uint8_t* src_row, bool ok,
                                        int kb, int half, AFetch& f) {
  if (ok) {
    const uint4* p = (const uint4*)(src_row + kb * 128 + half * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) f.v[i] = p[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) f.v[i] = make_uint4(0, 0, 0, 0);
  }
}

__device__ __forceinline__ void store_a(uint8_t* lds, int row, int half,
                                        const AFetch& f) {
  uint4* p = (uint4*)(lds + row * G_LDS_STRIDE + half * 64);
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = f.v[i];
}

// A operand for row subtile mi from the LDS tile: 32 contiguous bytes at
// 32 g (fp8 x fp8), or 16 bytes at 16 g and 16 at 64 + 16 g (fp8 x fp4).
template <int BF>
__device__ __forceinline__ v8i lds_a_frag(const uint8_t* lds, int mi,
                                          int lane) {
  const uint8_t* row = lds + (mi * 16 + (lane & 15)) * G_LDS_STRIDE;
  const int g = lane >> 4;
  const uint8_t* p0 = BF == BF_FP4 ? row + g * 16 : row + g * 32;
  const uint8_t* p1 = BF == BF_FP4 ? row + 64 + g * 16 : row + g * 32 + 16;
  const uint4 lo = *(const uint4*)p0, hi = *(const uint4*)p1;
  return (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
               (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

// One B subtile operand for K step kb: row pointer already at this lane's
// column and K group.
template <int BF>
__device__ __forceinline__ v8i load_b(const uint8_t* row, int kb) {
  if constexpr (BF == BF_FP4) {
    const uint4 v = *(const uint4*)(row + kb * 64);
    return (v8i){(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
  } else {
    const uint8_t* p = row + kb * 128;
    const uint4 lo = *(const uint4*)p, hi = *(const uint4*)(p + 16);
    return (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                 (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  }
}

// Geometry of one weight tensor (E, N, K) in format BF for lane addressing.
template <int BF>
__device__ __forceinline__ const uint8_t* b_row(const uint8_t* w, int e, int n,
                                                int N, int K, int lane) {
  const size_t rb = BF == BF_FP4 ? (size_t)K / 2 : (size_t)K;
  const size_t kofs = BF == BF_FP4 ? (size_t)(lane >> 4) * 16
                                   : (size_t)(lane >> 4) * 32;
  return w + ((size_t)e * N + n) * rb + kofs;
}

// ---------------------------------------------------------------------------
// gemm1: gate/up + SwiGLU (+ clamp, + routing weight) + e4m3 re-quant.
// Column slab nt covers h columns [128 nt, 128 nt + 128); wave w owns
// h columns 128 nt + 32 w + [0, 32): subtiles 0,1 = gate (W1), 2,3 = up (W3);
// the same lane holds matching gate and up values.
// ---------------------------------------------------------------------------
template <int BF>
__global__ __launch_bounds__(256, 2) void moe_gemm1_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ sx,
    const int* __restrict__ sorted_idx, int topk, int total_rows,
    const int* __restrict__ tile_info, const int* __restrict__ num_tiles,
    const int* __restrict__ offsets, const uint8_t* __restrict__ w1,
    const void* __restrict__ w1_s, const uint8_t* __restrict__ w3,
    const void* __restrict__ w3_s, int I, int H,
    const float* __restrict__ route_w, float limit, int pow2,
    uint8_t* __restrict__ hq, float* __restrict__ hs) {
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[G_BM * G_LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) float sa_lds[G_BM];
  __shared__ float red[4][G_BM];

  const int ntn = I / 128;
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = logical / ntn, nt = logical % ntn;
  TileRows tr;
  if (!resolve_tile(tile, tile_info, num_tiles, offsets, total_rows, tr))
    return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, lc = lane & 15;
  const int KB = H / 128;
  const int my_row = tid >> 1, half = tid & 1;
  const bool row_ok = my_row < tr.rows;
  int src = 0;
  if (row_ok) {
    const int pos = tr.row_begin + my_row;
    src = sorted_idx ? sorted_idx[pos] / topk : pos;
  }
  const uint8_t* a_src = xq + (size_t)src * H;
  const bool s_ok = tid < tr.rows;
  int s_src = 0;
  if (s_ok) {
    const int pos = tr.row_begin + tid;
    s_src = sorted_idx ? sorted_idx[pos] / topk : pos;
  }
  const uint8_t* bp[4];
  int bn[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bn[s] = nt * 128 + wave * 32 + (s & 1) * 16 + lc;
    bp[s] = b_row<BF>(s < 2 ? w1 : w3, tr.e, bn[s], I, H, lane);
  }
  const int nmi = (tr.rows + 15) >> 4;

  f32x4 acc[8][4];
#pragma unroll
  for (int mi = 0; mi < 8; ++mi)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[mi][s] = (f32x4){0.f, 0.f, 0.f, 0.f};

  AFetch af;
  fetch_a(a_src, row_ok, 0, half, af);
  float sa_next = s_ok ? sx[(size_t)s_src * KB] : 0.f;
  v8i b[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) b[s] = load_b<BF>(bp[s], 0);

  for (int kb = 0; kb < KB; ++kb) {
    store_a(a_lds, my_row, half, af);
    if (tid < G_BM) sa_lds[tid] = sa_next;
    __syncthreads();
    v8i bnx[4];
    if (kb + 1 < KB) {
      fetch_a(a_src, row_ok, kb + 1, half, af);
      if (s_ok) sa_next = sx[(size_t)s_src * KB + kb + 1];
#pragma unroll
      for (int s = 0; s < 4; ++s) bnx[s] = load_b<BF>(bp[s], kb + 1);
    }
    // weight scales for this K step
    float sbf[2] = {0.f, 0.f};
    uint32_t sbe[4] = {0, 0, 0, 0};
    if constexpr (BF == BF_FP4) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint8_t* sc = (const uint8_t*)(s < 2 ? w1_s : w3_s);
        sbe[s] = sc[((size_t)tr.e * I + bn[s]) * (H / 32) + kb * 4 + lg];
      }
    } else {
      const float* sg = (const float*)w1_s + ((size_t)tr.e * ntn + nt) * KB;
      const float* su = (const float*)w3_s + ((size_t)tr.e * ntn + nt) * KB;
      sbf[0] = sg[kb];
      sbf[1] = su[kb];
#pragma unroll
      for (int s = 0; s < 4; ++s) sbe[s] = e8m0_of(sbf[s >> 1]);
    }
#pragma unroll
    for (int mi = 0; mi < 8; ++mi) {
      if (mi < nmi) {
        const v8i a = lds_a_frag<BF>(a_lds, mi, lane);
        if constexpr (BF == BF_FP8_F32S) {
          const float4 sav =
              *(const float4*)(sa_lds + mi * 16 + lg * 4);
          const float sv[4] = {sav.x, sav.y, sav.z, sav.w};
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const f32x4 p = mma<BF>(a, b[s], acc[mi][s], 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v)
              acc[mi][s][v] = fmaf(p[v], sv[v] * sbf[s >> 1], acc[mi][s][v]);
          }
        } else {
          const uint32_t sae = e8m0_of(sa_lds[mi * 16 + lc]);
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc[mi][s] = mma<BF>(a, b[s], acc[mi][s], sae, sbe[s]);
        }
      }
    }
    __syncthreads();
    if (kb + 1 < KB) {
#pragma unroll
      for (int s = 0; s < 4; ++s) b[s] = bnx[s];
    }
  }

  // ---- epilogue: SwiGLU, per-row amax over the 128 h columns, re-quant ----
#pragma unroll
  for (int mi = 0; mi < 8; ++mi) {
    if (mi < nmi) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = mi * 16 + lg * 4 + v;
        float rw = 1.f;
        if (route_w && r < tr.rows) rw = route_w[sorted_idx[tr.row_begin + r]];
        float amax = 0.f;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          float g = acc[mi][s][v], u = acc[mi][s + 2][v];
          if (limit > 0.f) {
            u = fminf(fmaxf(u, -limit), limit);
            g = fminf(g, limit);
          }
          const float h = silu_f32(g) * u * rw;
          acc[mi][s][v] = h;
          amax = fmaxf(amax, fabsf(h));
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1)
          amax = fmaxf(amax, __shfl_xor(amax, o, 16));
        if (lc == 0) red[wave][r] = amax;
      }
    }
  }
  __syncthreads();
  uint8_t* h_lds = a_lds;  // reuse the A tile buffer for the e4m3 h tile
#pragma unroll
  for (int mi = 0; mi < 8; ++mi) {
    if (mi < nmi) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = mi * 16 + lg * 4 + v;
        const float amax =
            fmaxf(fmaxf(red[0][r], red[1][r]), fmaxf(red[2][r], red[3][r]));
        float sc = fmaxf(amax, 1e-4f) * (1.0f / 448.0f);
        if (pow2) {
          const uint32_t bits = __float_as_uint(sc);
          const int ex =
              (int)((bits >> 23) & 0xFF) - 127 + ((bits & 0x7FFFFF) ? 1 : 0);
          sc = __uint_as_float((uint32_t)(ex + 127) << 23);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const float y = fminf(fmaxf(acc[mi][s][v] / sc, -448.f), 448.f);
          h_lds[r * G_LDS_STRIDE + wave * 32 + s * 16 + lc] =
              (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(y, 0.f, 0, false) & 0xFF);
        }
        if (wave == 0 && lc == 0 && r < tr.rows)
          hs[(size_t)(tr.row_begin + r) * ntn + nt] = sc;
      }
    }
  }
  __syncthreads();
  if (row_ok) {
    const uint4* p = (const uint4*)(h_lds + my_row * G_LDS_STRIDE + half * 64);
    uint4* dst = (uint4*)(hq + (size_t)(tr.row_begin + my_row) * I + nt * 128 +
                          half * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = p[i];
  }
}

// ---------------------------------------------------------------------------
// gemm2: y = h W2^T (K = I), times a per-row weight (routing weight or shared
// gate, optional), stored bf16. Column slab nt covers output columns
// [256 nt, 256 nt + 256); wave w owns 64 of them (4 subtiles), all inside one
// 128-column weight-scale block.
// ---------------------------------------------------------------------------
template <int BF>
__global__ __launch_bounds__(256, 2) void moe_gemm2_kernel(
    const uint8_t* __restrict__ hq, const float* __restrict__ hs,
    const int* __restrict__ sorted_idx, int total_rows,
    const int* __restrict__ tile_info, const int* __restrict__ num_tiles,
    const int* __restrict__ offsets, const uint8_t* __restrict__ w2,
    const void* __restrict__ w2_s, int I, int H,
    const float* __restrict__ row_w, uint16_t* __restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[G_BM * G_LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) float sa_lds[G_BM];

  const int ntn = H / 256;
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = logical / ntn, nt = logical % ntn;
  TileRows tr;
  if (!resolve_tile(tile, tile_info, num_tiles, offsets, total_rows, tr))
    return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, lc = lane & 15;
  const int KB = I / 128;
  const int my_row = tid >> 1, half = tid & 1;
  const bool row_ok = my_row < tr.rows;
  const uint8_t* a_src =
      hq + (size_t)(tr.row_begin + (row_ok ? my_row : 0)) * I;
  const bool s_ok = tid < tr.rows;
  const float* s_src = hs + (size_t)(tr.row_begin + (s_ok ? tid : 0)) * KB;

  const uint8_t* bp[4];
  int bn[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bn[s] = nt * 256 + wave * 64 + s * 16 + lc;
    bp[s] = b_row<BF>(w2, tr.e, bn[s], H, I, lane);
  }
  const int nblk = (nt * 256 + wave * 64) / 128;
  const int nmi = (tr.rows + 15) >> 4;

  f32x4 acc[8][4];
#pragma unroll
  for (int mi = 0; mi < 8; ++mi)
#pragma unroll
    for (int s = 0; s < 4; ++s) acc[mi][s] = (f32x4){0.f, 0.f, 0.f, 0.f};

  AFetch af;
  fetch_a(a_src, row_ok, 0, half, af);
  float sa_next = s_ok ? s_src[0] : 0.f;
  v8i b[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) b[s] = load_b<BF>(bp[s], 0);

  for (int kb = 0; kb < KB; ++kb) {
    store_a(a_lds, my_row, half, af);
    if (tid < G_BM) sa_lds[tid] = sa_next;
    __syncthreads();
    v8i bnx[4];
    if (kb + 1 < KB) {
      fetch_a(a_src, row_ok, kb + 1, half, af);
      if (s_ok) sa_next = s_src[kb + 1];
#pragma unroll
      for (int s = 0; s < 4; ++s) bnx[s] = load_b<BF>(bp[s], kb + 1);
    }
    float sbf = 0.f;
    uint32_t sbe[4] = {0, 0, 0, 0};
    if constexpr (BF == BF_FP4) {
      const uint8_t* sc = (const uint8_t*)w2_s;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        sbe[s] = sc[((size_t)tr.e * H + bn[s]) * (I / 32) + kb * 4 + lg];
    } else {
      sbf = ((const float*)w2_s)[((size_t)tr.e * (H / 128) + nblk) * KB + kb];
#pragma unroll
      for (int s = 0; s < 4; ++s) sbe[s] = e8m0_of(sbf);
    }
#pragma unroll
    for (int mi = 0; mi < 8; ++mi) {
      if (mi < nmi) {
        const v8i a = lds_a_frag<BF>(a_lds, mi, lane);
        if constexpr (BF == BF_FP8_F32S) {
          const float4 sav = *(const float4*)(sa_lds + mi * 16 + lg * 4);
          const float c[4] = {sav.x * sbf, sav.y * sbf, sav.z * sbf,
                              sav.w * sbf};
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const f32x4 p = mma<BF>(a, b[s], acc[mi][s], 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v)
              acc[mi][s][v] = fmaf(p[v], c[v], acc[mi][s][v]);
          }
        } else {
          const uint32_t sae = e8m0_of(sa_lds[mi * 16 + lc]);
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc[mi][s] = mma<BF>(a, b[s], acc[mi][s], sae, sbe[s]);
        }
      }
    }
    __syncthreads();
    if (kb + 1 < KB) {
#pragma unroll
      for (int s = 0; s < 4; ++s) b[s] = bnx[s];
    }
  }

#pragma unroll
  for (int mi = 0; mi < 8; ++mi) {
    if (mi < nmi) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int r = mi * 16 + lg * 4 + v;
        if (r < tr.rows) {
          const int pos = tr.row_begin + r;
          float w = 1.f;
          if (row_w) w = row_w[sorted_idx ? sorted_idx[pos] : pos];
          uint16_t* dst = y + (size_t)pos * H + nt * 256 + wave * 64 + lc;
#pragma unroll
          for (int s = 0; s < 4; ++s)
            dst[s * 16] = f32_to_bf16(acc[mi][s][v] * w);
        }
      }
    }
  }
}

template <int BF>
static int go_gemm1(const uint8_t* xq, const float* sx, const int* sorted_idx,
                    int topk, int total_rows, const int* tile_info,
                    const int* num_tiles, int max_tiles, const int* offsets,
                    const uint8_t* w1, const void* w1_s, const uint8_t* w3,
                    const void* w3_s, int I, int H, const float* route_w,
                    float limit, int pow2, uint8_t* hq, float* hs,
                    hipStream_t st) {
  SLLM_REQUIRE(xq && sx && w1 && w1_s && w3 && w3_s && hq && hs,
               "gemm1: null pointer");
  SLLM_REQUIRE(I % 128 == 0 && H % 128 == 0 && I > 0 && H > 0,
               "gemm1: need I, H multiples of 128 (I=%d H=%d)", I, H);
  SLLM_REQUIRE(!route_w || sorted_idx, "gemm1: route_w needs sorted_idx");
  const int tiles = tile_info ? max_tiles : ceil_div(total_rows, G_BM);
  if (tiles <= 0) return 0;
  const long grid = (long)tiles * (I / 128);
  SLLM_REQUIRE(grid < (1L << 31), "gemm1: grid too large");
  moe_gemm1_kernel<BF><<<(unsigned)grid, 256, 0, st>>>(
      xq, sx, sorted_idx, topk, total_rows, tile_info, num_tiles, offsets, w1,
      w1_s, w3, w3_s, I, H, route_w, limit, pow2, hq, hs);
  SLLM_LAUNCHED();
  return 0;
}

template <int BF>
static int go_gemm2(const uint8_t* hq, const float* hs, const int* sorted_idx,
                    int total_rows, const int* tile_info, const int* num_tiles,
                    int max_tiles, const int* offsets, const uint8_t* w2,
                    const void* w2_s, int I, int H, const float* row_w,
                    uint16_t* y, hipStream_t st) {
  SLLM_REQUIRE(hq && hs && w2 && w2_s && y, "gemm2: null pointer");
  SLLM_REQUIRE(I % 128 == 0 && H % 256 == 0 && I > 0 && H > 0,
               "gemm2: need I %% 128 == 0 and H %% 256 == 0 (I=%d H=%d)", I,
               H);
  const int tiles = tile_info ? max_tiles : ceil_div(total_rows, G_BM);
  if (tiles <= 0) return 0;
  const long grid = (long)tiles * (H / 256);
  SLLM_REQUIRE(grid < (1L << 31), "gemm2: grid too large");
  moe_gemm2_kernel<BF><<<(unsigned)grid, 256, 0, st>>>(
      hq, hs, sorted_idx, total_rows, tile_info, num_tiles, offsets, w2, w2_s,
      I, H, row_w, y);
  SLLM_LAUNCHED();
  return 0;
}

int launch_gemm1_fp8(const uint8_t* xq, const float* sx, const int* sorted_idx,
                     int topk, int total_rows, const int* tile_info,
                     const int* num_tiles, int max_tiles, const int* offsets,
                     const uint8_t* wg, const float* wg_s, const uint8_t* wu,
                     const float* wu_s, int I, int H, const float* route_w,
                     float limit, int pow2, uint8_t* hq, float* hs,
                     hipStream_t st) {
  return go_gemm1<BF_FP8_F32S>(xq, sx, sorted_idx, topk, total_rows, tile_info,
                               num_tiles, max_tiles, offsets, wg, wg_s, wu,
                               wu_s, I, H, route_w, limit, pow2, hq, hs, st);
}

int launch_gemm2_fp8(const uint8_t* hq, const float* hs, const int* sorted_idx,
                     int topk, int total_rows, const int* tile_info,
                     const int* num_tiles, int max_tiles, const int* offsets,
                     const uint8_t* wd, const float* wd_s, int I, int H,
                     const float* row_w, uint16_t* y, hipStream_t st) {
  (void)topk;
  return go_gemm2<BF_FP8_F32S>(hq, hs, sorted_idx, total_rows, tile_info,
                               num_tiles, max_tiles, offsets, wd, wd_s, I, H,
                               row_w, y, st);
}

int launch_gemm1_mx(int b_fp4, const uint8_t* xq, const float* sx,
                    const int* sorted_idx, int topk, int total_rows,
                    const int* tile_info, const int* num_tiles, int max_tiles,
                    const int* offsets, const uint8_t* w1, const void* w1_s,
                    const uint8_t* w3, const void* w3_s, int I, int H,
                    const float* route_w, float limit, uint8_t* hq, float* hs,
                    hipStream_t st) {
  if (b_fp4)
    return go_gemm1<BF_FP4>(xq, sx, sorted_idx, topk, total_rows, tile_info,
                            num_tiles, max_tiles, offsets, w1, w1_s, w3, w3_s,
                            I, H, route_w, limit, 1, hq, hs, st);
  return go_gemm1<BF_FP8_POW2>(xq, sx, sorted_idx, topk, total_rows, tile_info,
                               num_tiles, max_tiles, offsets, w1, w1_s, w3,
                               w3_s, I, H, route_w, limit, 1, hq, hs, st);
}

int launch_gemm2_mx(int b_fp4, const uint8_t* hq, const float* hs,
                    const int* sorted_idx, int topk, int total_rows,
                    const int* tile_info, const int* num_tiles, int max_tiles,
                    const int* offsets, const uint8_t* w2, const void* w2_s,
                    int I, int H, uint16_t* y, hipStream_t st) {
  (void)topk;
  if (b_fp4)
    return go_gemm2<BF_FP4>(hq, hs, sorted_idx, total_rows, tile_info,
                            num_tiles, max_tiles, offsets, w2, w2_s, I, H,
                            nullptr, y, st);
  return go_gemm2<BF_FP8_POW2>(hq, hs, sorted_idx, total_rows, tile_info,
                               num_tiles, max_tiles, offsets, w2, w2_s, I, H,
                               nullptr, y, st);
}

}  // namespace sllm
