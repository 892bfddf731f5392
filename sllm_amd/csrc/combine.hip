// Weighted combine (unpermute) and the reference's elementwise MoE helpers.
//
// combine: out[t] = sum_{j ascending} y[inv_pos[t*k + j]] + y_shared[t],
// the order of ref/qwen4_exp.py:175-183 (routed slots, then the gated shared
// expert; the routing weight / shared gate were folded into y by the down
// GEMM's epilogue). One workgroup per token, 16-byte vector loads.
//
// Compat helpers replace kernels/cuda/qwen4.cu:301-382 and :795-814
// (sllm_q4_swiglu, sllm_q4_axpy_rows, sllm_q4_shared_gate_accum and their
// _dev variants) with the same names, argument meaning and error codes.
#include "launch.h"

namespace sllm {

template <typename TY>
__device__ __forceinline__ void load8(const TY* p, float (&v)[8]);

template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p,
                                                float (&v)[8]) {
  const uint4 r = *(const uint4*)p;
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
  }
}

template <>
__device__ __forceinline__ void load8<float>(const float* p, float (&v)[8]) {
  const float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// TY: bf16 (uint16_t) or fp32 expert rows; out bf16 or fp32.
template <typename TY>
__global__ __launch_bounds__(1024) void combine_kernel(
    const TY* __restrict__ y, const int* __restrict__ inv_pos, int topk,
    const TY* __restrict__ y_shared, int H, int out_f32,
    void* __restrict__ out) {
  __shared__ int pos[64];
  const int t = blockIdx.x;
  if (threadIdx.x < topk) pos[threadIdx.x] = inv_pos[(size_t)t * topk + threadIdx.x];
  __syncthreads();
  for (int c = threadIdx.x * 8; c < H; c += blockDim.x * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < topk; ++j) {
      if (pos[j] < 0) continue;  // a dropped assignment (expert id outside [0, E))
      float v[8];
      load8<TY>(y + (size_t)pos[j] * H + c, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += v[i];
    }
    if (y_shared) {
      float v[8];
      load8<TY>(y_shared + (size_t)t * H + c, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += v[i];
    }
    if (out_f32) {
      float* o = (float*)out + (size_t)t * H + c;
      *(float4*)o = make_float4(acc[0], acc[1], acc[2], acc[3]);
      *(float4*)(o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = pk_bf16(acc[2 * i], acc[2 * i + 1]);
      *(uint4*)((uint16_t*)out + (size_t)t * H + c) =
          make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

// fp32 rows (the decode paths), possibly as ks K-chunk slices (split-K).
// A workgroup covers 256 columns of one token (so that a few tokens still
// spread over many CUs); its 4 waves take every 4th of the topk * ks routed
// slices and the ks_sh shared ones (slot-major, then K slice, then shared),
// issue them in batches of 8 independent loads, and the 4 wave sums are
// added in wave order through LDS: a fixed order for every call.
constexpr int CF_WAVES = 4;
constexpr int CF_COLS = 256;
constexpr int CF_BATCH = 8;

__global__ __launch_bounds__(64 * CF_WAVES) void combine_f32_kernel(
    const float* __restrict__ y, const int* __restrict__ inv_pos, int topk,
    const float* __restrict__ y_shared, int H, int out_f32,
    void* __restrict__ out, int ks, long kstride, int ks_sh,
    long kstride_sh) {
  __shared__ int pos[64];
  __shared__ float4 part[CF_WAVES][64];
  const int t = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (threadIdx.x < topk)  // null inv_pos: the identity permutation
    pos[threadIdx.x] = inv_pos ? inv_pos[(size_t)t * topk + threadIdx.x]
                               : t * topk + threadIdx.x;
  __syncthreads();
  const int c = min(blockIdx.x * CF_COLS + lane * 4, H - 4);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  const int nr = topk * ks, nsl = nr + (y_shared ? ks_sh : 0);
  for (int b = wave; b < nsl; b += CF_WAVES * CF_BATCH) {
    float4 v[CF_BATCH];
#pragma unroll
    for (int u = 0; u < CF_BATCH; ++u) {
      const int sl = min(b + u * CF_WAVES, nsl - 1);
      // a dropped assignment (expert id outside [0, E)) has position -1: it
      // reads row 0 and is not added
      const float* src =
          sl < nr ? y + (sl % ks) * kstride + (size_t)max(pos[sl / ks], 0) * H
                  : y_shared + (sl - nr) * kstride_sh + (size_t)t * H;
      v[u] = *(const float4*)(src + c);
    }
#pragma unroll
    for (int u = 0; u < CF_BATCH; ++u) {
      const int sl = b + u * CF_WAVES;
      if (sl < nsl && (sl >= nr || pos[sl / ks] >= 0)) {
        acc.x += v[u].x;
        acc.y += v[u].y;
        acc.z += v[u].z;
        acc.w += v[u].w;
      }
    }
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0 || blockIdx.x * CF_COLS + lane * 4 >= H) return;
#pragma unroll
  for (int w = 1; w < CF_WAVES; ++w) {
    const float4 q = part[w][lane];
    acc.x += q.x;
    acc.y += q.y;
    acc.z += q.z;
    acc.w += q.w;
  }
  if (out_f32) {
    *(float4*)((float*)out + (size_t)t * H + c) = acc;
  } else {
    *(uint2*)((uint16_t*)out + (size_t)t * H + c) =
        make_uint2(pk_bf16(acc.x, acc.y), pk_bf16(acc.z, acc.w));
  }
}

int launch_combine(const void* y, int y_f32, const int* inv_pos, int topk,
                   const void* y_shared, int T, int H, int out_f32, void* out,
                   hipStream_t st) {
  SLLM_REQUIRE(y && inv_pos && out, "combine: null pointer");
  SLLM_REQUIRE(T > 0 && H % 8 == 0 && topk > 0 && topk <= 64,
               "combine: bad sizes (T=%d H=%d k=%d)", T, H, topk);
  if (y_f32)
    return launch_combine_split((const float*)y, inv_pos, topk,
                                (const float*)y_shared, T, H, out_f32, out, 1,
                                0, 1, 0, st);
  else
    // one pass over the row: H / 8 threads (a whole number of waves, at
    // most 1024) of eight columns each (C4, H 7168: 896 threads; with 256,
    // the fourth pass had half of them idle and the launch took 249 against
    // 234 us)
    combine_kernel<uint16_t><<<T, std::min(1024, (H / 8 + 63) / 64 * 64), 0, st>>>(
        (const uint16_t*)y, inv_pos, topk, (const uint16_t*)y_shared, H,
        out_f32, out);
  SLLM_LAUNCHED();
  return 0;
}

int launch_combine_split(const float* y, const int* inv_pos, int topk,
                         const float* y_shared, int T, int H, int out_f32,
                         void* out, int ks, long kstride, int ks_sh,
                         long kstride_sh, hipStream_t st) {
  SLLM_REQUIRE(y && out, "combine: null pointer");
  SLLM_REQUIRE(T > 0 && T < 65536 && H % 4 == 0 && H >= 4 && topk > 0 &&
                   topk <= 64 &&
                   ks >= 1 && ks_sh >= 1 && kstride % 4 == 0 &&
                   kstride_sh % 4 == 0,
               "combine: bad sizes (T=%d H=%d k=%d ks=%d/%d)", T, H, topk, ks,
               ks_sh);
  const dim3 grid((H + CF_COLS - 1) / CF_COLS, T);
  combine_f32_kernel<<<grid, 64 * CF_WAVES, 0, st>>>(y, inv_pos, topk, y_shared,
                                                  H, out_f32, out, ks, kstride,
                                                  ks_sh, kstride_sh);
  SLLM_LAUNCHED();
  return 0;
}

// ---------------------------------------------------------------------------
// reference elementwise helpers (fp32)
// ---------------------------------------------------------------------------
__global__ void swiglu_elem_kernel(const float* __restrict__ g,
                                   const float* __restrict__ u,
                                   float* __restrict__ out, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = silu_f32(g[i]) * u[i];
}

__global__ void silu_mul_kernel(const float* __restrict__ g,
                                const float* __restrict__ u,
                                void* __restrict__ out, long n, int bf16) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = silu_f32(g[i]) * u[i];
  if (bf16) ((uint16_t*)out)[i] = f32_to_bf16(v);
  else ((float*)out)[i] = v;
}

__global__ void axpy_rows_kernel(float* __restrict__ out,
                                 const float* __restrict__ y,
                                 const float* __restrict__ w, int n, int H) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)n * H) return;
  out[i] += w[i / H] * y[i];
}

__global__ void shared_gate_kernel(float* __restrict__ out,
                                   const float* __restrict__ sh,
                                   const float* __restrict__ g, int n, int H) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)n * H) return;
  out[i] += sigmoid_f32(g[i / H]) * sh[i];
}

static unsigned blocks_for(long n) { return (unsigned)((n + 255) / 256); }

}  // namespace sllm

using namespace sllm;

namespace {

// Host-pointer helper: allocate device copies, run, copy back, free.
struct DevTmp {
  void* p = nullptr;
  ~DevTmp() {
    if (p) (void)hipFree(p);
  }
};

int h2d_tmp(DevTmp& d, const void* src, size_t n) {
  SLLM_HIP(hipMalloc(&d.p, n ? n : 4));
  if (src && n) SLLM_HIP(hipMemcpy(d.p, src, n, hipMemcpyHostToDevice));
  return 0;
}

}  // namespace

extern "C" {

int sllm_moe_combine(const void* y, int y_f32, const int* inv_pos, int topk,
                     const void* y_shared, int T, int H, int out_f32,
                     void* out, void* stream) {
  return launch_combine(y, y_f32, inv_pos, topk, y_shared, T, H, out_f32, out,
                        (hipStream_t)stream);
}

// ref: kernels/cuda/qwen4.cu:308-320
int sllm_q4_swiglu(const float* g, const float* u, float* out, long n) {
  SLLM_REQUIRE(g && u && out && n >= 0, "sllm_q4_swiglu: bad args");
  if (n == 0) return 0;
  DevTmp dg, du, dout;
  const size_t nb = (size_t)n * sizeof(float);
  if (h2d_tmp(dg, g, nb) || h2d_tmp(du, u, nb) || h2d_tmp(dout, nullptr, nb))
    return -1;
  swiglu_elem_kernel<<<blocks_for(n), 256>>>((float*)dg.p, (float*)du.p,
                                             (float*)dout.p, n);
  SLLM_LAUNCHED();
  SLLM_HIP(hipMemcpy(out, dout.p, nb, hipMemcpyDeviceToHost));
  return 0;
}

// ref: kernels/cuda/qwen4.cu:795-799
int sllm_q4_swiglu_dev(const float* g, const float* u, float* out, long n) {
  SLLM_REQUIRE(g && u && out && n >= 0, "sllm_q4_swiglu_dev: bad args");
  if (n == 0) return 0;
  swiglu_elem_kernel<<<blocks_for(n), 256>>>(g, u, out, n);
  SLLM_LAUNCHED();
  return 0;
}

// ref: kernels/cuda/kernels.cu:897-919 (sllm_silu_mul): out = silu(g) * u
// from fp32 g, u, stored as fp32 (out_type 0) or bf16 (out_type 1, RNE);
// device pointers; n <= 0 does nothing.
int sllm_silu_mul(const void* g, const void* u, void* out, long n,
                  int out_type) {
  if (n <= 0) return 0;
  SLLM_REQUIRE(g && u && out, "sllm_silu_mul: null pointer");
  silu_mul_kernel<<<blocks_for(n), 256>>>((const float*)g, (const float*)u,
                                         out, n, out_type == 1);
  SLLM_LAUNCHED();
  return 0;
}

// ref: kernels/cuda/qwen4.cu:332-351
int sllm_q4_axpy_rows(float* out, const float* y, const float* w, int n,
                      int H) {
  SLLM_REQUIRE(out && y && w && n >= 0 && H >= 0, "sllm_q4_axpy_rows: bad args");
  const long tot = (long)n * H;
  if (tot == 0) return 0;
  DevTmp dout, dy, dw;
  if (h2d_tmp(dout, out, tot * 4) || h2d_tmp(dy, y, tot * 4) ||
      h2d_tmp(dw, w, (size_t)n * 4))
    return -1;
  axpy_rows_kernel<<<blocks_for(tot), 256>>>((float*)dout.p, (float*)dy.p,
                                             (float*)dw.p, n, H);
  SLLM_LAUNCHED();
  SLLM_HIP(hipMemcpy(out, dout.p, tot * 4, hipMemcpyDeviceToHost));
  return 0;
}

// ref: kernels/cuda/qwen4.cu:801-806
int sllm_q4_axpy_rows_dev(float* out, const float* y, const float* w, int n,
                          int H) {
  SLLM_REQUIRE(out && y && w && n >= 0 && H >= 0,
               "sllm_q4_axpy_rows_dev: bad args");
  const long tot = (long)n * H;
  if (tot == 0) return 0;
  axpy_rows_kernel<<<blocks_for(tot), 256>>>(out, y, w, n, H);
  SLLM_LAUNCHED();
  return 0;
}

// ref: kernels/cuda/qwen4.cu:363-382
int sllm_q4_shared_gate_accum(float* out, const float* shared, const float* g,
                              int n, int H) {
  SLLM_REQUIRE(out && shared && g && n >= 0 && H >= 0,
               "sllm_q4_shared_gate_accum: bad args");
  const long tot = (long)n * H;
  if (tot == 0) return 0;
  DevTmp dout, dsh, dg;
  if (h2d_tmp(dout, out, tot * 4) || h2d_tmp(dsh, shared, tot * 4) ||
      h2d_tmp(dg, g, (size_t)n * 4))
    return -1;
  shared_gate_kernel<<<blocks_for(tot), 256>>>((float*)dout.p, (float*)dsh.p,
                                               (float*)dg.p, n, H);
  SLLM_LAUNCHED();
  SLLM_HIP(hipMemcpy(out, dout.p, tot * 4, hipMemcpyDeviceToHost));
  return 0;
}

// ref: kernels/cuda/qwen4.cu:808-814
int sllm_q4_shared_gate_accum_dev(float* out, const float* shared,
                                  const float* g, int n, int H) {
  SLLM_REQUIRE(out && shared && g && n >= 0 && H >= 0,
               "sllm_q4_shared_gate_accum_dev: bad args");
  const long tot = (long)n * H;
  if (tot == 0) return 0;
  shared_gate_kernel<<<blocks_for(tot), 256>>>(out, shared, g, n, H);
  SLLM_LAUNCHED();
  return 0;
}

}  // extern "C"
