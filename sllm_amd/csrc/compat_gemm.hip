// Reference-compatible standalone GEMM entry points.
//
//   sllm_fp8_gemm(_dev)   ref kernels/cuda/fp8.cu:72-110
//   sllm_ds_fp4_gemm      ref kernels/cuda/deepseek.cu:57-73
//   sllm_gemm_ex          ref kernels/cuda/kernels.cu:752-767 (cublasGemmEx)
//   sllm_ds_fp4_gemm_packed  new: packed E2M1 + E8M0 weights on the device
//                         (the reference dequantizes FP4 on the host,
//                         kernels/_deepseek_cuda.py:89-94)
//
// All compute C (M, N) fp32 = A (M, K) . B(N, K)^T with fp32 accumulation.
// Scale orientation for the FP8 weight follows loaders/fp8.py:98-135 and the
// reference's own test (tests/test_fp8_gemm.py:49-55: the kernel must equal
// A @ dequant_weight_blocked(B, scale).T): scale_inv has shape
// (ceil(N/bh), ceil(K/bw)) and W[n, k] = e4m3(B[n, k]) * scale_inv[n/bh,
// k/bw]. The reference kernel's K-block-major index (fp8.cu:66) contradicts
// that contract; the contract is what is implemented.
//
// These are parity surfaces, not the layer's hot path: a 32x32 LDS-tiled
// fp32 kernel with on-the-fly dequantization of B (bf16 gemm_ex with
// k % 128 == 0 takes the MFMA router kernels instead).
#include "launch.h"

namespace sllm {

enum BFmt { B_F32 = 0, B_BF16 = 1, B_FP8_BLOCK = 2, B_FP4_PACKED = 3 };

struct BDesc {
  int fmt;
  const void* b;
  const void* scale;
  int bh, bw;  // fp8 block shape (N, K); fp4 uses bw along K
};

__device__ __forceinline__ float load_b_elem(const BDesc& d, int n, int k,
                                             int N, int K) {
  switch (d.fmt) {
    case B_F32: return ((const float*)d.b)[(size_t)n * K + k];
    case B_BF16: return bf16_to_f32(((const uint16_t*)d.b)[(size_t)n * K + k]);
    case B_FP8_BLOCK: {
      const uint8_t q = ((const uint8_t*)d.b)[(size_t)n * K + k];
      const int KB = (K + d.bw - 1) / d.bw;
      const float s = ((const float*)d.scale)[(size_t)(n / d.bh) * KB + k / d.bw];
      return __builtin_amdgcn_cvt_f32_fp8((int)q, 0) * s;
    }
    default: {
      const uint8_t byte = ((const uint8_t*)d.b)[(size_t)n * (K / 2) + k / 2];
      const uint32_t nib = (k & 1) ? (byte >> 4) : (byte & 15);
      const uint32_t e = (nib >> 1) & 3u, m = nib & 1u;
      uint32_t bits = e ? ((e + 126u) << 23) | (m << 22) : (m ? 0x3F000000u : 0u);
      const float v = __uint_as_float(bits | ((nib & 8u) << 28));
      const int KB = (K + d.bw - 1) / d.bw;
      const uint8_t sb = ((const uint8_t*)d.scale)[(size_t)n * KB + k / d.bw];
      const float s = sb == 0 ? 0.f : (sb == 255 ? __uint_as_float(0x7FC00000u)
                                                 : __uint_as_float((uint32_t)sb << 23));
      return v * s;
    }
  }
}

// sllm_q4_gemv_rows' post-op, in place: 1 silu(x / scale), 2 sigmoid.
__global__ void post_act_kernel(float* __restrict__ v, long n, int post,
                                float scale) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = v[i] / scale;
  v[i] = post == 1 ? silu_f32(x) : sigmoid_f32(x);
}

// 32x32 output tile per 256-thread block; each thread 4 outputs (rows).
__global__ __launch_bounds__(256) void tiled_gemm_kernel(
    const void* __restrict__ a, int a_bf16, BDesc bd, float* __restrict__ c,
    int M, int N, int K) {
  __shared__ float as[32][33];
  __shared__ float bs[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // ty 0..7
  const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < K; k0 += 32) {
    for (int i = threadIdx.x; i < 32 * 32; i += 256) {
      const int r = i / 32, kk = i % 32;
      const int m = m0 + r, n = n0 + r, k = k0 + kk;
      float av = 0.f, bv = 0.f;
      if (m < M && k < K)
        av = a_bf16 ? bf16_to_f32(((const uint16_t*)a)[(size_t)m * K + k])
                    : ((const float*)a)[(size_t)m * K + k];
      if (n < N && k < K) bv = load_b_elem(bd, n, k, N, K);
      as[r][kk] = av;
      bs[r][kk] = bv;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk) {
      const float bv = bs[tx][kk];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = fmaf(as[ty * 4 + q][kk], bv, acc[q]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int m = m0 + ty * 4 + q, n = n0 + tx;
    if (m < M && n < N) c[(size_t)m * N + n] = acc[q];
  }
}

int launch_tiled_gemm(const void* a, int a_bf16, const BDesc& bd, float* c,
                      int M, int N, int K, hipStream_t st) {
  SLLM_REQUIRE(a && bd.b && c, "gemm: null pointer");
  SLLM_REQUIRE(M > 0 && N > 0 && K > 0, "gemm: bad dims M=%d N=%d K=%d", M, N,
               K);
  dim3 grid(ceil_div(N, 32), ceil_div(M, 32));
  tiled_gemm_kernel<<<grid, 256, 0, st>>>(a, a_bf16, bd, c, M, N, K);
  SLLM_LAUNCHED();
  return 0;
}

}  // namespace sllm

using namespace sllm;

namespace {
struct Tmp {
  void* p = nullptr;
  ~Tmp() {
    if (p) (void)hipFree(p);
  }
};
}  // namespace

extern "C" {

int sllm_fp8_gemm_dev(const float* A, const unsigned char* B,
                      const float* scale_inv, float* C, int M, int N, int K,
                      int block_h, int block_w) {
  SLLM_REQUIRE(M > 0 && N > 0 && K > 0 && block_h > 0 && block_w > 0,
               "sllm_fp8_gemm: bad dims");
  SLLM_REQUIRE(scale_inv, "sllm_fp8_gemm: null scale");
  // decode-size batches with the loader's 128 x 128 blocks: the layer's
  // unpacked-weight GEMV (one wave per four weight rows, 16-byte weight
  // loads dequantized in registers), which streams B once per launch
  if (block_h == 128 && block_w == 128 && M <= 64 && N % 128 == 0 &&
      K % 128 == 0)
    return launch_gemv(0, 0, A, 0, 0, nullptr, 1, M, nullptr, nullptr, 1,
                       nullptr, B, scale_inv, nullptr, nullptr, N, K, nullptr,
                       0.f, C, nullptr);
  BDesc bd{B_FP8_BLOCK, B, scale_inv, block_h, block_w};
  return launch_tiled_gemm(A, 0, bd, C, M, N, K, 0);
}

int sllm_fp8_gemm(const float* A, const unsigned char* B,
                  const float* scale_inv, float* C, int M, int N, int K,
                  int block_h, int block_w) {
  SLLM_REQUIRE(A && B && scale_inv && C, "sllm_fp8_gemm: null pointer");
  SLLM_REQUIRE(M > 0 && N > 0 && K > 0 && block_h > 0 && block_w > 0,
               "sllm_fp8_gemm: bad dims");
  const size_t sa = (size_t)M * K * 4, sb = (size_t)N * K,
               sc = (size_t)M * N * 4,
               ss = (size_t)ceil_div(N, block_h) * ceil_div(K, block_w) * 4;
  Tmp dA, dB, dS, dC;
  SLLM_HIP(hipMalloc(&dA.p, sa));
  SLLM_HIP(hipMalloc(&dB.p, sb));
  SLLM_HIP(hipMalloc(&dS.p, ss));
  SLLM_HIP(hipMalloc(&dC.p, sc));
  SLLM_HIP(hipMemcpy(dA.p, A, sa, hipMemcpyHostToDevice));
  SLLM_HIP(hipMemcpy(dB.p, B, sb, hipMemcpyHostToDevice));
  SLLM_HIP(hipMemcpy(dS.p, scale_inv, ss, hipMemcpyHostToDevice));
  if (sllm_fp8_gemm_dev((const float*)dA.p, (const unsigned char*)dB.p,
                        (const float*)dS.p, (float*)dC.p, M, N, K, block_h,
                        block_w))
    return -1;
  SLLM_HIP(hipMemcpy(C, dC.p, sc, hipMemcpyDeviceToHost));
  return 0;
}

int sllm_ds_fp4_gemm(float* o, const float* a, const float* b, int M, int N,
                     int K, float scale, float* opts) {
  (void)scale;
  (void)opts;
  SLLM_REQUIRE(o && a && b, "sllm_ds_fp4_gemm: null pointer");
  SLLM_REQUIRE(M > 0 && N > 0 && K > 0, "sllm_ds_fp4_gemm: bad dims");
  const size_t sa = (size_t)M * K * 4, sb = (size_t)N * K * 4,
               sc = (size_t)M * N * 4;
  Tmp dA, dB, dC;
  SLLM_HIP(hipMalloc(&dA.p, sa));
  SLLM_HIP(hipMalloc(&dB.p, sb));
  SLLM_HIP(hipMalloc(&dC.p, sc));
  SLLM_HIP(hipMemcpy(dA.p, a, sa, hipMemcpyHostToDevice));
  SLLM_HIP(hipMemcpy(dB.p, b, sb, hipMemcpyHostToDevice));
  BDesc bd{B_F32, dB.p, nullptr, 0, 0};
  if (launch_tiled_gemm(dA.p, 0, bd, (float*)dC.p, M, N, K, 0)) return -1;
  SLLM_HIP(hipMemcpy(o, dC.p, sc, hipMemcpyDeviceToHost));
  return 0;
}

// Device pointers: a (M, K) fp32, packed (N, K/2) E2M1, scale (N, K/bw) E8M0.
int sllm_ds_fp4_gemm_packed_dev(float* o, const float* a, const void* packed,
                                const void* scale_e8m0, int M, int N, int K,
                                int block_w) {
  SLLM_REQUIRE(K % 2 == 0 && block_w > 0, "fp4 gemm: K even, block_w > 0");
  // decode-size batches with 32-column scale blocks: the layer's
  // unpacked-weight GEMV in its MXFP4 form (the same nibble order, E2M1
  // values and 0x00 / 0xFF scale convention)
  if (block_w == 32 && M <= 64 && K % 32 == 0 && N % 16 == 0)
    return launch_gemv(1, 0, a, 0, 0, nullptr, 1, M, nullptr, nullptr, 1,
                       nullptr, (const uint8_t*)packed, scale_e8m0, nullptr,
                       nullptr, N, K, nullptr, 0.f, o, nullptr);
  BDesc bd{B_FP4_PACKED, packed, scale_e8m0, 1, block_w};
  return launch_tiled_gemm(a, 0, bd, o, M, N, K, 0);
}

// Host pointers: same arguments as the device variant.
int sllm_ds_fp4_gemm_packed(float* o, const float* a, const void* packed,
                            const void* scale_e8m0, int M, int N, int K,
                            int block_w) {
  SLLM_REQUIRE(o && a && packed && scale_e8m0, "fp4 gemm: null pointer");
  SLLM_REQUIRE(M > 0 && N > 0 && K > 0 && K % 2 == 0 && block_w > 0,
               "fp4 gemm: bad dims");
  const size_t sa = (size_t)M * K * 4, sp = (size_t)N * (K / 2),
               ss = (size_t)N * ceil_div(K, block_w), sc = (size_t)M * N * 4;
  Tmp dA, dP, dS, dC;
  SLLM_HIP(hipMalloc(&dA.p, sa));
  SLLM_HIP(hipMalloc(&dP.p, sp));
  SLLM_HIP(hipMalloc(&dS.p, ss));
  SLLM_HIP(hipMalloc(&dC.p, sc));
  SLLM_HIP(hipMemcpy(dA.p, a, sa, hipMemcpyHostToDevice));
  SLLM_HIP(hipMemcpy(dP.p, packed, sp, hipMemcpyHostToDevice));
  SLLM_HIP(hipMemcpy(dS.p, scale_e8m0, ss, hipMemcpyHostToDevice));
  if (sllm_ds_fp4_gemm_packed_dev((float*)dC.p, (const float*)dA.p, dP.p, dS.p,
                                  M, N, K, block_w))
    return -1;
  SLLM_HIP(hipMemcpy(o, dC.p, sc, hipMemcpyDeviceToHost));
  return 0;
}

// c (m, n) fp32 = a (m, k) . w (n, k)^T; atype 0 = fp32, 1 = bf16 for both a
// and w (dtype tags of kernels/_sllm_cuda.py:490-491). Device pointers.
// bf16 with k % 128 == 0 runs on the router GEMM kernels (the same contract:
// bf16 products on the matrix cores, fp32 accumulation; m <= 64, the decode
// loops' GEMVs, on the K-split small-batch kernel); other batches of at most
// 64 rows (fp32, or bf16 with other k) on the unpacked-weight GEMV; the rest
// on the tiled kernel.
int sllm_gemm_ex(const void* a, int atype, const void* w, void* c, int m,
                 int n, int k) {
  SLLM_REQUIRE(atype == 0 || atype == 1, "sllm_gemm_ex: atype must be 0 or 1");
  SLLM_REQUIRE(a && w && c && m > 0 && n > 0 && k > 0,
               "sllm_gemm_ex: null pointer or empty shape (m=%d n=%d k=%d)",
               m, n, k);
  if (atype == 1 && k % 128 == 0)
    return launch_router_gemm((const uint16_t*)a, (const uint16_t*)w,
                              (float*)c, m, n, k, nullptr, 1);
  // other decode-size batches: the unpacked-weight GEMV (bf16 or fp32 rows)
  if (m <= 64 && n % 16 == 0 && k % (atype == 1 ? 8 : 4) == 0)
    return launch_gemv(atype == 1 ? 2 : 3, 0, a, atype, 0, nullptr, 1, m,
                       nullptr, nullptr, 1, nullptr, (const uint8_t*)w,
                       nullptr, nullptr, nullptr, n, k, nullptr, 0.f,
                       (float*)c, nullptr);
  BDesc bd{atype == 1 ? B_BF16 : B_F32, w, nullptr, 0, 0};
  return launch_tiled_gemm(a, atype, bd, (float*)c, m, n, k, 0);
}

// ref: kernels/cuda/qwen4.cu:98-136, :699-708 (sllm_q4_gemv_rows[_dev]):
// out (rows, O) fp32 = A (rows, K) . W (O, K)^T, then post 1: silu(x /
// scale), post 2: sigmoid(x / scale), other values: none. rows, K or O
// not positive: -1, as the reference. Batches of at most 64 rows on the
// unpacked-weight GEMV (fp32 weight rows), larger ones on the tiled kernel.
int sllm_q4_gemv_rows_dev(const float* A, const float* W, float* out, int rows,
                          int K, int O, int post, float scale) {
  SLLM_REQUIRE(rows > 0 && K > 0 && O > 0,
               "sllm_q4_gemv_rows: rows, K, O must be positive");
  SLLM_REQUIRE(A && W && out, "sllm_q4_gemv_rows: null pointer");
  int rc;
  if (rows <= 64 && O % 16 == 0 && K % 4 == 0) {
    rc = launch_gemv(3, 0, A, 0, 0, nullptr, 1, rows, nullptr, nullptr, 1,
                     nullptr, (const uint8_t*)W, nullptr, nullptr, nullptr, O,
                     K, nullptr, 0.f, out, nullptr);
  } else {
    BDesc bd{B_F32, W, nullptr, 0, 0};
    rc = launch_tiled_gemm(A, 0, bd, out, rows, O, K, 0);
  }
  if (rc || (post != 1 && post != 2)) return rc;
  const long n = (long)rows * O;
  post_act_kernel<<<(unsigned)((n + 255) / 256), 256>>>(out, n, post, scale);
  SLLM_LAUNCHED();
  return 0;
}

int sllm_q4_gemv_rows(const float* A, const float* W, float* out, int rows,
                      int K, int O, int post, float scale) {
  SLLM_REQUIRE(rows > 0 && K > 0 && O > 0,
               "sllm_q4_gemv_rows: rows, K, O must be positive");
  SLLM_REQUIRE(A && W && out, "sllm_q4_gemv_rows: null pointer");
  const size_t sa = (size_t)rows * K * 4, sw = (size_t)O * K * 4,
               so = (size_t)rows * O * 4;
  Tmp dA, dW, dO;
  SLLM_HIP(hipMalloc(&dA.p, sa));
  SLLM_HIP(hipMalloc(&dW.p, sw));
  SLLM_HIP(hipMalloc(&dO.p, so));
  SLLM_HIP(hipMemcpy(dA.p, A, sa, hipMemcpyHostToDevice));
  SLLM_HIP(hipMemcpy(dW.p, W, sw, hipMemcpyHostToDevice));
  if (sllm_q4_gemv_rows_dev((const float*)dA.p, (const float*)dW.p,
                            (float*)dO.p, rows, K, O, post, scale))
    return -1;
  SLLM_HIP(hipMemcpy(out, dO.p, so, hipMemcpyDeviceToHost));
  return 0;
}

}  // extern "C"
