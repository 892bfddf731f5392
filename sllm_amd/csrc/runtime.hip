// Device runtime surface: error buffer, device buffers, sync.
//
// Replaces the buffer / sync half of the reference's shared runtime
// (kernels/cuda/kernels.cu:17-29, 150-194, 425-429): sllm_buf_new/free,
// sllm_buf_h2d/h2d_raw/d2h, sllm_mem_free_bytes, sllm_sync,
// sllm_device_count, sllm_last_error. Same names and argument meaning; the
// error buffer is thread-local instead of a process-global static.
#include <stdarg.h>
#include <string.h>

#include <algorithm>

#include "common.h"

namespace sllm {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

const char* last_error() { return g_err; }

// Counter-based normal generator for synthetic data: value i is a pure
// function of (seed, i) -- splitmix64 of the pair index gives two uniforms,
// Box-Muller gives two normals -- so any launch shape yields the same array.
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// grid-stride copy: 16-byte vectors, then the byte tail
__global__ void copy_kernel(const uint8_t* __restrict__ src,
                            uint8_t* __restrict__ dst, long nbytes) {
  const long n16 = nbytes / 16;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    ((uint4*)dst)[i] = ((const uint4*)src)[i];
  const long t = n16 * 16 + (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < nbytes) dst[t] = src[t];
}

__global__ void fill_normal_kernel(float* __restrict__ dst, long n,
                                   uint64_t seed, float stdv) {
  const long pair = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long i = 2 * pair;
  if (i >= n) return;
  const uint64_t r = splitmix64(seed * 0xD1B54A32D192ED03ull + (uint64_t)pair);
  // uniforms in (0, 1] and [0, 1)
  const float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);
  const float u2 = (float)((r >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
  const float rad = sqrtf(-2.0f * logf(u1)) * stdv;
  float sv, cv;
  sincosf(6.28318530717958647692f * u2, &sv, &cv);
  dst[i] = rad * cv;
  if (i + 1 < n) dst[i + 1] = rad * sv;
}

}  // namespace sllm

using namespace sllm;

extern "C" {

const char* sllm_last_error(void) { return last_error(); }
const char* sllm_q4_last_error(void) { return last_error(); }
const char* sllm_fp8_last_error(void) { return last_error(); }
const char* sllm_ds_last_error(void) { return last_error(); }
const char* sllm_moe_last_error(void) { return last_error(); }

int sllm_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    set_error("hipGetDeviceCount failed");
    return -1;
  }
  return n;
}

void* sllm_buf_new(long nbytes) {
  if (nbytes <= 0) {
    set_error("sllm_buf_new: nbytes must be positive (got %ld)", nbytes);
    return nullptr;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, (size_t)nbytes);
  if (e != hipSuccess) {
    set_error("hipMalloc(%ld): %s", nbytes, hipGetErrorString(e));
    return nullptr;
  }
  return p;
}

int sllm_buf_free(void* p) {
  if (!p) return 0;
  // work already queued may still read the buffer: drain the device first
  // (the reference's cudaFree gives the same guarantee implicitly)
  SLLM_HIP(hipDeviceSynchronize());
  SLLM_HIP(hipFree(p));
  return 0;
}

int sllm_buf_h2d(void* dst, const float* src, long nbytes) {
  SLLM_REQUIRE(dst && src && nbytes >= 0, "sllm_buf_h2d: bad args");
  SLLM_HIP(hipMemcpy(dst, src, (size_t)nbytes, hipMemcpyHostToDevice));
  return 0;
}

int sllm_buf_h2d_raw(void* dst, const void* src, long nbytes) {
  SLLM_REQUIRE(dst && src && nbytes >= 0, "sllm_buf_h2d_raw: bad args");
  SLLM_HIP(hipMemcpy(dst, src, (size_t)nbytes, hipMemcpyHostToDevice));
  return 0;
}

int sllm_buf_d2h(float* dst, const void* src, long nbytes) {
  SLLM_REQUIRE(dst && src && nbytes >= 0, "sllm_buf_d2h: bad args");
  SLLM_HIP(hipMemcpy(dst, src, (size_t)nbytes, hipMemcpyDeviceToHost));
  return 0;
}

int sllm_buf_d2h_raw(void* dst, const void* src, long nbytes) {
  SLLM_REQUIRE(dst && src && nbytes >= 0, "sllm_buf_d2h_raw: bad args");
  SLLM_HIP(hipMemcpy(dst, src, (size_t)nbytes, hipMemcpyDeviceToHost));
  return 0;
}

void* sllm_host_new(long nbytes) {
  if (nbytes <= 0) {
    set_error("sllm_host_new: nbytes must be positive");
    return nullptr;
  }
  void* p = nullptr;
  if (hipHostMalloc(&p, (size_t)nbytes, hipHostMallocDefault) != hipSuccess) {
    set_error("sllm_host_new: hipHostMalloc of %ld bytes failed", nbytes);
    return nullptr;
  }
  return p;
}

int sllm_host_free(void* p) {
  if (!p) return 0;
  SLLM_HIP(hipDeviceSynchronize());  // queued copies may still use it
  SLLM_HIP(hipHostFree(p));
  return 0;
}

int sllm_copy_async(void* dst, const void* src, long nbytes, void* stream) {
  SLLM_REQUIRE(dst && src && nbytes >= 0, "sllm_copy_async: bad args");
  if (nbytes == 0) return 0;
  SLLM_HIP(hipMemcpyAsync(dst, src, (size_t)nbytes, hipMemcpyDefault,
                          (hipStream_t)stream));
  return 0;
}

int sllm_stream_sync(void* stream) {
  SLLM_HIP(hipStreamSynchronize((hipStream_t)stream));
  return 0;
}

// Host-side fp32 -> bf16 bits, round to nearest even on the 32-bit pattern
// (the carry of 0xFFFFFFFF wraps to 0, as in a 16-bit truncation of the
// widened sum).
int sllm_host_f32_to_bf16(void* dst, const float* src, long n) {
  SLLM_REQUIRE(dst && src && n >= 0, "sllm_host_f32_to_bf16: bad args");
  const uint32_t* u = (const uint32_t*)src;
  uint16_t* d = (uint16_t*)dst;
  for (long i = 0; i < n; ++i) {
    const uint64_t v = (uint64_t)u[i] + 0x7FFFu + ((u[i] >> 16) & 1u);
    d[i] = (uint16_t)(v >> 16);
  }
  return 0;
}

long sllm_mem_free_bytes(void) {
  size_t fr = 0, tot = 0;
  if (hipMemGetInfo(&fr, &tot) != hipSuccess) {
    set_error("hipMemGetInfo failed");
    return -1;
  }
  return (long)fr;
}

int sllm_sync(void) {
  SLLM_HIP(hipDeviceSynchronize());
  return 0;
}

void* sllm_event_new(void) {
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) {
    set_error("hipEventCreate: %s", hipGetErrorString(e));
    return nullptr;
  }
  return (void*)ev;
}

int sllm_event_free(void* ev) {
  if (!ev) return 0;
  SLLM_HIP(hipEventDestroy((hipEvent_t)ev));
  return 0;
}

int sllm_event_record(void* ev, void* stream) {
  SLLM_REQUIRE(ev, "sllm_event_record: null event");
  SLLM_HIP(hipEventRecord((hipEvent_t)ev, (hipStream_t)stream));
  return 0;
}

int sllm_event_sync(void* ev) {
  SLLM_REQUIRE(ev, "sllm_event_sync: null event");
  SLLM_HIP(hipEventSynchronize((hipEvent_t)ev));
  return 0;
}

float sllm_event_elapsed_ms(void* start, void* stop) {
  float ms = -1.f;
  hipError_t e = hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)stop);
  if (e != hipSuccess) {
    set_error("hipEventElapsedTime: %s", hipGetErrorString(e));
    return -1.f;
  }
  return ms;
}

int sllm_memset(void* dst, int value, long nbytes, void* stream) {
  SLLM_REQUIRE(dst && nbytes >= 0, "sllm_memset: bad args");
  SLLM_HIP(hipMemsetAsync(dst, value, (size_t)nbytes, (hipStream_t)stream));
  return 0;
}

int sllm_buf_copy(void* dst, const void* src, long nbytes, void* stream) {
  SLLM_REQUIRE(dst && src && nbytes >= 0 && ((uintptr_t)dst % 16) == 0 &&
                   ((uintptr_t)src % 16) == 0,
               "sllm_buf_copy: need 16-byte aligned non-null buffers");
  if (nbytes == 0) return 0;
  const long n16 = nbytes / 16;
  const int dev_cus = 256;
  const long blocks = n16 > 0 ? std::min<long>((n16 + 255) / 256, 8L * dev_cus) : 1;
  copy_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(
      (const uint8_t*)src, (uint8_t*)dst, nbytes);
  SLLM_LAUNCHED();
  return 0;
}

int sllm_fill_normal(float* dst, long n, unsigned long long seed, float stdv,
                     void* stream) {
  SLLM_REQUIRE(dst && n >= 0, "sllm_fill_normal: bad args");
  if (n == 0) return 0;
  const long pairs = (n + 1) / 2;
  fill_normal_kernel<<<(unsigned)((pairs + 255) / 256), 256, 0,
                       (hipStream_t)stream>>>(dst, n, (uint64_t)seed, stdv);
  SLLM_LAUNCHED();
  return 0;
}

}  // extern "C"
