// Device runtime surface: error buffer, device buffers, sync.
//
// Replaces the buffer / sync half of the reference's shared runtime
// (kernels/cuda/kernels.cu:17-29, 150-194, 425-429): sllm_buf_new/free,
// sllm_buf_h2d/h2d_raw/d2h, sllm_mem_free_bytes, sllm_sync,
// sllm_device_count, sllm_last_error. Same names and argument meaning; the
// error buffer is thread-local instead of a process-global static.
#include <stdarg.h>
#include <string.h>

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

}  // extern "C"
