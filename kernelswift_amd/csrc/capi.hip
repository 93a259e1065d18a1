// C-ABI plumbing: error reporting, version, and the traffic-calibration copy kernel.
#include "common.h"

#include <cstdarg>
#include <string>

namespace ks {

std::string &last_error() {
  thread_local std::string msg;
  return msg;
}

int fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

// Grid-stride 16-byte copy: every lane moves one uint4 per iteration.
__global__ __launch_bounds__(256) void copy16_kernel(const uint4 *__restrict__ src,
                                                     uint4 *__restrict__ dst, int64_t n16) {
  int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride)
    dst[i] = src[i];
}

}  // namespace ks

extern "C" const char *ks_last_error(void) { return ks::last_error().c_str(); }

extern "C" int ks_version(void) { return 100; }

extern "C" int ks_copy_bytes(const void *src, void *dst, int64_t n_bytes, void *stream) {
  ks::last_error().clear();
  KS_CHECK_ARG(n_bytes >= 0 && n_bytes % 16 == 0, "ks_copy_bytes: n_bytes=%lld must be a non-negative multiple of 16",
               (long long)n_bytes);
  if (n_bytes == 0) return KS_OK;
  KS_CHECK_ARG(src && dst, "ks_copy_bytes: null pointer");
  KS_CHECK_ARG(ks::aligned(src, 16) && ks::aligned(dst, 16), "ks_copy_bytes: pointers must be 16-byte aligned");
  const int64_t n16 = n_bytes / 16;
  const int64_t blocks = std::min<int64_t>(ks::ceil_div(n16, 256), 256 * 32);
  hipLaunchKernelGGL(ks::copy16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint4 *>(src), static_cast<uint4 *>(dst), n16);
  KS_CHECK_LAUNCH("copy16_kernel");
  return KS_OK;
}
