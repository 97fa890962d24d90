// Error slot, launch checking and device queries shared by every entry point.
#include "eg_common.hpp"

#include <string.h>

namespace eg {

static thread_local char g_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return 2;
  }
  return 0;
}

__global__ void zero_bytes_kernel(unsigned char* __restrict__ p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

int zero_fill(void* p, size_t bytes, hipStream_t st, const char* what) {
  if (bytes == 0) return 0;
  if (!p) { set_error("%s: null pointer", what); return 1; }
  size_t blocks = (bytes + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(zero_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                     (unsigned char*)p, bytes);
  return check_launch(what);
}

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace eg

extern "C" int eg_abi_version(void) { return 1; }

extern "C" const char* eg_last_error(void) { return eg::g_error; }
