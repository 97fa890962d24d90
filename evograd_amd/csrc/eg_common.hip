// Error slot, launch checking and device queries shared by every entry point.
#include "eg_common.hpp"

#include <string.h>

namespace eg {

static thread_local char g_error[1024] = "";

// Kernel-timing hook: eg_time_kernel arms this thread's launches from the next
// entry-point call on; the `index`-th of them (counted across calls) records
// `start` and `stop`.
struct TimingArm {
  hipEvent_t start = nullptr, stop = nullptr;
  int index = 0;
  int next = 0;
  bool pending = false;
  bool active = false;
};
static thread_local TimingArm g_arm;
static thread_local char g_label[64] = "";

void set_timed_label(const char* expr) {
  // "(name<T, ...>)" or "name": keep the identifier
  while (*expr == '(' || *expr == ' ') ++expr;
  size_t n = 0;
  while (n + 1 < sizeof(g_label) &&
         ((expr[n] >= 'a' && expr[n] <= 'z') || (expr[n] >= 'A' && expr[n] <= 'Z') ||
          (expr[n] >= '0' && expr[n] <= '9') || expr[n] == '_'))
    ++n;
  memcpy(g_label, expr, n);
  g_label[n] = '\0';
}

bool timed_launch(hipEvent_t* start, hipEvent_t* stop) {
  if (!g_arm.active) return false;
  const bool hit = g_arm.next == g_arm.index;
  ++g_arm.next;
  if (!hit) return false;
  *start = g_arm.start;
  *stop = g_arm.stop;
  g_arm.active = false;
  return true;
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() {
  g_error[0] = '\0';
  if (g_arm.pending) {  // a fresh arm starts counting at this call
    g_arm.active = true;
    g_arm.pending = false;
    g_arm.next = 0;
  }
}

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
  EG_LAUNCH(zero_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (unsigned char*)p, bytes);
  return check_launch(what);
}

}  // namespace eg

extern "C" int eg_time_kernel_missed(void) {
  const int missed = (eg::g_arm.pending || eg::g_arm.active) ? 1 : 0;
  eg::g_arm.pending = false;
  eg::g_arm.active = false;
  return missed;
}

extern "C" int eg_abi_version(void) { return 4; }

extern "C" const char* eg_time_kernel_label(void) { return eg::g_label; }

extern "C" const char* eg_last_error(void) { return eg::g_error; }

extern "C" int eg_time_kernel(void* start_event, void* stop_event, int index) {
  if (!start_event || !stop_event || index < 0) {
    eg::set_error("eg_time_kernel: null event or negative index");
    return 1;
  }
  eg::g_arm.start = reinterpret_cast<hipEvent_t>(start_event);
  eg::g_arm.stop = reinterpret_cast<hipEvent_t>(stop_event);
  eg::g_arm.index = index;
  eg::g_label[0] = '\0';
  eg::g_arm.pending = true;
  eg::g_arm.active = false;
  return 0;
}
