// Error reporting shared by every C-ABI entry point of libuttt_hip.so.
#include <stdarg.h>

#include "common.h"

namespace {
thread_local char g_last_error[512] = {0};
}

namespace uttt {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

// Turns a failed launch into UTTT_ERR_HIP with the runtime's message.
int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return UTTT_ERR_HIP;
  }
  return UTTT_OK;
}

namespace {
// Zero bytes [0, n) of p: 16-byte stores when p is 16-byte aligned (the tail
// bytewise by the first thread), else bytewise.
__global__ __launch_bounds__(256) void zero_fill_kernel(uint8_t* __restrict__ p, size_t n,
                                                        int vec) {
  const size_t stride = (size_t)gridDim.x * 256;
  const size_t first = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (!vec) {
    for (size_t i = first; i < n; i += stride) p[i] = 0;
    return;
  }
  const size_t vecs = n / 16;
  for (size_t i = first; i < vecs; i += stride)
    reinterpret_cast<uint4*>(p)[i] = make_uint4(0u, 0u, 0u, 0u);
  if (first == 0)
    for (size_t i = vecs * 16; i < n; ++i) p[i] = 0;
}
}  // namespace

// A kernel rather than hipMemsetAsync, so that a caller may capture the call
// in a HIP graph.
int zero_fill_async(void* p, size_t bytes, hipStream_t st, const char* what) {
  if (bytes == 0) return UTTT_OK;
  const int vec = (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
  const size_t items = vec ? (bytes + 15) / 16 : bytes;
  const unsigned blocks = (unsigned)(items < 256 * 1024 ? (items + 255) / 256 : 1024);
  hipLaunchKernelGGL(zero_fill_kernel, dim3(blocks), dim3(256), 0, st,
                     static_cast<uint8_t*>(p), bytes, vec);
  return check_launch(what);
}

}  // namespace uttt

extern "C" int uttt_abi_version(void) { return 4; }

extern "C" const char* uttt_last_error(void) { return g_last_error; }
