// Scratch memory of the allocation-free linear (ne_exl3_lin_run_noalloc): one file-scope device array per GPU, of a
// fixed size, held until the process ends. Its device address comes from hipGetSymbolAddress, taken once per device
// with that device current (at the library's device set-up, or at the first call on another device); host code only
// ever passes that address, never the array's name (a host-side stand-in that is not device memory).
//
// Every call on one GPU shares its array and finds the previous call's contents: the block counters are cleared by a
// fill kernel at the start of each call (a kernel, not a memset, so that a captured call replays correctly). Calls that overlap on one GPU (two streams, two threads) race on the array.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kernels.h"

namespace ijah {

namespace {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
void *g_scratch[kMaxDevices] = {};
std::mutex g_mu;

__global__ __launch_bounds__(256) void zero_u32(uint32_t *p, uint32_t n) {
  for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

}  // namespace

uint8_t *noalloc_scratch() {
  int dev = 0;
  IJ_HIP(hipGetDevice(&dev));
  IJ_CHECK(dev >= 0 && dev < kMaxDevices, "no-alloc scratch: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> g(g_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    IJ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    IJ_CHECK(p, "no-alloc scratch: no device address");
    g_scratch[dev] = p;
  }
  return (uint8_t *)g_scratch[dev];
}

void launch_zero_u32(uint32_t *p, size_t n, hipStream_t s) {
  if (!n) return;
  IJ_CHECK(n < (1ull << 32), "zero fill: %zu words", n);
  const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(zero_u32, dim3(grid), dim3(256), 0, s, p, (uint32_t)n);
}

}  // namespace ijah
