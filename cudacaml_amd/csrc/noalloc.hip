// The static scratch of the allocation-free entry point
// (cchip_program_run_resident_noalloc, backend.cpp).
//
// Template scratch (look-back status words and tile counters, split
// reduction partials, scatter counts, offsets and staged pairs, split-k
// partials) normally lives in each executor's pool. The allocation-free
// entry point takes it from the array below instead, so a call needs no
// device memory beyond what the caller passes and the program's pool.
// Every GPU the library runs on holds its own copy of the array (at its own
// address) until the process ends. Calls that overlap on one GPU share it
// and race.

#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.hpp"

namespace {
constexpr size_t kScratchBytes = size_t(32) << 20;
}

// In host code this name is a host-side stand-in for the device array, not
// a device address: only the pointer hipGetSymbolAddress returns for the
// current device may be passed to kernels or copies.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// Zero fill of [p, p + 16 n16): a kernel rather than hipMemsetAsync, so a
// caller may record it into a HIP graph.
__global__ __launch_bounds__(256) void cchip_scratch_clear(uint4 *__restrict__ p, size_t n16) {
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) p[i] = z;
}

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_base[kMaxDevices];

}  // namespace

namespace cchip {

size_t noalloc_scratch_capacity() { return kScratchBytes; }

// The array's device address on `device`, looked up once per device with
// that device current (the caller makes it current).
void *noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) throw Failure(strf("noalloc scratch: device %d out of range", device));
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_base[device]) {
    int cur = -1;
    check_hip(hipGetDevice(&cur), "hipGetDevice");
    if (cur != device) throw Failure("noalloc scratch: device is not current");
    void *ptr = nullptr;
    check_hip(hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!ptr) throw Failure("noalloc scratch: hipGetSymbolAddress returned no address");
    g_base[device] = ptr;
  }
  return g_base[device];
}

// Queues a zero fill of the first `bytes` of the scratch at `base` (an
// address noalloc_scratch returned) on `stream`.
void noalloc_scratch_clear(void *base, size_t bytes, void *stream) {
  if (bytes > kScratchBytes) throw InvalidArgument("noalloc scratch: clear beyond the array");
  size_t n16 = (bytes + 15) / 16;
  if (!n16) return;
  unsigned grid = (unsigned)std::min<size_t>((n16 + 255) / 256, 1024);
  uint4 *p = (uint4 *)base;
  void *args[] = {&p, &n16};
  check_hip(hipLaunchKernel((const void *)cchip_scratch_clear, dim3(grid), dim3(256), args, 0, (hipStream_t)stream),
            "hipLaunchKernel(scratch clear)");
}

}  // namespace cchip
