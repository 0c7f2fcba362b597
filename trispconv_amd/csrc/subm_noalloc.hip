// Submanifold pairs without any allocation: tsc_subm_pairs_noalloc.
//
// The same build as tsc_subm_pairs (trispconv/pytorch/indices.py:67-140, see
// pairs_subm.hip), for callers that cannot allocate device memory — code
// under HIP graph capture, tight serving loops, harnesses that forbid it.
// Its scratch (the occupancy bitmap and its scan, or the hash table, and the
// column words) is a fixed device array in this library's code object: one
// copy per GPU, kStaticScratchBytes long, held until the process ends.  Every
// call on a GPU uses that GPU's copy, and the kernels clear what they need
// before use, so calls that overlap on one GPU (two streams, two threads)
// race; calls in stream order do not.
#include "common.hpp"

#include <mutex>

constexpr int64_t kStaticScratchBytes = int64_t(64) << 20;

// Host code never uses this name as an address (in host code it is only a
// stand-in): the device address comes from hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// This GPU's copy of the scratch, looked up once per device (the first call
// there), with that device current.
int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return tsc::set_error(-static_cast<int>(e), "subm_noalloc: hipGetDevice: %s",
                          hipGetErrorString(e));
  TSC_REQUIRE(dev >= 0 && dev < kMaxDevices, "subm_noalloc: device %d beyond %d devices", dev,
              kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
      return tsc::set_error(-static_cast<int>(e), "subm_noalloc: hipGetSymbolAddress: %s",
                            hipGetErrorString(e));
    TSC_REQUIRE(p != nullptr, "subm_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}
}  // namespace

extern "C" int64_t tsc_subm_pairs_noalloc_limit(void) { return kStaticScratchBytes; }

extern "C" int tsc_subm_pairs_noalloc(const int32_t* coords, int64_t n, int32_t batch_size,
                                      const int32_t spatial[3], const int32_t ksize[3],
                                      const int32_t dilation[3], int32_t* cols_row,
                                      int32_t* nbr, int32_t* counts, tsc_stream_t stream) {
  void* ws = nullptr;
  if (int rc = scratch_of_current_device(&ws)) return rc;
  return tsc::subm_pairs_ws(coords, n, batch_size, spatial, ksize, dilation, ws,
                            kStaticScratchBytes, kStaticScratchBytes, cols_row, nbr, counts,
                            stream);
}
