// Execution order for the fused convolution.
//
// The convolution kernel computes tiles of output rows and, for each slot k,
// runs the MFMA work for the whole tile if any row of the tile has an input
// through k.  Rows whose neighbour sets differ therefore waste work when they
// share a tile.  This builder sorts output rows by their slot-occupancy mask
// (bit k set when nbr[o][k] >= 0; slots beyond 32 fold onto bit k mod 32)
// with a stable LSD radix sort, so tiles mostly hold rows with one mask.
// Output values do not depend on the order: every row's fp32 accumulation
// sees the same slots in the same ascending order and absent slots add zero.
//
// Radix sort: 8-bit digits; per pass one histogram kernel (per-block digit
// counts, stored digit-major), one exclusive scan over all counts and one
// stable scatter in which each wave ranks equal digits with eight ballots.
#include "common.hpp"

namespace tsc {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 8;                     // per thread per block
constexpr int kTile = kThreads * kItems;      // items per block
constexpr int kRadix = 256;

__global__ void __launch_bounds__(256) mask_kernel(const int32_t* __restrict__ nbr, int64_t n, int K,
                                                   uint32_t* __restrict__ keys,
                                                   uint32_t* __restrict__ vals) {
  const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (o >= n) return;
  const int32_t* row = nbr + o * K;
  uint32_t m = 0;
  for (int k = 0; k < K; ++k) m |= (row[k] >= 0 ? 1u : 0u) << (k & 31);
  keys[o] = m;
  vals[o] = static_cast<uint32_t>(o);
}

__global__ void __launch_bounds__(kThreads) radix_hist_kernel(const uint32_t* __restrict__ keys,
                                                              int64_t n, int shift,
                                                              uint32_t* __restrict__ hist,
                                                              int nblk) {
  __shared__ uint32_t s_h[kRadix];
  s_h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t base = blockIdx.x * (int64_t)kTile;
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = base + j * kThreads + threadIdx.x;
    if (i < n) atomicAdd(&s_h[(keys[i] >> shift) & 0xffu], 1u);
  }
  __syncthreads();
  hist[(int64_t)threadIdx.x * nblk + blockIdx.x] = s_h[threadIdx.x];
}

__global__ void __launch_bounds__(kThreads) radix_scatter_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n,
    int shift, const uint32_t* __restrict__ hist_off, int nblk, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t s_run[kRadix];                   // placed so far, per digit
  __shared__ uint32_t s_wc[kThreads / kWave][kRadix];  // this round, per wave, per digit
  const int t = threadIdx.x;
  const int w = t / kWave;
  s_run[t] = hist_off[(int64_t)t * nblk + blockIdx.x];
  const int64_t base = blockIdx.x * (int64_t)kTile;
  for (int j = 0; j < kItems; ++j) {
#pragma unroll
    for (int ww = 0; ww < kThreads / kWave; ++ww) s_wc[ww][t] = 0;
    __syncthreads();
    const int64_t i = base + j * kThreads + t;  // items stay in index order
    const bool valid = i < n;
    const uint32_t key = valid ? keys_in[i] : 0u;
    const uint32_t val = valid ? vals_in[i] : 0u;
    const uint32_t d = (key >> shift) & 0xffu;
    // lanes of this wave holding the same digit
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint64_t ones = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? ones : ~ones;
    }
    const int rank = rank_in_wave(peers);
    if (valid && rank == 0) s_wc[w][d] = __popcll(peers);
    __syncthreads();
    if (valid) {
      uint32_t pos = s_run[d] + rank;
      for (int ww = 0; ww < w; ++ww) pos += s_wc[ww][d];
      if (pos < n) {  // always true when the digit offsets are consistent
        keys_out[pos] = key;
        vals_out[pos] = val;
      }
    }
    __syncthreads();
    uint32_t add = 0;
#pragma unroll
    for (int ww = 0; ww < kThreads / kWave; ++ww) add += s_wc[ww][t];
    s_run[t] += add;
    __syncthreads();
  }
}

struct Buffers {
  uint32_t *keys_a, *vals_a, *keys_b, *vals_b, *hist, *hist_off, *scratch;
};

Buffers carve(void* ws, int64_t n, int64_t* used) {
  Carver c(ws);
  const int64_t m = n > 0 ? n : 1;
  const int64_t nblk = ceil_div(m, kTile);
  Buffers b;
  b.keys_a = c.take<uint32_t>(m);
  b.vals_a = c.take<uint32_t>(m);
  b.keys_b = c.take<uint32_t>(m);
  b.vals_b = c.take<uint32_t>(m);
  b.hist = c.take<uint32_t>(nblk * kRadix);
  b.hist_off = c.take<uint32_t>(nblk * kRadix);
  b.scratch = c.take<uint32_t>(scan_scratch_words(nblk * kRadix));
  if (used) *used = c.used;
  return b;
}

}  // namespace
}  // namespace tsc

using namespace tsc;

extern "C" int64_t tsc_plan_workspace_bytes(int64_t n_out, int32_t k_vol) {
  (void)k_vol;
  int64_t used = 0;
  carve(nullptr, n_out, &used);
  return used;
}

extern "C" int tsc_conv_plan(const int32_t* nbr, int64_t n_out, int32_t k_vol, void* ws,
                             int64_t ws_bytes, int32_t* order, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(n_out >= 0 && n_out < (int64_t(1) << 31), "plan: n_out out of range");
  TSC_REQUIRE(k_vol > 0, "plan: invalid kernel volume");
  if (n_out == 0) return 0;
  TSC_REQUIRE(nbr && order && ws, "plan: null pointer");
  TSC_REQUIRE(ws_bytes >= tsc_plan_workspace_bytes(n_out, k_vol), "plan: workspace too small");
  Buffers b = carve(ws, n_out, nullptr);
  const int nblk = static_cast<int>(ceil_div(n_out, kTile));
  mask_kernel<<<ceil_div(n_out, 256), 256, 0, s>>>(nbr, n_out, k_vol, b.keys_a, b.vals_a);
  TSC_LAUNCH_CHECK("plan_mask");
  const int bits = k_vol < 32 ? k_vol : 32;
  const int passes = (bits + 7) / 8;
  uint32_t *ki = b.keys_a, *vi = b.vals_a, *ko = b.keys_b, *vo = b.vals_b;
  for (int p = 0; p < passes; ++p) {
    const int shift = 8 * p;
    if (p == passes - 1) {
      // the last pass writes the values straight into the caller's order
      vo = reinterpret_cast<uint32_t*>(order);
    }
    radix_hist_kernel<<<nblk, kThreads, 0, s>>>(ki, n_out, shift, b.hist, nblk);
    TSC_LAUNCH_CHECK("plan_hist");
    int rc = exclusive_scan_u32(b.hist, 2, (int64_t)nblk * kRadix, b.hist_off, nullptr, b.scratch, s);
    if (rc) return rc;
    radix_scatter_kernel<<<nblk, kThreads, 0, s>>>(ki, vi, n_out, shift, b.hist_off, nblk, ko, vo);
    TSC_LAUNCH_CHECK("plan_scatter");
    uint32_t* tk = ki;
    ki = ko;
    ko = tk;
    uint32_t* tv = vi;
    vi = vo;
    vo = tv;
  }
  return 0;
}
