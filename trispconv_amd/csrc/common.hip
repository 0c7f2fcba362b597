// Error reporting, fills and the two scans shared by the pair builders.
#include "common.hpp"

#include <cstdarg>
#include <mutex>
#include <utility>
#include <vector>

namespace tsc {

namespace {
thread_local std::string g_error;
}

int set_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

const char* last_error() { return g_error.c_str(); }

// ------------------------------------------------------------------ fills --
__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

__global__ void fill_u64_kernel(unsigned long long* p, int64_t n, unsigned long long v) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

static int fill_grid(int64_t n) {
  int64_t g = ceil_div(n, 256);
  return static_cast<int>(g < 4096 ? (g < 1 ? 1 : g) : 4096);
}

// Two fills in one launch: the first g1 blocks fill (p1, n1), the rest (p2, n2).
__global__ void fill2_u32_kernel(uint32_t* p1, int64_t n1, uint32_t v1, int g1, uint32_t* p2,
                                 int64_t n2, uint32_t v2) {
  const bool first = static_cast<int>(blockIdx.x) < g1;
  uint32_t* p = first ? p1 : p2;
  const int64_t n = first ? n1 : n2;
  const uint32_t v = first ? v1 : v2;
  const int64_t b = first ? blockIdx.x : blockIdx.x - g1;
  const int64_t nb = first ? g1 : gridDim.x - g1;
  for (int64_t i = b * blockDim.x + threadIdx.x; i < n; i += nb * blockDim.x) p[i] = v;
}

int fill2_u32(uint32_t* p1, int64_t n1, uint32_t v1, uint32_t* p2, int64_t n2, uint32_t v2,
              hipStream_t s) {
  const int g1 = fill_grid(n1), g2 = fill_grid(n2);
  fill2_u32_kernel<<<g1 + g2, 256, 0, s>>>(p1, n1, v1, g1, p2, n2, v2);
  TSC_LAUNCH_CHECK("fill2_u32");
  return 0;
}

// Dynamic LDS limits are a per-device attribute of a kernel: each (kernel,
// device) pair is raised once, on the first launch on that device.
int allow_dynamic_lds(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::vector<std::pair<const void*, int>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(-static_cast<int>(e), "hipGetDevice: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& d : done)
    if (d.first == kernel && d.second == dev) return 0;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess)
    return set_error(-static_cast<int>(e), "dynamic LDS of %d bytes: %s", bytes, hipGetErrorString(e));
  done.emplace_back(kernel, dev);
  return 0;
}

int fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t s) {
  if (n <= 0) return 0;
  fill_u32_kernel<<<fill_grid(n), 256, 0, s>>>(p, n, v);
  TSC_LAUNCH_CHECK("fill_u32");
  return 0;
}

int fill_u64(unsigned long long* p, int64_t n, unsigned long long v, hipStream_t s) {
  if (n <= 0) return 0;
  fill_u64_kernel<<<fill_grid(n), 256, 0, s>>>(p, n, v);
  TSC_LAUNCH_CHECK("fill_u64");
  return 0;
}

// ---------------------------------------------------- per-slot block scan --
// Slot k's exclusive scan along blocks, by one thread block of any size that
// is a multiple of 64.
__device__ void slot_scan_block(const SlotScan& a, int k, uint32_t* s_wave) {
  const int nblk = a.nblk, K = a.K;
  const int32_t* cnt = a.cnt;
  int32_t* off = a.off;
  int32_t* totals = a.totals;
  int32_t* extra_total = a.extra_total;
  const int32_t* c = cnt + (int64_t)k * nblk;
  int32_t* o = off + (int64_t)k * nblk;
  uint32_t carry = 0;
  for (int base = 0; base < nblk; base += blockDim.x) {
    const int i = base + threadIdx.x;
    uint32_t v = i < nblk ? static_cast<uint32_t>(c[i]) : 0u;
    uint32_t tot;
    uint32_t ex = block_exclusive(v, s_wave, &tot);
    if (i < nblk) o[i] = static_cast<int32_t>(carry + ex);
    carry += tot;
  }
  if (threadIdx.x == 0) {
    if (k < K)
      totals[k] = static_cast<int32_t>(carry);
    else
      *extra_total = static_cast<int32_t>(carry);
    if (k == 0 && a.mark_words) *a.status = mark_flags(a.mark_words, a.gen);
  }
}

__global__ void __launch_bounds__(1024) scan_slot_blocks_kernel(SlotScan a) {
  __shared__ uint32_t s_wave[33];
  slot_scan_block(a, blockIdx.x, s_wave);
}

int scan_slot_blocks(const int32_t* cnt, int32_t* off, int32_t* totals, int K, int nblk,
                     hipStream_t s, int32_t* extra_total) {
  const SlotScan a{cnt, off, totals, K, nblk, extra_total};
  scan_slot_blocks_kernel<<<a.blocks(), 1024, 0, s>>>(a);
  TSC_LAUNCH_CHECK("scan_slot_blocks");
  return 0;
}

// One block per slot: totals[k] = sum over blocks of cnt[k][*].
__global__ void __launch_bounds__(256) sum_slot_blocks_kernel(const int32_t* __restrict__ cnt,
                                                              int32_t* __restrict__ totals,
                                                              int nblk) {
  __shared__ uint32_t s_wave[33];
  const int32_t* c = cnt + (int64_t)blockIdx.x * nblk;
  uint32_t acc = 0;
  for (int i = threadIdx.x; i < nblk; i += blockDim.x) acc += static_cast<uint32_t>(c[i]);
  uint32_t tot;
  block_exclusive(acc, s_wave, &tot);
  if (threadIdx.x == 0) totals[blockIdx.x] = static_cast<int32_t>(tot);
}

int sum_slot_blocks(const int32_t* cnt, int32_t* totals, int K, int nblk, hipStream_t s) {
  sum_slot_blocks_kernel<<<K, 256, 0, s>>>(cnt, totals, nblk);
  TSC_LAUNCH_CHECK("sum_slot_blocks");
  return 0;
}

// ---------------------------------------------------- device-wide scan --
constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;                       // per thread
constexpr int kScanTile = kScanThreads * kScanItems; // per block

__device__ __forceinline__ uint32_t scan_value(const uint32_t* src, int kind, int64_t i) {
  uint32_t v = src[i];
  if (kind == 0) return __popc(v);
  if (kind == 1) return v != 0u ? 1u : 0u;
  return v;
}

__global__ void __launch_bounds__(kScanThreads) scan_reduce_kernel(const uint32_t* __restrict__ src,
                                                                   int kind, int64_t n,
                                                                   uint32_t* __restrict__ sums) {
  __shared__ uint32_t s_wave[33];
  const int64_t base = blockIdx.x * (int64_t)kScanTile;
  uint32_t acc = 0;
#pragma unroll 4
  for (int j = 0; j < kScanItems; ++j) {
    const int64_t i = base + j * kScanThreads + threadIdx.x;  // coalesced
    if (i < n) acc += scan_value(src, kind, i);
  }
  uint32_t tot;
  block_exclusive(acc, s_wave, &tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

__global__ void __launch_bounds__(1024) scan_sums_kernel(uint32_t* __restrict__ sums, int64_t nblk,
                                                         int32_t* __restrict__ total) {
  __shared__ uint32_t s_wave[33];
  uint32_t carry = 0;
  for (int64_t b = 0; b < nblk; b += blockDim.x) {
    const int64_t i = b + threadIdx.x;
    uint32_t v = i < nblk ? sums[i] : 0u;
    uint32_t tot;
    uint32_t ex = block_exclusive(v, s_wave, &tot);
    if (i < nblk) sums[i] = carry + ex;
    carry += tot;
  }
  if (threadIdx.x == 0 && total) *total = static_cast<int32_t>(carry);
}

__global__ void __launch_bounds__(kScanThreads) scan_apply_kernel(const uint32_t* __restrict__ src,
                                                                  int kind, int64_t n,
                                                                  const uint32_t* __restrict__ sums,
                                                                  uint32_t* __restrict__ out) {
  __shared__ uint32_t s_wave[33];
  // each thread owns kScanItems consecutive items so the prefix stays in order
  const int64_t base = blockIdx.x * (int64_t)kScanTile + threadIdx.x * (int64_t)kScanItems;
  uint32_t v[kScanItems];
  uint32_t acc = 0;
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    const int64_t i = base + j;
    v[j] = i < n ? scan_value(src, kind, i) : 0u;
    acc += v[j];
  }
  uint32_t tot;
  uint32_t run = sums[blockIdx.x] + block_exclusive(acc, s_wave, &tot);
#pragma unroll
  for (int j = 0; j < kScanItems; ++j) {
    const int64_t i = base + j;
    if (i < n) out[i] = run;
    run += v[j];
  }
}

// Inputs of up to kSmallScan items (one chunk of 1024 x 12 consecutive
// items, 48 KB of LDS) are scanned by one workgroup in a single launch; one
// workgroup is slower than the three-kernel scan beyond that.
constexpr int kSmallItems = 12;
constexpr int64_t kSmallScan = 1024 * kSmallItems;

__global__ void __launch_bounds__(1024) scan_small_kernel(const uint32_t* __restrict__ src, int kind,
                                                          int64_t n, uint32_t* __restrict__ out,
                                                          int32_t* __restrict__ total) {
  // A chunk goes through LDS both ways, so global reads and writes are
  // coalesced while each thread scans 16 consecutive values.
  __shared__ uint32_t s_val[1024 * kSmallItems];
  __shared__ uint32_t s_wave[33];
  uint32_t carry = 0;
  for (int64_t base = 0; base < n; base += 1024 * kSmallItems) {
    const int m = static_cast<int>(n - base < 1024 * kSmallItems ? n - base : 1024 * kSmallItems);
    for (int i = threadIdx.x; i < m; i += 1024) s_val[i] = scan_value(src, kind, base + i);
    __syncthreads();
    const int b0 = threadIdx.x * kSmallItems;
    uint32_t v[kSmallItems];
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < kSmallItems; ++j) {
      v[j] = b0 + j < m ? s_val[b0 + j] : 0u;
      acc += v[j];
    }
    uint32_t tot;
    uint32_t run = carry + block_exclusive(acc, s_wave, &tot);
#pragma unroll
    for (int j = 0; j < kSmallItems; ++j) {
      if (b0 + j < m) s_val[b0 + j] = run;
      run += v[j];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < m; i += 1024) out[base + i] = s_val[i];
    __syncthreads();
    carry += tot;
  }
  if (threadIdx.x == 0 && total) *total = static_cast<int32_t>(carry);
}

int64_t scan_scratch_words(int64_t n) { return ceil_div(n > 0 ? n : 1, kScanTile); }

int exclusive_scan_u32(const uint32_t* src, int kind, int64_t n, uint32_t* out, int32_t* total,
                       uint32_t* scratch, hipStream_t s) {
  if (n <= 0) {
    if (total) {
      int rc = fill_u32(reinterpret_cast<uint32_t*>(total), 1, 0u, s);
      if (rc) return rc;
    }
    return 0;
  }
  if (n <= kSmallScan) {
    scan_small_kernel<<<1, 1024, 0, s>>>(src, kind, n, out, total);
    TSC_LAUNCH_CHECK("scan_small");
    return 0;
  }
  const int64_t nblk = ceil_div(n, kScanTile);
  scan_reduce_kernel<<<nblk, kScanThreads, 0, s>>>(src, kind, n, scratch);
  TSC_LAUNCH_CHECK("scan_reduce");
  scan_sums_kernel<<<1, 1024, 0, s>>>(scratch, nblk, total);
  TSC_LAUNCH_CHECK("scan_sums");
  scan_apply_kernel<<<nblk, kScanThreads, 0, s>>>(src, kind, n, scratch, out);
  TSC_LAUNCH_CHECK("scan_apply");
  return 0;
}


// ------------------------------------------------------ bitmap rank scan --
// Exclusive popcount scan of the bitmap words into their y fields.  A tile is
// 1024 words (256 threads x 4); the reduce pass writes each tile's popcount,
// the apply pass takes its tile's offset from those (summing them itself when
// `pre` is null, else from `pre`, their exclusive scan) and writes the ranks.
constexpr int kBmThreads = 256;
constexpr int kBmTile = kBmThreads * 4;
static_assert(kBmTile == kBitmapTileWords, "one scan tile per touched flag");

__global__ void __launch_bounds__(kBmThreads) bitmap_reduce_kernel(const uint4* __restrict__ wr2,
                                                                   int64_t nw,
                                                                   uint32_t* __restrict__ sums,
                                                                   int nsum, SlotScan scan,
                                                                   int32_t* started,
                                                                   const uint8_t* __restrict__ touched) {
  __shared__ uint32_t s_wave[33];
  signal_started(started);
  if (static_cast<int>(blockIdx.x) >= nsum) {  // blocks past the tiles: a slot scan riding along
    slot_scan_block(scan, blockIdx.x - nsum, s_wave);
    return;
  }
  if (touched && !touched[blockIdx.x]) {  // no word of this tile is set (block-uniform)
    if (threadIdx.x == 0) sums[blockIdx.x] = 0;
    return;
  }
  const int64_t p = (blockIdx.x * (int64_t)kBmTile) / 2 + 2 * threadIdx.x;  // entry pairs
  uint32_t acc = 0;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (2 * (p + j) < nw) {
      const uint4 v = wr2[p + j];  // word pairs past nw are zero padding
      acc += __popc(v.x) + __popc(v.z);
    }
  }
  uint32_t tot;
  block_exclusive(acc, s_wave, &tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

// The reduce pass for occupancy given as one byte per cell (set where the
// byte equals the build's generation value): packs each word's 32 bytes into
// its bit mask (word x, y zeroed; the padding word past nw packs bytes that
// no build marks) and sums the tile's popcounts.
// A byte y of v ^ (gen * 0x01010101) is 0 exactly where v's byte equals gen,
// and then, only then, bit 7 of ~(((y & 0x7f) + 0x7f) | y) is set (the sum
// stays within the byte).  Those bits, moved to bit 0 of their bytes b0..b3,
// give the nibble b0 + 2b1 + 4b2 + 8b3 in the top byte of dword * 0x01020408
// (no carries reach it).
__device__ __forceinline__ uint32_t marked_nibble(uint32_t v, uint32_t rep) {
  const uint32_t y = v ^ rep;
  const uint32_t z = ~(((y & 0x7f7f7f7fu) + 0x7f7f7f7fu) | y) & 0x80808080u;
  return ((z >> 7) * 0x01020408u) >> 24;
}

__device__ __forceinline__ uint32_t pack_bytes(uint4 a, uint4 b, uint32_t rep) {
  return marked_nibble(a.x, rep) | marked_nibble(a.y, rep) << 4 | marked_nibble(a.z, rep) << 8 |
         marked_nibble(a.w, rep) << 12 | marked_nibble(b.x, rep) << 16 |
         marked_nibble(b.y, rep) << 20 | marked_nibble(b.z, rep) << 24 |
         marked_nibble(b.w, rep) << 28;
}

// One thread per entry pair (512 per tile): twice the waves of two pairs a
// thread, for a pass that only streams the byte marks (measured: the 16.7 MB
// surface build 0.0720-0.0729 -> 0.0710-0.0732 ms, the 23.6 MB LiDAR strided
// build 0.0956-0.0970 -> 0.0938-0.0943 ms).
constexpr int kPackThreads = kBmTile / 2;

__global__ void __launch_bounds__(kPackThreads) bitmap_pack_kernel(const uint4* __restrict__ bytes,
                                                                   uint4* __restrict__ wr2,
                                                                   int64_t nw,
                                                                   uint32_t* __restrict__ sums,
                                                                   int nsum, SlotScan scan,
                                                                   int32_t* started, uint32_t gen) {
  __shared__ uint32_t s_wave[33];
  signal_started(started);
  if (static_cast<int>(blockIdx.x) >= nsum) {  // blocks past the tiles: a slot scan riding along
    slot_scan_block(scan, blockIdx.x - nsum, s_wave);
    return;
  }
  const int64_t p = (blockIdx.x * (int64_t)kBmTile) / 2 + threadIdx.x;  // entry pair
  uint32_t acc = 0;
  if (2 * p < nw) {
    // words 2p and 2p + 1: 64 bytes, four 16-byte loads (the byte map covers
    // whole entry pairs)
    const uint4* src = bytes + 4 * p;
    const uint32_t rep = gen * 0x01010101u;
    const uint32_t m0 = pack_bytes(src[0], src[1], rep);
    const uint32_t m1 = pack_bytes(src[2], src[3], rep);
    wr2[p] = make_uint4(m0, 0u, m1, 0u);
    acc = __popc(m0) + __popc(m1);
  }
  uint32_t tot;
  block_exclusive(acc, s_wave, &tot);
  if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

// One thread per entry pair (512 per tile), like the pack pass; the pair is
// loaded before the tile-sum scan, so the two round trips overlap.
__global__ void __launch_bounds__(kPackThreads) bitmap_apply_kernel(uint4* __restrict__ wr2,
                                                                    int64_t nw,
                                                                    const uint32_t* __restrict__ sums,
                                                                    const uint32_t* __restrict__ pre,
                                                                    int nsum,
                                                                    int32_t* __restrict__ n_unique,
                                                                    const uint8_t* __restrict__ touched) {
  __shared__ uint32_t s_wave[33];
  // a tile without a set bit has no rank to write (block-uniform)
  const bool live = !touched || touched[blockIdx.x];
  const int64_t p = (blockIdx.x * (int64_t)kBmTile) / 2 + threadIdx.x;
  const bool in = live && 2 * p < nw;
  uint4 v = in ? wr2[p] : make_uint4(0u, 0u, 0u, 0u);
  uint32_t base;
  if (pre) {
    base = pre[blockIdx.x];
  } else {
    // this tile's offset, and on block 0 the total, from the tile sums
    const int lim = blockIdx.x == 0 ? nsum : static_cast<int>(blockIdx.x);
    uint32_t part = 0;
    for (int i = threadIdx.x; i < lim; i += kPackThreads) part += sums[i];
    uint32_t tot;
    block_exclusive(part, s_wave, &tot);
    base = blockIdx.x == 0 ? 0u : tot;
    if (blockIdx.x == 0 && threadIdx.x == 0) *n_unique = static_cast<int32_t>(tot);
  }
  if (!live) return;
  const uint32_t c0 = __popc(v.x), c1 = __popc(v.z);
  uint32_t tot;
  const uint32_t run = base + block_exclusive(c0 + c1, s_wave, &tot);
  // a rank is only looked up for a set bit, so pairs of empty words keep
  // theirs unwritten (on sparse grids nearly every pair: the pass then mostly
  // reads)
  v.y = run;
  v.w = run + c0;
  if (in && (v.x | v.z)) wr2[p] = v;
}

// Bitmap scans of up to this many tiles let every apply block sum the tile
// sums before it (one launch less); longer ones scan the sums first.
constexpr int64_t kBmDirectTiles = 2048;

int64_t bitmap_entries(int64_t nw) { return 2 * ceil_div(nw > 0 ? nw : 1, 2); }

int64_t bitmap_scan_scratch_words(int64_t nw) {
  const int64_t nsum = ceil_div(nw > 0 ? nw : 1, kBmTile);
  return 2 * nsum + scan_scratch_words(nsum);
}

int bitmap_scan(uint2* wr, int64_t nw, uint32_t* scratch, int32_t* total, hipStream_t s,
                const uint8_t* bytes, const SlotScan* scan, int32_t* started,
                const uint8_t* touched, uint32_t gen) {
  TSC_REQUIRE(!touched || !bytes, "bitmap_scan: touched tiles are for bitmaps marked in place");
  TSC_REQUIRE(!bytes || (gen >= 1 && gen <= 255), "bitmap_scan: mark value %u outside 1..255",
              gen);
  const int64_t nsum = ceil_div(nw > 0 ? nw : 1, kBmTile);
  uint32_t* sums = scratch;
  uint32_t* pre = scratch + nsum;
  uint32_t* more = scratch + 2 * nsum;
  uint4* wr2 = reinterpret_cast<uint4*>(wr);
  const SlotScan none{nullptr, nullptr, nullptr, 0, 0, nullptr};
  const SlotScan& sc = scan ? *scan : none;
  const unsigned grid = static_cast<unsigned>(nsum + sc.blocks());
  if (bytes) {
    bitmap_pack_kernel<<<grid, kPackThreads, 0, s>>>(reinterpret_cast<const uint4*>(bytes), wr2,
                                                     nw, sums, static_cast<int>(nsum), sc, started,
                                                     gen);
    TSC_LAUNCH_CHECK("bitmap_pack");
  } else {
    bitmap_reduce_kernel<<<grid, kBmThreads, 0, s>>>(wr2, nw, sums, static_cast<int>(nsum), sc,
                                                     started, touched);
    TSC_LAUNCH_CHECK("bitmap_reduce");
  }
  const uint32_t* p = nullptr;
  if (nsum > kBmDirectTiles) {
    int rc = exclusive_scan_u32(sums, 2, nsum, pre, total, more, s);
    if (rc) return rc;
    p = pre;
  }
  bitmap_apply_kernel<<<static_cast<unsigned>(nsum), kPackThreads, 0, s>>>(
      wr2, nw, sums, p, static_cast<int>(nsum < kBmDirectTiles ? nsum : kBmDirectTiles), total,
      touched);
  TSC_LAUNCH_CHECK("bitmap_apply");
  return 0;
}

// --------------------------------------------------- host status words --
namespace {
constexpr int kMaxStatusDevices = 64;

// Blocks of threads that have ended, per device, handed to the next thread
// that needs one.  A block is idle when its thread ends: every call that
// enqueues a write into it waits for that write before it returns, and each
// call clears the words it waits on first.  So a program that builds pairs
// from many short-lived threads holds as many blocks as it has such threads
// alive at once, not one per thread it ever started.
std::mutex g_free_mu;
std::vector<HostStatus> g_free_blocks[kMaxStatusDevices];

struct ThreadStatus {
  HostStatus dev[kMaxStatusDevices] = {};
  ~ThreadStatus() {
    std::lock_guard<std::mutex> lock(g_free_mu);
    for (int d = 0; d < kMaxStatusDevices; ++d)
      if (dev[d].host) g_free_blocks[d].push_back(dev[d]);
  }
};
thread_local ThreadStatus t_status;
}  // namespace

int host_status(HostStatus* out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(-static_cast<int>(e), "host_status: hipGetDevice: %s", hipGetErrorString(e));
  TSC_REQUIRE(dev >= 0 && dev < kMaxStatusDevices, "host_status: device %d beyond %d devices",
              dev, kMaxStatusDevices);
  HostStatus& h = t_status.dev[dev];
  if (!h.host) {
    std::lock_guard<std::mutex> lock(g_free_mu);
    if (!g_free_blocks[dev].empty()) {
      h = g_free_blocks[dev].back();
      g_free_blocks[dev].pop_back();
    }
  }
  if (!h.host) {
    void* p = nullptr;
    e = hipHostMalloc(&p, kHostWords * sizeof(int32_t), hipHostMallocMapped | hipHostMallocCoherent);
    if (e != hipSuccess)
      return set_error(-static_cast<int>(e), "host_status: hipHostMalloc: %s",
                       hipGetErrorString(e));
    void* d = nullptr;
    e = hipHostGetDevicePointer(&d, p, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(p);
      return set_error(-static_cast<int>(e), "host_status: hipHostGetDevicePointer: %s",
                       hipGetErrorString(e));
    }
    h.host = static_cast<int32_t*>(p);
    h.dev = static_cast<int32_t*>(d);
  }
  *out = h;
  return 0;
}

int wait_host_word(const int32_t* w, hipStream_t s, int* seen) {
  for (uint32_t i = 1;; ++i) {
    if (__atomic_load_n(w, __ATOMIC_ACQUIRE)) {
      *seen = 1;
      return 0;
    }
    if ((i & 255) == 0) {  // every few microseconds: has the stream drained or failed?
      const hipError_t e = hipStreamQuery(s);
      if (e == hipSuccess) {
        *seen = __atomic_load_n(w, __ATOMIC_ACQUIRE) != 0;
        return 0;
      }
      if (e != hipErrorNotReady)
        return set_error(-static_cast<int>(e), "waiting for a host word: %s",
                         hipGetErrorString(e));
    }
    __builtin_ia32_pause();
  }
}

}  // namespace tsc

extern "C" const char* tsc_last_error(void) { return tsc::last_error(); }
extern "C" int tsc_abi_version(void) { return 12; }
