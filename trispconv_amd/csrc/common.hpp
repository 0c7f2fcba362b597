// Shared device/host helpers for libtrispconv_hip: error reporting, launch
// checks, integer geometry, the coordinate hash and wave-level primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <type_traits>
#include <utility>

#include "../../include/trispconv_abi.h"

namespace tsc {

// ---------------------------------------------------------------- errors --
int set_error(int code, const char* fmt, ...);
const char* last_error();

#define TSC_REQUIRE(cond, ...)                                        \
  do {                                                                \
    if (!(cond)) return ::tsc::set_error(TSC_EINVAL, __VA_ARGS__);    \
  } while (0)

#define TSC_LAUNCH_CHECK(what)                                                     \
  do {                                                                             \
    hipError_t e_ = hipGetLastError();                                             \
    if (e_ != hipSuccess)                                                          \
      return ::tsc::set_error(-static_cast<int>(e_), "%s: %s", what,               \
                              hipGetErrorString(e_));                              \
  } while (0)

constexpr int kWave = 64;
// Output rows per workgroup tile of the MFMA convolution (4 waves x 64 rows);
// the execution order reorders whole tiles of this size.
constexpr int kConvTileRows = 256;

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t align_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

// Carves typed sub-buffers out of one caller-provided workspace; every
// carve is 256-byte aligned.
struct Carver {
  char* base;
  int64_t used = 0;
  explicit Carver(void* p) : base(static_cast<char*>(p)) {}
  template <typename T>
  T* take(int64_t count) {
    T* p = reinterpret_cast<T*>(base ? base + used : nullptr);
    used += align_up(count * static_cast<int64_t>(sizeof(T)), 256);
    return p;
  }
};

// --------------------------------------------------------------- geometry --
struct Box {            // 3-D extents or per-axis parameters, z-y-x order
  int32_t z, y, x;
};

inline Box box(const int32_t* v) { return Box{v[0], v[1], v[2]}; }

// slot k -> (kz, ky, kx) for a kD x kH x kW kernel
__device__ __forceinline__ void slot_to_zyx(int k, const Box& ks, int& kz, int& ky, int& kx) {
  kx = k % ks.x;
  int r = k / ks.x;
  ky = r % ks.y;
  kz = r / ks.y;
}

// ------------------------------------------------------------------ hash --
// Open addressing, linear probing, power-of-two capacity, one 64-bit word per
// slot: (key << 32) | row.  Keys are the packed (b,z,y,x) cell id, which the
// host guarantees to be < 2^32 - 1, so an all-ones word marks an empty slot.
constexpr uint64_t kEmpty = ~0ull;

__device__ __forceinline__ uint32_t hash32(uint32_t k) {
  // murmur3 finaliser
  k ^= k >> 16;
  k *= 0x85ebca6bu;
  k ^= k >> 13;
  k *= 0xc2b2ae35u;
  k ^= k >> 16;
  return k;
}

__device__ __forceinline__ void hash_insert(unsigned long long* table, uint32_t mask,
                                            uint32_t key, uint32_t row) {
  const unsigned long long word = (static_cast<unsigned long long>(key) << 32) | row;
  uint32_t h = hash32(key) & mask;
  while (true) {
    unsigned long long old = atomicCAS(&table[h], static_cast<unsigned long long>(kEmpty), word);
    if (old == kEmpty) return;
    if (static_cast<uint32_t>(old >> 32) == key) {
      // repeated coordinate: the larger row id wins, as a sequential
      // "table[key] = row" over rows in order would leave it
      atomicMax(&table[h], word);
      return;
    }
    h = (h + 1) & mask;
  }
}

__device__ __forceinline__ int32_t hash_find(const unsigned long long* __restrict__ table,
                                             uint32_t mask, uint32_t key) {
  uint32_t h = hash32(key) & mask;
  while (true) {
    unsigned long long w = table[h];
    if (w == kEmpty) return -1;
    if (static_cast<uint32_t>(w >> 32) == key) return static_cast<int32_t>(w & 0xffffffffu);
    h = (h + 1) & mask;
  }
}

// ------------------------------------------------------------ wave tools --
__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint64_t lanes_below() {
  const int l = __lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

__device__ __forceinline__ int rank_in_wave(uint64_t ballot) {
  return __popcll(ballot & lanes_below());
}

// Pointers into global memory (so that a store through one is a global store,
// not a flat one, also where the compiler cannot trace it to a kernel argument).
typedef __attribute__((address_space(1))) char global_char;
typedef __attribute__((address_space(1))) int32_t global_int;

// Lane L of v = the wave-uniform value x: one v_writelane_b32.
template <int L>
__device__ __forceinline__ void write_lane(int32_t& v, int32_t x) {
  static_assert(L >= 0 && L < kWave, "lane out of range");
  asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(x), "n"(L));
}

// Lanes set in m take a, the others b (one v_cndmask_b32 on values already
// loaded).
__device__ __forceinline__ uint32_t select_lanes(uint64_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_cndmask_b32 %0, %1, %2, %3" : "=v"(r) : "v"(b), "v"(a), "s"(m));
  return r;
}

// The same for 64-bit values (addresses): a C++ select of an address that
// takes arithmetic makes the compiler branch around the arithmetic, one
// exec-masked block per address.
__device__ __forceinline__ uint64_t select_lanes64(uint64_t m, uint64_t a, uint64_t b) {
  const uint32_t lo = select_lanes(m, static_cast<uint32_t>(a), static_cast<uint32_t>(b));
  const uint32_t hi = select_lanes(m, static_cast<uint32_t>(a >> 32), static_cast<uint32_t>(b >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// A pointer into global memory from an address, so that loads through it are
// global loads rather than flat ones.
template <typename T>
__device__ __forceinline__ const T* global_ptr(uint64_t a) {
  return (const T*)reinterpret_cast<const __attribute__((address_space(1))) T*>(a);
}

// f(std::integral_constant<int, Q>{}) for Q = 0, 1, ... in order.
template <typename F, int... Q>
__device__ __forceinline__ void for_each_index(F&& f, std::integer_sequence<int, Q...>) {
  (f(std::integral_constant<int, Q>{}), ...);
}

// ------------------------------------------------------------ conversions --
template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<__half>(__half v) { return __half2float(v); }
template <> __device__ __forceinline__ float to_f32<__hip_bfloat16>(__hip_bfloat16 v) {
  return __bfloat162float(v);
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ __half from_f32<__half>(float v) { return __float2half_rn(v); }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float v) {
  return __float2bfloat16(v);  // round to nearest even
}

inline int dtype_bytes(int dt) { return dt == TSC_F32 ? 4 : 2; }
inline bool dtype_ok(int dt) { return dt == TSC_F32 || dt == TSC_F16 || dt == TSC_BF16; }

// ------------------------------------------------------ shared kernels --
// ------------------------------------------------------------ block scan --
// Inclusive scan across a wave with shuffles.
__device__ __forceinline__ uint32_t wave_inclusive(uint32_t v) {
  const int l = __lane_id();
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    uint32_t t = __shfl_up(v, d, kWave);
    if (l >= d) v += t;
  }
  return v;
}

// Exclusive scan across the block (blockDim.x a multiple of 64, <= 1024).
// Returns the thread's exclusive prefix; *block_total receives the sum.
__device__ __forceinline__ uint32_t block_exclusive(uint32_t v, uint32_t* s_wave, uint32_t* block_total) {
  const int w = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  uint32_t inc = wave_inclusive(v);
  if (__lane_id() == kWave - 1) s_wave[w] = inc;
  __syncthreads();
  if (w == 0) {
    uint32_t t = __lane_id() < nw ? s_wave[__lane_id()] : 0u;
    uint32_t ti = wave_inclusive(t);
    if (__lane_id() < nw) s_wave[__lane_id()] = ti - t;  // exclusive wave offsets
    if (__lane_id() == nw - 1) s_wave[32] = ti;
  }
  __syncthreads();
  uint32_t res = s_wave[w] + inc - v;
  *block_total = s_wave[32];
  __syncthreads();
  return res;
}

__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v);
__global__ void fill_u64_kernel(unsigned long long* p, int64_t n, unsigned long long v);
int fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t s);
// Two fills in one launch.
int fill2_u32(uint32_t* p1, int64_t n1, uint32_t v1, uint32_t* p2, int64_t n2, uint32_t v2,
              hipStream_t s);
// Raises kernel's dynamic LDS limit to bytes on the current device (once per
// kernel and device); 0 or an error code.
int allow_dynamic_lds(const void* kernel, int bytes);
int fill_u64(unsigned long long* p, int64_t n, unsigned long long v, hipStream_t s);

// Per-slot, per-block counts -> exclusive offsets along blocks, plus totals:
// cnt and off are [K][nblk]; totals[k] receives the sum of slot k.  With
// extra_total, cnt and off hold one more row whose sum goes to *extra_total.
struct SlotScan {
  const int32_t* cnt;
  int32_t* off;
  int32_t* totals;
  int K, nblk;
  int32_t* extra_total;
  // with mark_words: *status = the flags the marks' status words hold for
  // generation gen (mark_flags), written by the first slot's block
  const uint32_t* mark_words = nullptr;
  uint32_t gen = 0;
  int32_t* status = nullptr;
  __host__ __device__ int blocks() const { return cnt ? K + (extra_total ? 1 : 0) : 0; }
};

// Per-slot, per-block counts -> exclusive offsets along blocks, plus totals.
// cnt and off are [K][nblk]; totals[k] receives the sum of slot k.  With
// extra_total, cnt and off hold one more row whose sum goes to *extra_total
// (a per-block count summed without a contended atomic).
int scan_slot_blocks(const int32_t* cnt, int32_t* off, int32_t* totals, int K, int nblk,
                     hipStream_t s, int32_t* extra_total = nullptr);

// Per-slot totals of per-block counts: totals[k] = sum of cnt[k][0..nblk).
int sum_slot_blocks(const int32_t* cnt, int32_t* totals, int K, int nblk, hipStream_t s);

// Exclusive scan of n uint32 values produced by `kind` from `src`:
//   kind 0: popcount(src[i])   kind 1: src[i] != 0   kind 2: src[i]
// out[i] receives the prefix, *total the sum (device pointer, may be null).
// Scratch: scan_scratch_words(n) uint32 words.
int64_t scan_scratch_words(int64_t n);

// Occupancy bitmaps with ranks: one 8-byte entry per 32 cells, x = the cells'
// bits, y = the number of set bits in all earlier entries (the rank of the
// entry's first cell), so a rank lookup is one load.  The entry count is
// rounded up to even (entries are processed in pairs; the pad entry is zero).
// bitmap_scan fills y from the x fields wherever a pair of entries has a set
// bit (a rank is only looked up for a set bit; other y are left as they were)
// and writes the total to *total.
int64_t bitmap_entries(int64_t nw);
int64_t bitmap_scan_scratch_words(int64_t nw);

// Occupancy marked as one byte per cell (bitmap builds on dense grids): the
// bytes of whole bitmap entries (32 per entry), then kMarkWords status words.
// A build stores its generation value gen (1..255) into the byte of each cell
// it marks and, for a row it rejects, into that row's status word; it reads a
// byte or a word as set only when it holds gen.  So marks left by earlier
// builds need no zeroing until a value comes round again.  Status words:
// kMarkBatch (a batch index outside [0, B)), kMarkGrid (a coordinate outside
// the grid).
constexpr int kMarkWords = 4;
constexpr int kMarkBatch = 0, kMarkGrid = 1;
inline int64_t marks_bytes(int64_t nw) { return bitmap_entries(nw) * 32 + 4 * kMarkWords; }
inline uint32_t* mark_words(uint8_t* marks, int64_t nw) {
  return reinterpret_cast<uint32_t*>(marks + bitmap_entries(nw) * 32);
}
// The status flags (TSC_FLAG_*) the status words hold for generation gen.
__device__ __forceinline__ int32_t mark_flags(const uint32_t* words, uint32_t gen) {
  return (words[kMarkBatch] == gen ? TSC_FLAG_BATCH_OUT_OF_RANGE : 0) |
         (words[kMarkGrid] == gen ? TSC_FLAG_COORD_OUT_OF_GRID : 0);
}
// With scan, that slot scan (scan_slot_blocks) runs in the same launch as
// the first pass.
// started (may be null): a word of pinned host memory the first launch sets
// when it begins (signal_started).  touched (may be null): one byte per tile
// of kBitmapTileWords words, 0 for tiles none of whose words is set; their
// entries are neither read (they may hold anything) nor written, and count 0.
constexpr int kBitmapTileWords = 1024;
inline int64_t bitmap_tiles(int64_t nw) { return ceil_div(nw > 0 ? nw : 1, kBitmapTileWords); }
// bytes (may be null): byte marks (above) to pack, a cell occupied where its
// byte equals gen.
int bitmap_scan(uint2* wr, int64_t nw, uint32_t* scratch, int32_t* total, hipStream_t s,
                const uint8_t* bytes = nullptr, const SlotScan* scan = nullptr,
                int32_t* started = nullptr, const uint8_t* touched = nullptr,
                uint32_t gen = 1);
// Two words of pinned host memory that kernels store into, one pair per host
// thread and device (allocated on first use there and kept until the process
// ends).  A build that must report bad coordinates before it returns, but
// need not wait for the rest of its kernels, has its checking kernel store a
// non-zero value into the flag word, and the kernel after it store 1 into
// the started word when it begins (so the check has finished); the host
// waits for the started word only.
// After them, room for a build's per-slot counts (up to 4096 slots, plus
// two words) that a kernel copies there, and one word per slot that the
// kernel sets once that slot's count is there.
struct HostStatus {
  int32_t* host;  // host view: [kHostFlag] flag, [kHostStarted] started, counts, done words
  int32_t* dev;   // the same words as kernels address them
};
constexpr int kHostFlag = 0;
constexpr int kHostStarted = 32;  // another 128-byte line
constexpr int kHostCounts = 64;
constexpr int kHostMaxSlots = 4096;
constexpr int kHostDone = kHostCounts + kHostMaxSlots + 32;  // past the counts' two extra words
constexpr int kHostWords = kHostDone + kHostMaxSlots;
int host_status(HostStatus* out);
// Spins until the host word w (the host view of a HostStatus word) is
// non-zero.  If the stream drains first (or reports an error) it stops
// there; *seen = 0 then says the word was never set.
int wait_host_word(const int32_t* w, hipStream_t s, int* seen);

// Block 0's first thread stores 1 into a word of pinned host memory (may be
// null): this kernel has begun, so every kernel before it on the stream has
// finished.
__device__ __forceinline__ void signal_started(int32_t* host_word) {
  if (host_word && blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(host_word, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The submanifold build (tsc_subm_pairs) on a given workspace.  ws_limit > 0:
// ws is that many bytes of fixed scratch, the bitmap is used only when it
// fits and a build that fits in neither way is an argument error; 0: ws is
// the caller's workspace of ws_bytes, sized by tsc_subm_workspace_bytes.
// hs (may be null): the coordinate check also goes to hs's flag word, the
// next kernel sets its started word, and the call waits for that before it
// returns.  mask_row != 0 (K <= 32): nbr has a row K, and the bitmap path's
// probe writes each column's slot mask there.  slot_blocks (may be null): the
// probe's per-(slot, block) counts
// go there ([K][ceil(n / 256)] int32) and counts[0..K) are left for
// tsc_subm_counts; otherwise they are summed into counts.  *raster (may be
// null) = 1 when the map's columns are in (b,z,y,x) order.  marks (may be
// null): byte marks of marks_size bytes that the caller keeps between builds,
// taken instead of the workspace's when the build marks through bytes, with
// gen (1..255) as this build's value; ws then needs the size
// tsc_subm_workspace_bytes gives with marks_outside.
int subm_pairs_ws(const int32_t* coords, int64_t n, int32_t batch_size, const int32_t spatial[3],
                  const int32_t ksize[3], const int32_t dilation[3], void* ws, int64_t ws_bytes,
                  int64_t ws_limit, int32_t* cols_row, int32_t* nbr, int32_t* counts,
                  tsc_stream_t stream, const HostStatus* hs = nullptr,
                  int32_t* slot_blocks = nullptr, int32_t* raster = nullptr,
                  int32_t mask_row = 0, uint8_t* marks = nullptr, int64_t marks_size = 0,
                  int32_t gen = 0);
int exclusive_scan_u32(const uint32_t* src, int kind, int64_t n, uint32_t* out, int32_t* total,
                       uint32_t* scratch, hipStream_t s);

}  // namespace tsc
