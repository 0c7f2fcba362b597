// Execution order for the fused convolution.
//
// The convolution kernel computes tiles of output rows.  Two things make a
// tile cheap:
//   * its rows need the same kernel slots — for each slot k the MFMA work of a
//     32-row block is skipped only when no row of the block has an input
//     through k, so rows with different slot sets waste matrix-core work;
//   * its rows, and the tiles an XCD runs around the same time, gather from
//     nearby input rows — the gathered rows then come from cache instead of
//     HBM.
// The order built here serves both: output rows are put in Morton (z-order)
// order, cut into regions of `region_rows` consecutive rows (the caller sizes
// them so one region's input rows fit in cache), and sorted inside each
// region by their slot-occupancy mask (bit k set when nbr[k][o] >= 0; slots
// beyond 32 fold onto bit k mod 32), ties kept in Morton order.  (With a
// single region the Morton sort is skipped: ties keep the column order.)  Last, whole
// 256-row tiles (the convolution's workgroup tiles) are reordered inside each
// region by the number of slots their rows use, most first, the partial tile
// staying last: the convolution deals tiles to the XCDs in this order, so
// the heavy ones start early and the launch does not end on a few of them.
//
// Output values never depend on the order: every row's fp32 accumulation
// sees the same slots in the same ascending order and absent slots add zero.
//
// The permuted map is gathered from a row-major copy of the map (maps of up
// to 32 slots), which the mask pass writes: one 128-byte row per position
// instead of one scattered entry per slot.
//
// Sorting: stable LSD radix passes with 9-bit digits (a 27-slot mask sorts
// in three passes).  Each pass is a histogram kernel (per-block digit counts,
// digit-major), a scan of each digit's counts over the blocks (one workgroup
// per digit) and a stable scatter, whose blocks add the digits' bases
// themselves and in which each wave ranks equal digits with nine ballots.  The first sort
// orders rows by their Morton code; the second carries Morton positions as
// values and takes its digits from the mask at that position, then from the
// region (position / region_rows).
#include "common.hpp"

#include <utility>

namespace tsc {
namespace {

constexpr int kThreads = 256;
constexpr int kItems = 4;                     // per thread per block
constexpr int kTile = kThreads * kItems;      // items per block
constexpr int kDigitBits = 9;
constexpr int kRadix = 1 << kDigitBits;

// Digit sources of a pass.
enum DigitSrc { kFromKey = 0, kFromMaskAtValue = 1, kFromRegionOfValue = 2 };

struct Digits {
  int src;
  int shift;
  const uint32_t* keys;      // kFromKey: keys[i]
  const uint32_t* mask_pos;  // kFromMaskAtValue: mask_pos[value]
  uint32_t region_rows;      // kFromRegionOfValue: value / region_rows
};

__device__ __forceinline__ uint32_t digit_of(const Digits& d, int64_t i, uint32_t value) {
  uint32_t k;
  if (d.src == kFromKey)
    k = d.keys[i];
  else if (d.src == kFromMaskAtValue)
    k = d.mask_pos[value];
  else
    k = value / d.region_rows;
  return (k >> d.shift) & (kRadix - 1u);
}

// Spreads the low 10 bits of v to every third bit.
__device__ __forceinline__ uint32_t spread3(uint32_t v) {
  v &= 0x3ffu;
  v = (v | (v << 16)) & 0x030000ffu;
  v = (v | (v << 8)) & 0x0300f00fu;
  v = (v | (v << 4)) & 0x030c30c3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}

// Morton code of each map column's row: the sample index in the bits at and
// above batch_shift, then the leading bits of the 30-bit z-order code of
// (z, y, x) >> coarse (coarse chosen by the host so the largest axis fits 10
// bits).  Columns without a row sort last.
__global__ void __launch_bounds__(256) spatial_key_kernel(const int4* __restrict__ coords,
                                                          const int32_t* __restrict__ cols_row,
                                                          int64_t n, int coarse, int batch_shift,
                                                          uint32_t* __restrict__ keys,
                                                          uint32_t* __restrict__ vals) {
  const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (o >= n) return;
  vals[o] = static_cast<uint32_t>(o);
  const int32_t row = cols_row ? cols_row[o] : static_cast<int32_t>(o);
  if (row < 0) {
    keys[o] = 0xffffffffu;
    return;
  }
  const int4 c = coords[row];
  const uint32_t m = (spread3(static_cast<uint32_t>(c.y) >> coarse) << 2) |
                     (spread3(static_cast<uint32_t>(c.z) >> coarse) << 1) |
                     spread3(static_cast<uint32_t>(c.w) >> coarse);
  const uint32_t spatial = batch_shift >= 30 ? m : (m >> (30 - batch_shift));
  keys[o] = (batch_shift >= 32 ? 0u : (static_cast<uint32_t>(c.x) << batch_shift)) | spatial;
}

// mask_row[o] = slot mask of output row o.  Lanes take consecutive rows, so
// every slot's map column is read coalesced; eight slots' loads in flight.
// vals (may be null): vals[o] = o as well (columns that are their own
// Morton positions: mask_row is then mask_pos).
__global__ void __launch_bounds__(256) row_mask_kernel(const int32_t* __restrict__ nbr, int64_t n,
                                                       int K, uint32_t* __restrict__ mask_row,
                                                       uint32_t* __restrict__ vals) {
  const int64_t o = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (o >= n) return;
  if (vals) vals[o] = static_cast<uint32_t>(o);
  uint32_t m = 0;
  for (int k0 = 0; k0 < K; k0 += 8) {
    int32_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = nbr[(int64_t)(k0 + i < K ? k0 + i : K - 1) * n + o];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + i < K) m |= (v[i] >= 0 ? 1u : 0u) << ((k0 + i) & 31);
  }
  mask_row[o] = m;
}

// mask_pos[i] = slot mask of output row rows[i]; vals[i] = i.
__global__ void __launch_bounds__(256) mask_at_pos_kernel(const uint32_t* __restrict__ mask_row,
                                                          int64_t n,
                                                          const uint32_t* __restrict__ rows,
                                                          uint32_t* __restrict__ mask_pos,
                                                          uint32_t* __restrict__ vals) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  mask_pos[i] = mask_row[rows[i]];
  vals[i] = static_cast<uint32_t>(i);
}

// Sort key of each full tile of the order (one 256-thread block per tile):
// the tile's region in the high bits, then 32 - (slots in the union of its
// rows' masks), so tiles with more slots sort first inside a region.
__global__ void __launch_bounds__(kConvTileRows) tile_key_kernel(
    const uint32_t* __restrict__ pos, const uint32_t* __restrict__ mask_pos,
    int64_t tiles_per_region, uint32_t* __restrict__ keys, uint32_t* __restrict__ vals) {
  __shared__ uint32_t s_or[kConvTileRows / kWave];
  const int64_t tile = blockIdx.x;
  uint32_t m = mask_pos[pos[tile * kConvTileRows + threadIdx.x]];
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) m |= __shfl_xor(m, off, kWave);
  if ((threadIdx.x & (kWave - 1)) == 0) s_or[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t u = 0;
#pragma unroll
    for (int w = 0; w < kConvTileRows / kWave; ++w) u |= s_or[w];
    const uint32_t region = static_cast<uint32_t>(tile / tiles_per_region);
    keys[tile] = (region << 6) | (32u - static_cast<uint32_t>(__popc(u)));
    vals[tile] = static_cast<uint32_t>(tile);
  }
}

// perm[i] = map column processed at position i; order[i] = its row;
// pos_masks[i] (when given) = its slot mask.  Positions inside the first
// n_tiles full tiles come from tile tile_perm[i/256] (when given); the rest
// stay where the sorts put them.
__global__ void __launch_bounds__(256) gather_rows_kernel(const uint32_t* __restrict__ pos,
                                                          const uint32_t* __restrict__ cols,
                                                          const int32_t* __restrict__ cols_row,
                                                          int64_t n,
                                                          const uint32_t* __restrict__ tile_perm,
                                                          int64_t n_tiles,
                                                          const uint32_t* __restrict__ mask_pos,
                                                          uint32_t* __restrict__ perm,
                                                          int32_t* __restrict__ order,
                                                          uint32_t* __restrict__ pos_masks) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t tile = i / kConvTileRows;
  const int64_t src = (tile_perm && tile < n_tiles)
                          ? static_cast<int64_t>(tile_perm[tile]) * kConvTileRows + i % kConvTileRows
                          : i;
  const uint32_t mp = pos[src];  // the column's Morton position
  const uint32_t col = cols ? cols[mp] : mp;  // null: columns in (b,z,y,x) order are their positions
  perm[i] = col;
  order[i] = cols_row ? cols_row[col] : static_cast<int32_t>(col);
  if (pos_masks) pos_masks[i] = mask_pos[mp];
}

// nbr_ordered[k][t] = nbr[k][perm[t]], four positions per thread.  Blocks are
// dispatched round-robin over the 8 XCDs in launch order; block b runs on XCD
// b % 8, which takes slots x, x+8, x+16, ... one after another, so each
// slot's column (and the order) is gathered through one XCD's L2 instead of
// being fetched by all eight.
__global__ void __launch_bounds__(256) permute_map_kernel(const int32_t* __restrict__ nbr,
                                                          const uint32_t* __restrict__ order,
                                                          int64_t n, int K, int chunks, int vec,
                                                          int32_t* __restrict__ out) {
  const int64_t b = blockIdx.x;
  const int64_t i = b / 8;                 // this XCD's i-th block
  const int k = static_cast<int>(b % 8 + 8 * (i / chunks));
  if (k >= K) return;
  const int64_t t0 = ((i % chunks) * (int64_t)blockDim.x + threadIdx.x) * 4;
  if (t0 >= n) return;
  const int32_t* col = nbr + (int64_t)k * n;
  int32_t* dst = out + (int64_t)k * n;
  if (vec && t0 + 4 <= n) {
    const uint4 o = *reinterpret_cast<const uint4*>(order + t0);
    *reinterpret_cast<int4*>(dst + t0) = make_int4(col[o.x], col[o.y], col[o.z], col[o.w]);
  } else {
    for (int64_t t = t0; t < n && t < t0 + 4; ++t) dst[t] = col[order[t]];
  }
}

// For maps of up to 32 slots: the slot mask of each column, as
// row_mask_kernel, and a row-major copy of the map, nbr_t[c][k] = nbr[k][c]
// in rows of 32 entries (128 bytes; entries k >= K hold -1), from which the
// permute reads one line per position instead of K scattered entries.  A
// block stages 256 columns of every slot in LDS and writes their rows as
// 16-byte vectors.
__global__ void __launch_bounds__(256) map_rows_kernel(const int32_t* __restrict__ nbr, int64_t n,
                                                       int K, int32_t* __restrict__ nbr_t,
                                                       uint32_t* __restrict__ mask_row,
                                                       uint32_t* __restrict__ vals) {
  __shared__ int32_t s_e[32][257];
  const int t = threadIdx.x;
  const int64_t c0 = blockIdx.x * (int64_t)256;
  const int64_t c = c0 + t;
  uint32_t m = 0;
  for (int k0 = 0; k0 < 32; k0 += 8) {
    int32_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = (c < n && k0 + i < K) ? nbr[(int64_t)(k0 + i) * n + c] : -1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s_e[k0 + i][t] = v[i];
      m |= (v[i] >= 0 ? 1u : 0u) << (k0 + i);
    }
  }
  if (c < n) {
    mask_row[c] = m;
    if (vals) vals[c] = static_cast<uint32_t>(c);
  }
  __syncthreads();
  int4* rows = reinterpret_cast<int4*>(nbr_t);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int i = j * 256 + t;  // 16-byte piece i: row i / 8, entries 4 (i % 8) ..
    const int r = i >> 3, q = i & 7;
    if (c0 + r < n)
      rows[(c0 + r) * 8 + q] = make_int4(s_e[4 * q][r], s_e[4 * q + 1][r], s_e[4 * q + 2][r],
                                         s_e[4 * q + 3][r]);
  }
}

// nbr_ordered[k][t] = nbr[k][perm[t]] from the row-major copy: each wave
// takes 64 positions, reads their rows two at a time (lanes 0..31 and
// 32..63 each read one 128-byte row, entry k by lane k), and writes every
// slot's 64 entries as one coalesced run after a transpose in LDS.
__global__ void __launch_bounds__(256) permute_rows_kernel(const int32_t* __restrict__ nbr_t,
                                                           const uint32_t* __restrict__ perm,
                                                           int64_t n, int K,
                                                           int32_t* __restrict__ out) {
  __shared__ int32_t s_e[4][32][65];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t p0 = (blockIdx.x * (int64_t)4 + w) * 64;
  const int k = lane & 31, half = lane >> 5;
  const uint32_t my_col = p0 + lane < n ? perm[p0 + lane] : 0u;
#pragma unroll 8
  for (int j = 0; j < 32; ++j) {
    const int pp = 2 * j + half;  // this half's position
    const uint32_t col = __shfl(my_col, pp, kWave);
    s_e[w][k][pp] = p0 + pp < n ? nbr_t[(int64_t)col * 32 + k] : -1;
  }
  __syncthreads();
  if (p0 + lane < n)
    for (int kk = 0; kk < K; ++kk) out[(int64_t)kk * n + p0 + lane] = s_e[w][kk][lane];
}

__global__ void __launch_bounds__(kThreads) radix_hist_kernel(const uint32_t* __restrict__ vals,
                                                              int64_t n, Digits d,
                                                              uint32_t* __restrict__ hist,
                                                              int nblk) {
  __shared__ uint32_t s_h[kRadix];
  for (int r = threadIdx.x; r < kRadix; r += kThreads) s_h[r] = 0;
  __syncthreads();
  const int64_t base = blockIdx.x * (int64_t)kTile;
#pragma unroll
  for (int j = 0; j < kItems; ++j) {
    const int64_t i = base + j * kThreads + threadIdx.x;
    if (i < n) atomicAdd(&s_h[digit_of(d, i, vals[i])], 1u);
  }
  __syncthreads();
  for (int r = threadIdx.x; r < kRadix; r += kThreads) hist[(int64_t)r * nblk + blockIdx.x] = s_h[r];
}

// One workgroup per digit: the exclusive scan of the digit's per-block counts
// (hist_off[r][j] = items of digit r in blocks before j) and its total.
__global__ void __launch_bounds__(kThreads) radix_digit_scan_kernel(
    const uint32_t* __restrict__ hist, int nblk, uint32_t* __restrict__ hist_off,
    uint32_t* __restrict__ digit_tot) {
  __shared__ uint32_t s_wave[33];
  const uint32_t* h = hist + (int64_t)blockIdx.x * nblk;
  uint32_t* o = hist_off + (int64_t)blockIdx.x * nblk;
  uint32_t carry = 0;
  for (int base = 0; base < nblk; base += kThreads * 4) {
    const int b0 = base + threadIdx.x * 4;  // four consecutive blocks per thread
    uint32_t v[4];
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = b0 + j < nblk ? h[b0 + j] : 0u;
      acc += v[j];
    }
    uint32_t tot;
    uint32_t run = carry + block_exclusive(acc, s_wave, &tot);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (b0 + j < nblk) o[b0 + j] = run;
      run += v[j];
    }
    carry += tot;
  }
  if (threadIdx.x == 0) digit_tot[blockIdx.x] = carry;
}

// Each block starts digit r at (items of smaller digits) + hist_off[r][block]:
// the digit bases are an exclusive scan of the digit totals, made by every
// block in LDS (two digits per thread), so a pass needs no separate scan of
// the digits.
static_assert(kRadix == 2 * kThreads, "two digits per thread in the digit-base scan");

__global__ void __launch_bounds__(kThreads) radix_scatter_kernel(
    const uint32_t* __restrict__ keys_in, const uint32_t* __restrict__ vals_in, int64_t n,
    Digits d, const uint32_t* __restrict__ hist_off, const uint32_t* __restrict__ digit_tot,
    int nblk, uint32_t* __restrict__ keys_out, uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t s_run[kRadix];                   // placed so far, per digit
  __shared__ uint32_t s_wc[kThreads / kWave][kRadix];  // this pass, per wave, per digit
  __shared__ uint32_t s_wave[33];
  const int t = threadIdx.x;
  const int w = t / kWave;
  {
    const uint32_t c0 = digit_tot[2 * t], c1 = digit_tot[2 * t + 1];
    const uint32_t o0 = hist_off[(int64_t)(2 * t) * nblk + blockIdx.x];
    const uint32_t o1 = hist_off[(int64_t)(2 * t + 1) * nblk + blockIdx.x];
    uint32_t tot;
    const uint32_t base = block_exclusive(c0 + c1, s_wave, &tot);
    s_run[2 * t] = base + o0;
    s_run[2 * t + 1] = base + c0 + o1;
  }
  const int64_t base = blockIdx.x * (int64_t)kTile;
  for (int j = 0; j < kItems; ++j) {
    for (int r = t; r < kRadix; r += kThreads)
#pragma unroll
      for (int ww = 0; ww < kThreads / kWave; ++ww) s_wc[ww][r] = 0;
    __syncthreads();
    const int64_t i = base + j * kThreads + t;  // items stay in index order
    const bool valid = i < n;
    const uint32_t val = valid ? vals_in[i] : 0u;
    const uint32_t key = (valid && keys_in) ? keys_in[i] : 0u;
    const uint32_t dg = valid ? digit_of(d, i, val) : 0u;
    // lanes of this wave holding the same digit
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kDigitBits; ++b) {
      const uint64_t ones = __ballot((dg >> b) & 1u);
      peers &= ((dg >> b) & 1u) ? ones : ~ones;
    }
    const int rank = rank_in_wave(peers);
    if (valid && rank == 0) s_wc[w][dg] = __popcll(peers);
    __syncthreads();
    if (valid) {
      uint32_t pos = s_run[dg] + rank;
      for (int ww = 0; ww < w; ++ww) pos += s_wc[ww][dg];
      if (pos < n) {  // always true when the digit offsets are consistent
        if (keys_out) keys_out[pos] = key;
        vals_out[pos] = val;
      }
    }
    __syncthreads();
    for (int r = t; r < kRadix; r += kThreads) {
      uint32_t add = 0;
#pragma unroll
      for (int ww = 0; ww < kThreads / kWave; ++ww) add += s_wc[ww][r];
      s_run[r] += add;
    }
    __syncthreads();
  }
}

// Short lists with keys of at most kDigitBits bits (a layer's full tiles, up
// to kSmallSortMax of them) are sorted by one workgroup in one launch instead
// of a radix pass's three: the digit counts in LDS and their scan, then
// rounds of kRadix items in index order, each item placed as in the radix
// scatter (lanes ranked by ballots, waves in order), so the sort is stable.
constexpr int64_t kSmallSortMax = int64_t(1) << 16;

__global__ void __launch_bounds__(kRadix) small_sort_kernel(const uint32_t* __restrict__ keys,
                                                            const uint32_t* __restrict__ vals,
                                                            int n, uint32_t* __restrict__ vals_out) {
  __shared__ uint32_t s_run[kRadix];                  // per digit: count, then next place
  __shared__ uint32_t s_wc[kRadix / kWave][kRadix];   // this round, per wave, per digit
  __shared__ uint32_t s_wave[33];
  const int t = threadIdx.x;  // also the digit whose counts this thread keeps
  const int w = t / kWave;
  s_run[t] = 0;
  __syncthreads();
  for (int i = t; i < n; i += kRadix) atomicAdd(&s_run[keys[i] & (kRadix - 1u)], 1u);
  __syncthreads();
  const uint32_t count = s_run[t];
  uint32_t tot;
  const uint32_t first = block_exclusive(count, s_wave, &tot);
  s_run[t] = first;
  for (int base = 0; base < n; base += kRadix) {
#pragma unroll
    for (int ww = 0; ww < kRadix / kWave; ++ww) s_wc[ww][t] = 0;
    __syncthreads();
    const int i = base + t;
    const bool valid = i < n;
    const uint32_t dg = valid ? keys[i] & (kRadix - 1u) : 0u;
    const uint32_t val = valid ? vals[i] : 0u;
    // lanes of this wave holding the same digit
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kDigitBits; ++b) {
      const uint64_t ones = __ballot((dg >> b) & 1u);
      peers &= ((dg >> b) & 1u) ? ones : ~ones;
    }
    const int rank = rank_in_wave(peers);
    if (valid && rank == 0) s_wc[w][dg] = __popcll(peers);
    __syncthreads();
    if (valid) {
      uint32_t pos = s_run[dg] + rank;
      for (int ww = 0; ww < w; ++ww) pos += s_wc[ww][dg];
      if (pos < static_cast<uint32_t>(n)) vals_out[pos] = val;  // always, with consistent counts
    }
    __syncthreads();
    uint32_t add = 0;
#pragma unroll
    for (int ww = 0; ww < kRadix / kWave; ++ww) add += s_wc[ww][t];
    s_run[t] += add;
  }
}

struct Buffers {
  uint32_t *keys_a, *keys_b, *vals_a, *vals_b, *rows, *mask_pos, *hist, *hist_off, *digit_tot;
  int32_t* nbr_t;  // the map's row-major copy (K <= 32), else null
};

Buffers carve(void* ws, int64_t n, int K, int64_t* used) {
  Carver c(ws);
  const int64_t m = n > 0 ? n : 1;
  const int64_t nblk = ceil_div(m, kTile);
  Buffers b;
  b.nbr_t = K <= 32 ? c.take<int32_t>(m * 32) : nullptr;
  b.keys_a = c.take<uint32_t>(m);
  b.keys_b = c.take<uint32_t>(m);
  b.vals_a = c.take<uint32_t>(m);
  b.vals_b = c.take<uint32_t>(m);
  b.rows = c.take<uint32_t>(m);
  b.mask_pos = c.take<uint32_t>(m);
  b.hist = c.take<uint32_t>(nblk * kRadix);
  b.hist_off = c.take<uint32_t>(nblk * kRadix);
  b.digit_tot = c.take<uint32_t>(kRadix);
  if (used) *used = c.used;
  return b;
}

// One stable pass: (keys, vals) in -> out, digits from d.
int radix_pass(const Buffers& b, const uint32_t* keys_in, const uint32_t* vals_in,
               uint32_t* keys_out, uint32_t* vals_out, int64_t n, const Digits& d,
               hipStream_t s) {
  const int nblk = static_cast<int>(ceil_div(n, kTile));
  radix_hist_kernel<<<nblk, kThreads, 0, s>>>(vals_in, n, d, b.hist, nblk);
  TSC_LAUNCH_CHECK("plan_hist");
  radix_digit_scan_kernel<<<kRadix, kThreads, 0, s>>>(b.hist, nblk, b.hist_off, b.digit_tot);
  TSC_LAUNCH_CHECK("plan_digit_scan");
  radix_scatter_kernel<<<nblk, kThreads, 0, s>>>(keys_in, vals_in, n, d, b.hist_off, b.digit_tot,
                                                 nblk, keys_out, vals_out);
  TSC_LAUNCH_CHECK("plan_scatter");
  return 0;
}

int bits_for(uint64_t v) {  // bits needed to hold values 0..v
  int b = 0;
  while (b < 64 && (uint64_t(1) << b) <= v) ++b;
  return b;
}

}  // namespace
}  // namespace tsc

using namespace tsc;

extern "C" int64_t tsc_plan_workspace_bytes(int64_t n_out, int32_t k_vol) {
  (void)k_vol;
  int64_t used = 0;
  carve(nullptr, n_out, k_vol, &used);
  return used;
}

extern "C" int tsc_conv_plan(const int32_t* nbr, const int32_t* cols_row, int32_t raster,
                             const int32_t* out_coords, int64_t n_out, int32_t k_vol,
                             int32_t batch_size, const int32_t out_spatial[3],
                             int64_t region_rows, void* ws, int64_t ws_bytes, int32_t* order,
                             int32_t* nbr_ordered, int32_t* pos_masks, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(n_out >= 0 && n_out < (int64_t(1) << 31), "plan: n_out out of range");
  TSC_REQUIRE(k_vol > 0 && batch_size > 0, "plan: invalid kernel volume or batch size");
  TSC_REQUIRE(region_rows > 0 && region_rows < (int64_t(1) << 31),
              "plan: region_rows must be positive");
  TSC_REQUIRE(out_spatial && out_spatial[0] > 0 && out_spatial[1] > 0 && out_spatial[2] > 0,
              "plan: spatial shape must be positive");
  if (n_out == 0) return 0;
  TSC_REQUIRE(nbr && order && ws && (raster || out_coords || region_rows >= n_out),
              "plan: null pointer");
  TSC_REQUIRE(ws_bytes >= tsc_plan_workspace_bytes(n_out, k_vol), "plan: workspace too small");
  TSC_REQUIRE(!pos_masks || k_vol <= 32, "plan: slot masks need k_vol <= 32 (got %d)", k_vol);
  Buffers b = carve(ws, n_out, k_vol, nullptr);
  int rc;
  // With one region the spatial order only breaks ties between equal slot
  // masks (the column order does that instead; measured on the 600k-row
  // inverse layer: the plan 0.30 -> 0.145 ms, its convolution 62 -> 65 us)
  if (region_rows >= n_out) raster = 1;

  // ---- sort 1: map columns by the Morton code of their rows (columns that
  // are already in (b,z,y,x) order, or that need no spatial order, keep it)
  if (raster) {
    // each column is its own Morton position: its slot mask goes straight to
    // mask_pos, with the positions as the values to sort
    if (b.nbr_t)
      map_rows_kernel<<<ceil_div(n_out, 256), 256, 0, s>>>(nbr, n_out, k_vol, b.nbr_t, b.mask_pos,
                                                           b.vals_a);
    else
      row_mask_kernel<<<ceil_div(n_out, 256), 256, 0, s>>>(nbr, n_out, k_vol, b.mask_pos, b.vals_a);
    TSC_LAUNCH_CHECK("plan_row_mask");
  } else {
    int extent = out_spatial[0];
    if (out_spatial[1] > extent) extent = out_spatial[1];
    if (out_spatial[2] > extent) extent = out_spatial[2];
    const int axis_bits = bits_for(static_cast<uint64_t>(extent - 1));
    const int coarse = axis_bits > 10 ? axis_bits - 10 : 0;
    int batch_bits = bits_for(static_cast<uint64_t>(batch_size - 1));
    if (batch_bits > 16) batch_bits = 16;  // more samples than that only coarsen the order
    const int batch_shift = 32 - batch_bits;
    spatial_key_kernel<<<ceil_div(n_out, 256), 256, 0, s>>>(
        reinterpret_cast<const int4*>(out_coords), cols_row, n_out, coarse, batch_shift, b.keys_a,
        b.vals_a);
    TSC_LAUNCH_CHECK("plan_spatial_key");
    uint32_t *ki = b.keys_a, *ko = b.keys_b, *vi = b.vals_a, *vo = b.vals_b;
    for (int p = 0; p < 4; ++p) {
      const Digits d{kFromKey, kDigitBits * p, ki, nullptr, 1u};
      uint32_t* vdst = (p == 3) ? b.rows : vo;  // the last pass leaves columns in Morton order
      if ((rc = radix_pass(b, ki, vi, ko, vdst, n_out, d, s))) return rc;
      std::swap(ki, ko);
      std::swap(vi, vo);
    }
  }

  // ---- sort 2: Morton positions by (region, mask), stable
  // the sort-1 keys are dead now: keys_a holds each column's slot mask,
  // keys_b the final column permutation
  if (!raster) {
    if (b.nbr_t)
      map_rows_kernel<<<ceil_div(n_out, 256), 256, 0, s>>>(nbr, n_out, k_vol, b.nbr_t, b.keys_a,
                                                           nullptr);
    else
      row_mask_kernel<<<ceil_div(n_out, 256), 256, 0, s>>>(nbr, n_out, k_vol, b.keys_a, nullptr);
    TSC_LAUNCH_CHECK("plan_row_mask");
    mask_at_pos_kernel<<<ceil_div(n_out, 256), 256, 0, s>>>(b.keys_a, n_out, b.rows, b.mask_pos,
                                                            b.vals_a);
    TSC_LAUNCH_CHECK("plan_mask");
  }
  uint32_t* vi = b.vals_a;
  uint32_t* vo = b.vals_b;
  const int mask_bits = k_vol < 32 ? k_vol : 32;
  const int64_t regions = ceil_div(n_out, region_rows);
  const int region_bits = bits_for(static_cast<uint64_t>(regions - 1));
  for (int p = 0; p < (mask_bits + kDigitBits - 1) / kDigitBits; ++p) {
    const Digits d{kFromMaskAtValue, kDigitBits * p, nullptr, b.mask_pos, 1u};
    if ((rc = radix_pass(b, nullptr, vi, nullptr, vo, n_out, d, s))) return rc;
    std::swap(vi, vo);
  }
  for (int p = 0; p < (region_bits + kDigitBits - 1) / kDigitBits; ++p) {
    const Digits d{kFromRegionOfValue, kDigitBits * p, nullptr, nullptr,
                   static_cast<uint32_t>(region_rows)};
    if ((rc = radix_pass(b, nullptr, vi, nullptr, vo, n_out, d, s))) return rc;
    std::swap(vi, vo);
  }
  // ---- sort 3: full tiles by (region, slots used, descending), stable.  The
  // row masks in keys_a are dead: it holds the tile keys, vo the tile ids.
  const int64_t n_tiles = n_out / kConvTileRows;
  const uint32_t* tile_perm = nullptr;
  if (n_tiles > 1) {
    const int64_t tiles_per_region =
        region_rows >= kConvTileRows ? region_rows / kConvTileRows : 1;
    tile_key_kernel<<<static_cast<unsigned>(n_tiles), kConvTileRows, 0, s>>>(
        vi, b.mask_pos, tiles_per_region, b.keys_a, vo);
    TSC_LAUNCH_CHECK("plan_tile_key");
    const int key_bits = bits_for(static_cast<uint64_t>((n_tiles - 1) / tiles_per_region)) + 6;
    uint32_t *tki = b.keys_a, *tko = b.keys_a + n_tiles, *tvi = vo, *tvo = vo + n_tiles;
    if (key_bits <= kDigitBits && n_tiles <= kSmallSortMax) {
      small_sort_kernel<<<1, kRadix, 0, s>>>(tki, tvi, static_cast<int>(n_tiles), tvo);
      TSC_LAUNCH_CHECK("plan_small_sort");
      tile_perm = tvo;
    } else {
      for (int p = 0; p < (key_bits + kDigitBits - 1) / kDigitBits; ++p) {
        const Digits d{kFromKey, kDigitBits * p, tki, nullptr, 1u};
        if ((rc = radix_pass(b, tki, tvi, tko, tvo, n_tiles, d, s))) return rc;
        std::swap(tki, tko);
        std::swap(tvi, tvo);
      }
      tile_perm = tvi;
    }
  }
  gather_rows_kernel<<<ceil_div(n_out, 256), 256, 0, s>>>(
      vi, raster ? nullptr : b.rows, cols_row, n_out, tile_perm, n_tiles, b.mask_pos, b.keys_b, order,
      reinterpret_cast<uint32_t*>(pos_masks));
  TSC_LAUNCH_CHECK("plan_gather");
  if (nbr_ordered && b.nbr_t) {
    permute_rows_kernel<<<static_cast<unsigned>(ceil_div(n_out, 256)), 256, 0, s>>>(
        b.nbr_t, b.keys_b, n_out, k_vol, nbr_ordered);
    TSC_LAUNCH_CHECK("plan_permute_rows");
  } else if (nbr_ordered) {
    // int4 accesses need 16-byte aligned rows of the map and of the order
    const bool vec = (n_out & 3) == 0 && (reinterpret_cast<uintptr_t>(nbr_ordered) & 15) == 0;
    const int64_t chunks = ceil_div(ceil_div(n_out, 4), 256);  // blocks per slot
    const int64_t blocks = 8 * ceil_div(k_vol, 8) * chunks;
    TSC_REQUIRE(blocks < (int64_t(1) << 31), "plan: map too large to permute");
    permute_map_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(
        nbr, b.keys_b, n_out, k_vol, static_cast<int>(chunks), vec ? 1 : 0, nbr_ordered);
    TSC_LAUNCH_CHECK("plan_permute_map");
  }
  return 0;
}
