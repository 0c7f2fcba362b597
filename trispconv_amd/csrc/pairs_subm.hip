// Submanifold indice pairs on the GPU.
//
// Reference algorithm: trispconv/pytorch/indices.py:67-140.  For slot k (kernel
// offsets in (kz,ky,kx) lexicographic order, measured from the kernel centre)
// and every output row r in ascending order, the pair (in = j, out = r) exists
// when coord(r) + offset_k lies inside the grid and is the coordinate of row j.
//
// MI355X design.  The build produces what the convolution consumes: the
// neighbour map as columns ([K][n], column t belongs to row cols_row[t]) and
// the per-slot pair counts.  The reference's dense grid-sized lookup table
// (:54-64) becomes one of two compact structures, chosen by how dense the
// active set is:
//   * occupancy bitmap (grids of up to about 2048 cells per voxel): one bit per
//     cell, an exclusive popcount scan of its words (each occupied cell's rank
//     in (b,z,y,x) order) and rank -> (row + 1, cell), one 8-byte entry per
//     column.  Columns are the occupied cells in rank order (then any earlier
//     rows of repeated coordinates), so a wave's 64 lookups touch neighbouring
//     cells and share cache lines, its map writes are contiguous, and a column
//     reads its own cell from its entry (no gather of its row's coordinates).  Where the grid has at most 64 cells per row, or at most
//     2^22 cells, the bits are first marked as one byte per cell with plain
//     stores (the build's generation value, so marks a caller keeps between
//     builds need no zeroing) and packed by the scan; sparser grids set them
//     with atomics;
//   * open-addressing hash of 2N..4N 64-bit slots otherwise, probed in row
//     order (columns are rows).
// The reference's pair lists are derived from the map only when asked for
// (tsc_map_to_rows, tsc_pairs_from_map): per-(slot, block) counts, a per-slot
// scan and a wave-ballot compaction put every slot's list in ascending
// output-row order, exactly the reference's order.  Repeated coordinates
// resolve to the later row, as the reference's table scatter leaves them.
#include "common.hpp"

#include <algorithm>

namespace tsc {
namespace {

constexpr int kRows = 256;  // output rows per block in probe and fill

struct SubmGeom {
  int32_t B;
  Box shape, ks, dil;
  uint32_t mask;  // hash capacity - 1
};

__device__ __forceinline__ bool in_grid(const SubmGeom& g, int b, int z, int y, int x) {
  return b >= 0 && b < g.B && z >= 0 && z < g.shape.z && y >= 0 && y < g.shape.y && x >= 0 &&
         x < g.shape.x;
}

__device__ __forceinline__ uint32_t cell_key(const SubmGeom& g, int b, int z, int y, int x) {
  return ((static_cast<uint32_t>(b) * g.shape.z + z) * g.shape.y + y) * g.shape.x + x;
}

// (b, z, y, x) of a cell key.
__device__ __forceinline__ int4 cell_coords(const SubmGeom& g, uint32_t cell) {
  const uint32_t x = cell % static_cast<uint32_t>(g.shape.x);
  cell /= static_cast<uint32_t>(g.shape.x);
  const uint32_t y = cell % static_cast<uint32_t>(g.shape.y);
  cell /= static_cast<uint32_t>(g.shape.y);
  const uint32_t z = cell % static_cast<uint32_t>(g.shape.z);
  return make_int4(static_cast<int>(cell / static_cast<uint32_t>(g.shape.z)), static_cast<int>(z),
                   static_cast<int>(y), static_cast<int>(x));
}

// A row outside the grid: its status flag on the device and, when a caller
// waits for the check instead of for the whole build, a non-zero word in
// pinned host memory (a plain store; every writer stores 1).
__device__ __forceinline__ void flag_bad_row(const SubmGeom& g, int b, int32_t* status,
                                             int32_t* host_flag) {
  atomicOr(status, (b < 0 || b >= g.B) ? TSC_FLAG_BATCH_OUT_OF_RANGE : TSC_FLAG_COORD_OUT_OF_GRID);
  if (host_flag) __hip_atomic_store(host_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A map column of the bitmap path is one 8-byte entry: x = its row + 1 (0
// while unassigned; repeated cells keep the largest row by atomicMax on x)
// and y = its cell key.

__global__ void __launch_bounds__(256) subm_insert_kernel(const int4* __restrict__ coords,
                                                          int64_t n, SubmGeom g,
                                                          unsigned long long* table,
                                                          int32_t* status, int32_t* host_flag) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int4 c = coords[r];  // (b, z, y, x)
  if (!in_grid(g, c.x, c.y, c.z, c.w)) {
    flag_bad_row(g, c.x, status, host_flag);
    return;
  }
  hash_insert(table, g.mask, cell_key(g, c.x, c.y, c.z, c.w), static_cast<uint32_t>(r));
}

// One thread per output row.  Slots are processed in groups of kGroup: the
// first probe of every slot in the group is issued before any is inspected,
// so a thread keeps kGroup independent hash reads in flight; collisions are
// then followed slot by slot.  The map is slot-major ([K][n]), so for each
// slot a wave writes 64 consecutive entries.
constexpr int kGroup = 16;

__global__ void __launch_bounds__(kRows) subm_probe_kernel(const int4* __restrict__ coords,
                                                           int64_t n, int K, SubmGeom g,
                                                           const unsigned long long* __restrict__ table,
                                                           int32_t* __restrict__ nbr,
                                                           int32_t* __restrict__ blk_cnt,
                                                           int nblk, int32_t* started) {
  __shared__ int32_t s_cnt[kRows / kWave][64];  // per wave, per slot (slots < 64)
  signal_started(started);
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int64_t r = blockIdx.x * (int64_t)kRows + t;
  const bool valid = r < n;
  const int4 c = valid ? coords[r] : make_int4(-1, 0, 0, 0);
  const bool self_ok = valid && in_grid(g, c.x, c.y, c.z, c.w);

  for (int kb = 0; kb < K; kb += kGroup) {
    uint32_t key[kGroup], h[kGroup];
    unsigned long long word[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      const int k = kb + i;
      int kz, ky, kx;
      slot_to_zyx(k < K ? k : 0, g.ks, kz, ky, kx);
      const int z = c.y + (kz - g.ks.z / 2) * g.dil.z;
      const int y = c.z + (ky - g.ks.y / 2) * g.dil.y;
      const int x = c.w + (kx - g.ks.x / 2) * g.dil.x;
      const bool look = self_ok && k < K && in_grid(g, c.x, z, y, x);
      key[i] = look ? cell_key(g, c.x, z, y, x) : 0u;
      h[i] = hash32(key[i]) & g.mask;
      // unconditional read (slot h is always inside the table) so the group's
      // reads issue back to back; a slot that needs no lookup is then marked
      // empty
      const unsigned long long wv = table[h[i]];
      word[i] = look ? wv : kEmpty;
    }
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      const int k = kb + i;
      int32_t j = -1;
      while (word[i] != kEmpty) {
        if (static_cast<uint32_t>(word[i] >> 32) == key[i]) {
          j = static_cast<int32_t>(word[i] & 0xffffffffu);
          break;
        }
        h[i] = (h[i] + 1) & g.mask;
        word[i] = table[h[i]];
      }
      if (k < K) {
        const uint64_t hits = __ballot(j >= 0);
        if (valid) nbr[(int64_t)k * n + r] = j;
        if (__lane_id() == 0) {
          if (k < 64)
            s_cnt[w][k] = __popcll(hits);
          else  // K > 64: fold straight into the global count
            atomicAdd(&blk_cnt[(int64_t)k * nblk + blockIdx.x], (int)__popcll(hits));
        }
      }
    }
  }
  __syncthreads();
  if (t < K && t < 64) {
    int sum = 0;
#pragma unroll
    for (int ww = 0; ww < kRows / kWave; ++ww) sum += s_cnt[ww][t];
    blk_cnt[(int64_t)t * nblk + blockIdx.x] = sum;
  }
}

// ------------------------------------------------------ 64-bit cell keys --
// Grids of 2^32 - 1 cells or more (the reference's int64 keys, indices.py:45-51,
// work for any grid): an open-addressing table of 64-bit keys with the rows in
// a parallel int32 array (-1 = none), linear probing from a 64-bit murmur3
// finaliser.  Repeated coordinates keep the largest row, as the reference's
// table scatter over rows in order leaves them.
__device__ __forceinline__ uint64_t cell_key64(const SubmGeom& g, int b, int z, int y, int x) {
  return ((static_cast<uint64_t>(b) * g.shape.z + z) * g.shape.y + y) * g.shape.x + x;
}

__device__ __forceinline__ uint32_t hash64(uint64_t k) {
  k ^= k >> 33;
  k *= 0xff51afd7ed558ccdull;
  k ^= k >> 33;
  k *= 0xc4ceb9fe1a85ec53ull;
  k ^= k >> 33;
  return static_cast<uint32_t>(k);
}

__global__ void __launch_bounds__(256) subm_insert_wide_kernel(const int4* __restrict__ coords,
                                                               int64_t n, SubmGeom g,
                                                               unsigned long long* keys,
                                                               int32_t* vals, int32_t* status,
                                                               int32_t* host_flag) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int4 c = coords[r];  // (b, z, y, x)
  if (!in_grid(g, c.x, c.y, c.z, c.w)) {
    flag_bad_row(g, c.x, status, host_flag);
    return;
  }
  const unsigned long long key = cell_key64(g, c.x, c.y, c.z, c.w);
  uint32_t h = hash64(key) & g.mask;
  while (true) {
    const unsigned long long old = atomicCAS(&keys[h], static_cast<unsigned long long>(kEmpty), key);
    if (old == kEmpty || old == key) {
      atomicMax(&vals[h], static_cast<int32_t>(r));  // later rows win
      return;
    }
    h = (h + 1) & g.mask;
  }
}

// One thread per output row; the first probe of every slot of a group is
// issued before any is inspected, then collisions are followed slot by slot.
__global__ void __launch_bounds__(kRows) subm_probe_wide_kernel(
    const int4* __restrict__ coords, int64_t n, int K, SubmGeom g,
    const unsigned long long* __restrict__ keys, const int32_t* __restrict__ vals,
    int32_t* __restrict__ nbr, int32_t* __restrict__ blk_cnt, int nblk, int32_t* started) {
  __shared__ int32_t s_cnt[kRows / kWave][64];  // per wave, per slot (slots < 64)
  signal_started(started);
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int64_t r = blockIdx.x * (int64_t)kRows + t;
  const bool valid = r < n;
  const int4 c = valid ? coords[r] : make_int4(-1, 0, 0, 0);
  const bool self_ok = valid && in_grid(g, c.x, c.y, c.z, c.w);
  for (int kb = 0; kb < K; kb += kGroup) {
    unsigned long long key[kGroup], kw[kGroup];
    uint32_t h[kGroup];
    bool look[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      const int k = kb + i;
      int kz, ky, kx;
      slot_to_zyx(k < K ? k : 0, g.ks, kz, ky, kx);
      const int z = c.y + (kz - g.ks.z / 2) * g.dil.z;
      const int y = c.z + (ky - g.ks.y / 2) * g.dil.y;
      const int x = c.w + (kx - g.ks.x / 2) * g.dil.x;
      look[i] = self_ok && k < K && in_grid(g, c.x, z, y, x);
      key[i] = look[i] ? cell_key64(g, c.x, z, y, x) : 0ull;
      h[i] = hash64(key[i]) & g.mask;
      kw[i] = keys[h[i]];  // slot h is inside the table: unconditional reads
    }
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      const int k = kb + i;
      int32_t j = -1;
      if (look[i]) {
        while (kw[i] != kEmpty) {
          if (kw[i] == key[i]) {
            j = vals[h[i]];
            break;
          }
          h[i] = (h[i] + 1) & g.mask;
          kw[i] = keys[h[i]];
        }
      }
      if (k < K) {
        const uint64_t hits = __ballot(j >= 0);
        if (valid) nbr[(int64_t)k * n + r] = j;
        if (__lane_id() == 0) {
          if (k < 64)
            s_cnt[w][k] = __popcll(hits);
          else
            atomicAdd(&blk_cnt[(int64_t)k * nblk + blockIdx.x], (int)__popcll(hits));
        }
      }
    }
  }
  __syncthreads();
  if (t < K && t < 64) {
    int sum = 0;
#pragma unroll
    for (int ww = 0; ww < kRows / kWave; ++ww) sum += s_cnt[ww][t];
    blk_cnt[(int64_t)t * nblk + blockIdx.x] = sum;
  }
}

// ------------------------------------------------------------ bitmap path --
// One 8-byte entry per 32 cells: x = occupancy bits, y = rank of the word's
// first cell (occupied cells before it in (b,z,y,x) order), so a lookup is
// one load.

// Zeroes the occupancy marks (bitmap entries or the byte map, as 16-byte
// units) and the counters, in one launch.
__global__ void __launch_bounds__(256) subm_init_kernel(uint4* __restrict__ wr2, int64_t n_pairs,
                                                        int32_t* __restrict__ counts, int K,
                                                        int32_t* __restrict__ n_extra) {
  const int64_t i0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = i0; i < n_pairs; i += stride) wr2[i] = make_uint4(0u, 0u, 0u, 0u);
  if (blockIdx.x == 0) {
    for (int k = threadIdx.x; k < K + 2; k += blockDim.x)
      counts[k] = k == K + 1 ? 1 : 0;  // counts[K + 1] = 1: columns in (b,z,y,x) order
    if (threadIdx.x == 0) *n_extra = 0;
  }
}

// Marks each row's cell occupied; rows outside the grid only raise a status
// flag.  Also marks every column unassigned (the rank pass fills them in) and
// clears the count of repeated rows the rank pass takes.
// BYTES: byte marks (common.hpp): the cell's byte and a bad row's status word
// receive the build's generation value gen by plain stores (every writer
// stores the same value, so races are harmless); the scan packs the bytes
// equal to gen into the bitmap, and the rank pass turns the status words
// into the status flags.  Otherwise the cell's bit is set by a device-scope
// atomicOr, which on this part is carried out beyond the XCD's L2 (the L2s
// are not coherent with each other): several times the cost of the byte
// store and the packing pass together, taken only where the byte map would
// be large (sparse grids); bad rows raise their flag in *status.
template <bool BYTES>
__global__ void __launch_bounds__(256) subm_mark_kernel(const int4* __restrict__ coords, int64_t n,
                                                        SubmGeom g, uint2* wr,
                                                        uint8_t* __restrict__ bytes,
                                                        uint32_t* __restrict__ mark_words,
                                                        uint32_t gen, int32_t* status,
                                                        int32_t* host_flag,
                                                        uint2* __restrict__ col,
                                                        int32_t* __restrict__ n_extra) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r == 0) *n_extra = 0;
  if (r >= n) return;
  col[r] = make_uint2(0u, 0u);  // whole entries: no partly written sectors
  const int4 c = coords[r];
  if (!in_grid(g, c.x, c.y, c.z, c.w)) {
    if constexpr (BYTES) {
      mark_words[(c.x < 0 || c.x >= g.B) ? kMarkBatch : kMarkGrid] = gen;
      if (host_flag) __hip_atomic_store(host_flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    } else {
      flag_bad_row(g, c.x, status, host_flag);
    }
    return;
  }
  const uint32_t cell = cell_key(g, c.x, c.y, c.z, c.w);
  if constexpr (BYTES)
    bytes[cell] = static_cast<uint8_t>(gen);
  else
    atomicOr(&wr[cell >> 5].x, 1u << (cell & 31));
}

// Bitmaps marked by atomics (sparse grids): only the tiles of
// kBitmapTileWords words that hold a row's cell are zeroed, scanned and
// ranked.  touched[tile] = 1 for each row's tile (plain stores: every writer
// stores 1); rows outside the grid are skipped (the mark flags them).
__global__ void __launch_bounds__(256) subm_touch_kernel(const int4* __restrict__ coords, int64_t n,
                                                         SubmGeom g, uint8_t* __restrict__ touched) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int4 c = coords[r];
  if (!in_grid(g, c.x, c.y, c.z, c.w)) return;
  touched[(cell_key(g, c.x, c.y, c.z, c.w) >> 5) / kBitmapTileWords] = 1;
}

// One block per tile: the entries of a touched tile are zeroed (the others
// are never read).  Entry pairs past the bitmap's end are its padding, also
// zeroed while they lie in the last tile.
__global__ void __launch_bounds__(256) subm_zero_touched_kernel(uint4* __restrict__ wr2,
                                                                int64_t n_pairs,
                                                                const uint8_t* __restrict__ touched) {
  if (!touched[blockIdx.x]) return;
  const int64_t p0 = blockIdx.x * (int64_t)(kBitmapTileWords / 2);
#pragma unroll
  for (int j = 0; j < kBitmapTileWords / 2 / 256; ++j) {
    const int64_t p = p0 + j * 256 + threadIdx.x;
    if (p < n_pairs) wr2[p] = make_uint4(0u, 0u, 0u, 0u);
  }
}

// A bitmap entry, read as empty where its tile is untouched (touched may be
// null: every tile is initialised).  The entry is loaded either way (the
// address is in the bitmap) and the value selected, so the loads stay
// unconditional.
__device__ __forceinline__ uint2 entry_at(const uint2* __restrict__ wr,
                                          const uint8_t* __restrict__ touched, uint32_t w) {
  const uint2 e = wr[w];
  return (!touched || touched[w / kBitmapTileWords]) ? e : make_uint2(0u, 0u);
}

// Rank of an occupied cell: occupied cells before it in (b,z,y,x) order.
__device__ __forceinline__ uint32_t cell_rank(uint2 e, uint32_t cell) {
  return e.y + __popc(e.x & ((1u << (cell & 31)) - 1u));
}

// Column (rank of the row's cell) = the largest row with that cell, and the
// cell.  When every row has a cell of its own (n_unique == n) the ranks are
// distinct and plain stores do.  Otherwise repeated cells keep the largest
// row by atomicMax (entries start at 0; every writer stores the same cell),
// and every row that is not its cell's largest gets a column of its own
// after the n_unique cell columns (in no particular order; the values
// computed for it do not depend on where it sits).  The value atomicMax
// returns names such a row exactly once: a row that finds a larger row
// already there places itself; a row that finds a smaller one displaces
// that row, which then never returns as the maximum, and places it.
// With byte marks (mark_words), thread 0 also writes the status flags and
// the column-order flag: counts[K] = mark_flags, counts[K + 1] = 1.
__global__ void __launch_bounds__(256) subm_rank_kernel(const int4* __restrict__ coords, int64_t n,
                                                        SubmGeom g, const uint2* __restrict__ wr,
                                                        const int32_t* __restrict__ n_unique,
                                                        uint2* col, int32_t* n_extra,
                                                        const uint32_t* __restrict__ mark_words,
                                                        uint32_t gen, int32_t* __restrict__ counts,
                                                        int K) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r == 0 && mark_words) {
    counts[K] = mark_flags(mark_words, gen);
    counts[K + 1] = 1;
  }
  if (r >= n) return;
  const int32_t nu = *n_unique;
  const int4 c = coords[r];
  if (!in_grid(g, c.x, c.y, c.z, c.w)) return;
  const uint32_t cell = cell_key(g, c.x, c.y, c.z, c.w);
  const uint32_t rank = cell_rank(wr[cell >> 5], cell);
  const uint32_t me = static_cast<uint32_t>(r + 1);
  if (nu == n) {
    col[rank] = make_uint2(me, cell);
    return;
  }
  col[rank].y = cell;
  const uint32_t old = atomicMax(&col[rank].x, me);
  if (old == 0u) return;                   // the first row of its cell so far
  const uint32_t loser = old > me ? me : old;
  const int32_t c2 = nu + atomicAdd(n_extra, 1);  // < rows in the grid <= n
  col[c2] = make_uint2(loser, cell);
}

// Per-slot hit counts of the probes: per wave by ballot, per block in LDS.
// With a per-block table (blk_cnt, [K][nblk]) each block stores its counts
// there and a small kernel sums them; without one (the build on a strided
// output's bitmap has no workspace) each block adds them to counts.  Slots
// from 64 on are added per wave into the block's entry (zeroed beforehand)
// or into counts.
__device__ __forceinline__ int32_t* slot_counter(int k, int32_t* blk_cnt, int nblk,
                                                 int32_t* counts) {
  return blk_cnt ? &blk_cnt[(int64_t)k * nblk + blockIdx.x] : &counts[k];
}

__device__ __forceinline__ void count_hit(int k, bool hit, int32_t* s_cnt, int32_t* blk_cnt,
                                          int nblk, int32_t* counts) {
  const uint64_t hits = __ballot(hit);
  if (__lane_id() == 0 && hits) {
    if (k < 64)
      atomicAdd(&s_cnt[k], (int)__popcll(hits));
    else
      atomicAdd(slot_counter(k, blk_cnt, nblk, counts), (int)__popcll(hits));
  }
}

// One thread per map column (an occupied cell in rank order, or a repeated
// row after them): the column gets its row's K neighbours.  Eight slots'
// bitmap reads are in flight together, then their rank -> row reads.
constexpr int kLook = 8;

__global__ void __launch_bounds__(256) subm_probe_cols_kernel(
    int64_t n, int K, SubmGeom g, const uint2* __restrict__ wr,
    const uint2* __restrict__ col_e, const int32_t* __restrict__ n_unique,
    const int32_t* __restrict__ n_extra, int32_t* __restrict__ cols_row, int32_t* __restrict__ nbr,
    int32_t* __restrict__ blk_cnt, int nblk, int32_t* __restrict__ counts,
    uint32_t* __restrict__ col_masks, const uint8_t* __restrict__ touched) {
  __shared__ int32_t s_cnt[64];
  const int t = threadIdx.x;
  if (t < 64) s_cnt[t] = 0;
  __syncthreads();
  const int64_t col = blockIdx.x * (int64_t)blockDim.x + t;
  const bool live = col < *n_unique + *n_extra;  // the other columns are empty
  const uint2 me = live ? col_e[col] : make_uint2(0u, 0u);
  if (col < n) cols_row[col] = static_cast<int32_t>(me.x) - 1;
  const int4 c = cell_coords(g, me.y);
  uint32_t cmask = 0;  // the column's slot mask (slots below 32)
  for (int k0 = 0; k0 < K; k0 += kLook) {
    uint32_t cell[kLook];
    uint2 e[kLook];
    bool look[kLook];
#pragma unroll
    for (int i = 0; i < kLook; ++i) {
      const int k = k0 + i;
      int kz, ky, kx;
      slot_to_zyx(k < K ? k : 0, g.ks, kz, ky, kx);
      const int z = c.y + (kz - g.ks.z / 2) * g.dil.z;
      const int y = c.z + (ky - g.ks.y / 2) * g.dil.y;
      const int x = c.w + (kx - g.ks.x / 2) * g.dil.x;
      look[i] = live && k < K && in_grid(g, c.x, z, y, x);
      cell[i] = look[i] ? cell_key(g, c.x, z, y, x) : 0u;
      e[i] = entry_at(wr, touched, cell[i] >> 5);  // entry 0 exists: unconditional reads
    }
    int32_t jr[kLook];
#pragma unroll
    for (int i = 0; i < kLook; ++i) {
      const bool hit = look[i] && ((e[i].x >> (cell[i] & 31)) & 1u);
      // a hit's rank is below n_unique <= n; a miss reads column 0
      jr[i] = static_cast<int32_t>(col_e[hit ? cell_rank(e[i], cell[i]) : 0u].x) - 1;
      if (!hit) jr[i] = -1;
    }
#pragma unroll
    for (int i = 0; i < kLook; ++i) {
      const int k = k0 + i;
      if (k >= K) continue;
      if (col < n) nbr[(int64_t)k * n + col] = jr[i];
      cmask |= (jr[i] >= 0 && k < 32 ? 1u : 0u) << (k & 31);
      count_hit(k, jr[i] >= 0, s_cnt, blk_cnt, nblk, counts);
    }
  }
  if (col_masks && col < n) col_masks[col] = cmask;
  __syncthreads();
  if (t < K && t < 64) {
    if (blk_cnt)
      blk_cnt[(int64_t)t * nblk + blockIdx.x] = s_cnt[t];
    else if (s_cnt[t])
      atomicAdd(&counts[t], s_cnt[t]);
  }
}

// The same for kernels KX cells wide whose x extent (KX - 1) * dil.x + 1 is at
// most 32 cells: the KX cells of one (kz, ky) row then lie in two consecutive
// bitmap entries, so a row costs two 8-byte loads instead of KX.  All rows'
// entries are loaded before any rank -> row read.  KZ, KY > 0 fix the kernel's
// other extents at compile time (3x3x3: no division, fully unrolled); 0 reads
// them from g.  With K <= 64 slots a wave counts its hits with one lane per
// slot (lane k adds the popcount of slot k's ballot), so counting needs no
// branch per slot; larger kernels add each ballot to counts from lane 0.
//
// IDENT: the rows themselves are the occupied cells in rank order (row t has
// rank t, no repeats: a strided build's sorted output and its bitmap), so the
// columns are the rows, a row's cell comes from rows_coords and a hit's row
// is its rank.
//
// With dil.x == 1 the hits of one kernel row are consecutive cells, so their
// ranks are consecutive too: the columns of a run of up to three hits lie in
// the four entries from (first rank & ~1), two aligned 16-byte loads, instead
// of one load per hit.  The column array carries 4 entries of padding for
// them.  Three kernel rows are processed at a time, which keeps the kernel
// at eight waves per SIMD.
template <int KX, int KZ, int KY, bool IDENT>
__global__ void __launch_bounds__(256) subm_probe_rows_kernel(
    int64_t n, int K, SubmGeom g, const uint2* __restrict__ wr, int64_t nw,
    const uint2* __restrict__ col_e, const int4* __restrict__ rows_coords,
    const int32_t* __restrict__ n_unique, const int32_t* __restrict__ n_extra,
    int32_t* __restrict__ cols_row, int32_t* __restrict__ nbr, int32_t* __restrict__ blk_cnt,
    int nblk, int32_t* __restrict__ counts, uint32_t* __restrict__ col_masks,
    const uint8_t* __restrict__ touched) {
  constexpr bool kStatic = KZ > 0 && KY > 0;
  constexpr int kRowsAtOnce = kStatic ? KY : 3;  // rows whose entries load together
  // the fixed-extent path stores whole batches without a row bound
  static_assert(!kStatic || (KZ * KY) % kRowsAtOnce == 0, "row batches must tile the kernel");
  __shared__ int32_t s_cnt[kRows / kWave][64];
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const int64_t col = blockIdx.x * (int64_t)blockDim.x + t;
  int4 c;
  bool live;
  if constexpr (IDENT) {
    live = col < n;
    c = live ? rows_coords[col] : make_int4(0, 0, 0, 0);
    if (live) cols_row[col] = static_cast<int32_t>(col);
  } else {
    live = col < *n_unique + *n_extra;  // the other columns are empty
    const uint2 me = live ? col_e[col] : make_uint2(0u, 0u);
    if (col < n) cols_row[col] = static_cast<int32_t>(me.x) - 1;
    c = cell_coords(g, me.y);
  }
  const int ksz = kStatic ? KZ : g.ks.z;
  const int ksy = kStatic ? KY : g.ks.y;
  const int n_rows = ksz * ksy;
  const bool lane_counts = (kStatic && KZ * KY * KX <= kWave) || K <= kWave;
  int32_t my_cnt = 0;  // lane k: the wave's hits through slot k
  uint32_t cmask = 0;  // the column's slot mask (slots below 32)
  const int x_lo = c.w - (KX / 2) * g.dil.x;                 // the row's first cell
  const int x_first = x_lo > 0 ? x_lo : 0;                   // first cell inside the grid
  for (int q0 = 0; q0 < n_rows; q0 += kRowsAtOnce) {
    uint32_t base[kRowsAtOnce];
    bool row_ok[kRowsAtOnce];
    uint2 e0[kRowsAtOnce], e1[kRowsAtOnce];
#pragma unroll
    for (int i = 0; i < kRowsAtOnce; ++i) {
      const int q = q0 + i;
      const int kz = q / ksy, ky = q % ksy;
      const int z = c.y + (kz - ksz / 2) * g.dil.z;
      const int y = c.z + (ky - ksy / 2) * g.dil.y;
      row_ok[i] = live && q < n_rows && in_grid(g, c.x, z, y, x_first);
      base[i] = row_ok[i] ? cell_key(g, c.x, z, y, x_first) : 0u;  // key of x_first
      const uint32_t w0 = base[i] >> 5;
      e0[i] = entry_at(wr, touched, w0);
      e1[i] = entry_at(wr, touched, w0 + 1 < nw ? w0 + 1 : w0);
    }
    int32_t jr[kRowsAtOnce][KX];
    bool hit[kRowsAtOnce][KX];
    uint32_t rank[kRowsAtOnce][KX];
#pragma unroll
    for (int i = 0; i < kRowsAtOnce; ++i) {
#pragma unroll
      for (int kx = 0; kx < KX; ++kx) {
        const int x = x_lo + kx * g.dil.x;
        const bool ok = row_ok[i] && x >= 0 && x < g.shape.x;
        const uint32_t off = (base[i] & 31u) + static_cast<uint32_t>(x - x_first);  // < 64
        const uint2 e = off < 32u ? e0[i] : e1[i];
        const uint32_t b = off & 31u;
        hit[i][kx] = ok && ((e.x >> b) & 1u);
        rank[i][kx] = e.y + __popc(e.x & ((1u << b) - 1u));
      }
    }
    if constexpr (IDENT) {
      // the kernel row through the row's own cell (offset 0 on every axis:
      // slot ks/2 of each extent)
      const int q_self = (ksz / 2) * ksy + ksy / 2;
#pragma unroll
      for (int i = 0; i < kRowsAtOnce; ++i)
#pragma unroll
        for (int kx = 0; kx < KX; ++kx) {
          // a rank outside the rows: the rows are not the bitmap's cells
          const bool beyond = hit[i][kx] && rank[i][kx] >= static_cast<uint64_t>(n);
          // the row's own cell must be occupied and carry the row's own rank;
          // with no rank beyond n either, the rows are exactly the first n
          // occupied cells in rank order (a permuted or foreign row set fails)
          const bool self_bad = live && q0 + i == q_self && kx == KX / 2 &&
                                !(hit[i][kx] && rank[i][kx] == static_cast<uint64_t>(col));
          if (beyond || self_bad) atomicOr(&counts[K], TSC_FLAG_ROWS_NOT_BITMAP);
          if (beyond) hit[i][kx] = false;
          jr[i][kx] = hit[i][kx] ? static_cast<int32_t>(rank[i][kx]) : -1;
        }
    } else if (g.dil.x != 1) {
      // dilated rows skip cells, so other occupied cells can sit between the
      // hits: one load per hit
#pragma unroll
      for (int i = 0; i < kRowsAtOnce; ++i)
#pragma unroll
        for (int kx = 0; kx < KX; ++kx)
          jr[i][kx] = hit[i][kx] ? static_cast<int32_t>(col_e[rank[i][kx]].x) - 1 : -1;
    } else {
      // the row's first hit has the lowest rank; the others follow it
      static_assert(KX <= 3, "a run of hits must fit four entries");
      uint4 lo[kRowsAtOnce], hi[kRowsAtOnce];
      uint32_t at[kRowsAtOnce];
#pragma unroll
      for (int i = 0; i < kRowsAtOnce; ++i) {
        uint32_t first = 0u;
        bool any = false;
#pragma unroll
        for (int kx = KX - 1; kx >= 0; --kx) {
          first = hit[i][kx] ? rank[i][kx] : first;
          any = any || hit[i][kx];
        }
        at[i] = first & ~1u;  // < n_unique <= n: the window stays in the padded array
        const uint4* w = reinterpret_cast<const uint4*>(col_e + at[i]);
        lo[i] = w[0];  // entries at, at + 1
        // a run of up to three hits from first ends by entry (first & 1) + 2
        hi[i] = any && (first & 1u) + (KX - 1) >= 2u ? w[1] : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int i = 0; i < kRowsAtOnce; ++i)
#pragma unroll
        for (int kx = 0; kx < KX; ++kx) {
          const uint32_t d = rank[i][kx] - at[i];  // 0..3 for a hit
          const uint4 v = d < 2u ? lo[i] : hi[i];
          const uint32_t row1 = (d & 1u) ? v.z : v.x;
          jr[i][kx] = hit[i][kx] ? static_cast<int32_t>(row1) - 1 : -1;
        }
    }
#pragma unroll
    for (int i = 0; i < kRowsAtOnce; ++i) {
      const int q = q0 + i;
      if (!kStatic && q >= n_rows) continue;
#pragma unroll
      for (int kx = 0; kx < KX; ++kx) {
        const int k = q * KX + kx;
        const uint64_t hits = __ballot(jr[i][kx] >= 0);
        if (lane_counts)
          my_cnt += lane == k ? static_cast<int32_t>(__popcll(hits)) : 0;
        else if (lane == 0 && hits)
          atomicAdd(slot_counter(k, blk_cnt, nblk, counts), static_cast<int32_t>(__popcll(hits)));
      }
    }
    if (col < n) {  // the map stores, under one branch
#pragma unroll
      for (int i = 0; i < kRowsAtOnce; ++i) {
        const int q = q0 + i;
        if (!kStatic && q >= n_rows) continue;
#pragma unroll
        for (int kx = 0; kx < KX; ++kx) nbr[(int64_t)(q * KX + kx) * n + col] = jr[i][kx];
      }
    }
#pragma unroll
    for (int i = 0; i < kRowsAtOnce; ++i) {
      const int q = q0 + i;
      if (!kStatic && q >= n_rows) continue;
#pragma unroll
      for (int kx = 0; kx < KX; ++kx) {
        const int k = q * KX + kx;
        cmask |= (jr[i][kx] >= 0 && k < 32 ? 1u : 0u) << (k & 31);
      }
    }
  }
  if (col_masks && col < n) col_masks[col] = cmask;
  if (!lane_counts) return;
  s_cnt[t / kWave][lane] = my_cnt;
  __syncthreads();
  if (t < K) {
    int32_t sum = 0;
#pragma unroll
    for (int w = 0; w < kRows / kWave; ++w) sum += s_cnt[w][t];
    if (blk_cnt)
      blk_cnt[(int64_t)t * nblk + blockIdx.x] = sum;
    else if (sum)
      atomicAdd(&counts[t], sum);
  }
}

// The 3x3x3 kernel with dil.x == 1, for grids of fewer than 2^29 rows.  With
// every lane busy the probe is bound by its vector instructions (about 1,060
// per column in subm_probe_rows_kernel), not by its loads and stores, so this
// form spends far fewer.  A kernel row's three cells are consecutive cells of
// one bitmap word or two:
//  - one funnel shift of the two words gives the row's three occupancy bits
//    (h, bit kx for cell x - 1 + kx), masked by the x bounds (vmask, one per
//    column) and the row's z and y bounds (bit q of rv, one per column);
//  - the row's hits are consecutive occupied cells, so they have consecutive
//    ranks: the j-th hit in kx order has rank r0 + j, r0 the first hit's.
//    So the column entries r0, r0 + 1 and r0 + 2 are loaded unconditionally
//    (the column array carries 4 entries of padding) and picked by the bits
//    of h below kx; IDENT takes the ranks themselves;
//  - a slot's hit count is the popcount of its lane mask, and a row's three
//    counts go into one lane by a lane write; the slot mask is the rows' h
//    side by side.
// No store is under a lane condition, so the compiler keeps every load ahead
// of the stores: lanes past the last column work as the last column and
// store the same values to it, and the counts leave them out.  Loads and
// stores address a scalar base plus a 32-bit lane offset (the slot bases are
// opaque to the compiler, which would otherwise rebuild them per lane with
// 64-bit multiplies).  The map, its counts and its slot masks equal
// subm_probe_rows_kernel's.  TOUCHED: the entries of untouched tiles read as
// empty (the atomic-marked bitmap).
constexpr int64_t kProbe333Rows = int64_t(1) << 29;

template <bool IDENT, bool TOUCHED>
__global__ void __launch_bounds__(256) subm_probe_333_kernel(
    int64_t n, SubmGeom g, const uint2* __restrict__ wr, int64_t nw,
    const uint2* __restrict__ col_e, const int4* __restrict__ rows_coords,
    const int32_t* __restrict__ n_unique, const int32_t* __restrict__ n_extra,
    int32_t* __restrict__ cols_row, int32_t* __restrict__ nbr, int32_t* __restrict__ blk_cnt,
    int nblk, int32_t* __restrict__ counts, uint32_t* __restrict__ col_masks,
    const uint8_t* __restrict__ touched) {
  constexpr int K = 27;
  __shared__ int32_t s_cnt[kRows / kWave][9];
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1);
  const uint32_t un = static_cast<uint32_t>(n);  // 0 < n < 2^29
  const uint32_t col_t = blockIdx.x * static_cast<uint32_t>(kRows) + static_cast<uint32_t>(t);
  const uint64_t real = __ballot(col_t < un);  // lanes of real columns
  const uint32_t col = col_t < un ? col_t : un - 1;
  int4 c;  // (b, z, y, x)
  bool live;
  uint32_t key;
  if constexpr (IDENT) {
    live = true;
    c = rows_coords[col];
    key = cell_key(g, c.x, c.y, c.z, c.w);
    cols_row[col] = static_cast<int32_t>(col);
  } else {
    live = col < static_cast<uint32_t>(*n_unique + *n_extra);  // the other columns are empty
    const uint2 me = live ? col_e[col] : make_uint2(0u, 0u);
    cols_row[col] = static_cast<int32_t>(me.x) - 1;
    key = me.y;
    c = cell_coords(g, key);
  }
  // x: the row's cells are x - 1, x, x + 1; its first cell inside the grid
  // is x_first, shift = x_first - (x - 1)
  const int x_lo = c.w - 1;
  const int x_first = x_lo > 0 ? x_lo : 0;
  const uint32_t shift = static_cast<uint32_t>(x_first - x_lo) & 31u;
  const uint32_t W = static_cast<uint32_t>(g.shape.x);
  const uint32_t vmask = (static_cast<uint32_t>(x_lo) < W ? 1u : 0u) |
                         (static_cast<uint32_t>(c.w) < W ? 2u : 0u) |
                         (static_cast<uint32_t>(c.w + 1) < W ? 4u : 0u);
  const uint32_t key_first = key + static_cast<uint32_t>(x_first - c.w);
  // rows: bit kz * 3 + ky of rv when (b, z + (kz - 1) dz, y + (ky - 1) dy,
  // x_first) is inside the grid
  const bool col_ok = live && static_cast<uint32_t>(c.x) < static_cast<uint32_t>(g.B) &&
                      static_cast<uint32_t>(x_first) < W;
  const uint32_t D = static_cast<uint32_t>(g.shape.z), H = static_cast<uint32_t>(g.shape.y);
  const uint32_t yf = (static_cast<uint32_t>(c.z - g.dil.y) < H ? 1u : 0u) |
                      (static_cast<uint32_t>(c.z) < H ? 2u : 0u) |
                      (static_cast<uint32_t>(c.z + g.dil.y) < H ? 4u : 0u);
  uint32_t rv = (static_cast<uint32_t>(c.y - g.dil.z) < D ? yf : 0u) |
                (static_cast<uint32_t>(c.y) < D ? yf << 3 : 0u) |
                (static_cast<uint32_t>(c.y + g.dil.z) < D ? yf << 6 : 0u);
  rv = col_ok ? rv : 0u;
  const uint32_t plane = W * H;
  const uint32_t last_w = static_cast<uint32_t>(nw - 1);
  const char* const ce = reinterpret_cast<const char*>(col_e);
  const uint32_t col4 = col << 2;
  const uint64_t slot_bytes = static_cast<uint64_t>(n) * sizeof(int32_t);
  global_char* slot = (global_char*)nbr;
  uint32_t cmask = 0;
  int32_t my_cnt = 0;  // lane q: the wave's hits through slots 3q .. 3q + 2
  bool bad = false;    // IDENT: the rows are not the bitmap's cells
  auto kernel_row = [&](auto qc) {
    constexpr int q = decltype(qc)::value;
    constexpr int kz = q / 3, ky = q % 3;
    const uint32_t row_off = static_cast<uint32_t>((kz - 1) * g.dil.z) * plane +
                             static_cast<uint32_t>((ky - 1) * g.dil.y) * W;
    const uint32_t okm = static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int>(rv), q, 1));
    const uint32_t base = (key_first + row_off) & okm;  // cell 0 for rows outside the grid
    const uint32_t w0 = base >> 5;
    const uint32_t w1 = w0 + 1 < last_w ? w0 + 1 : last_w;  // past the last word: cells x >= W
    uint2 e0 = wr[w0], e1 = wr[w1];
    if constexpr (TOUCHED) {
      const bool t0 = touched[w0 / kBitmapTileWords], t1 = touched[w1 / kBitmapTileWords];
      e0 = t0 ? e0 : make_uint2(0u, 0u);
      e1 = t1 ? e1 : make_uint2(0u, 0u);
    }
    const uint32_t lo = base & 31u;  // the row's first cell's bit in e0
    const uint32_t bits = __builtin_amdgcn_alignbit(e1.x, e0.x, lo);
    uint32_t h = (bits << shift) & vmask & okm;
    // The first hit's rank.  An entry's rank field is only defined where its
    // pair of entries holds a set bit, so it comes from the entry holding the
    // hit: from e0 when a cell at or past the row's first one is set in e0
    // (where the row's cells reach into e1 they are e0's last cells, so such
    // a cell is the row's; cells masked by the x bound lie past any hit),
    // otherwise from e1, whose cells below the hit are the row's and empty.
    // Without a hit it is 0, so that the column loads stay in their array.
    // (A select by hand: as a C++ select the compiler branches around each
    // rank load and waits for it there, one memory round trip per row.)
    const uint32_t r_e0 = e0.y + __popc(e0.x & ~(0xffffffffu << lo));
    uint32_t r0 = select_lanes(__ballot((e0.x >> lo) != 0u), r_e0, e1.y);
    r0 = h ? r0 : 0u;
    int32_t jr0, jr1, jr2;
    if constexpr (IDENT) {
      // a hit ranked n or more: the rows are not the bitmap's cells; it is dropped
      if (r0 + static_cast<uint32_t>(__popc(h)) > un) {
        bad = true;
        uint32_t room = un > r0 ? un - r0 : 0u, kept = 0u;
#pragma unroll
        for (int kx = 0; kx < 3; ++kx)
          if ((h >> kx) & 1u) {
            if (room) {
              kept |= 1u << kx;
              --room;
            }
          }
        h = kept;
      }
      jr0 = (h & 1u) ? static_cast<int32_t>(r0) : -1;
      jr1 = (h & 2u) ? static_cast<int32_t>(r0 + (h & 1u)) : -1;
      jr2 = (h & 4u) ? static_cast<int32_t>(r0 + __popc(h & 3u)) : -1;
      // the row's own cell must be occupied and carry the row's own rank; with
      // no rank beyond n either, the rows are exactly the first n occupied
      // cells in rank order (a permuted or foreign row set fails)
      if (q == 4) bad = bad || jr1 != static_cast<int32_t>(col);
    } else {
      const uint32_t* v = reinterpret_cast<const uint32_t*>(ce + (r0 << 3));
      const int32_t m0 = static_cast<int32_t>(v[0]) - 1, m1 = static_cast<int32_t>(v[2]) - 1,
                    m2 = static_cast<int32_t>(v[4]) - 1;  // rows of ranks r0 .. r0 + 2
      const bool b0 = h & 1u, b1 = h & 2u;
      jr0 = b0 ? m0 : -1;
      jr1 = b1 ? (b0 ? m1 : m0) : -1;
      const int32_t u = b1 ? m1 : m0, w = b1 ? m2 : m1;
      jr2 = (h & 4u) ? (b0 ? w : u) : -1;
    }
    // a hit is a non-negative map entry (every occupied rank's column holds
    // its row + 1 >= 1), so the counts and the slot mask come from h; lane q
    // of my_cnt holds the row's three slot counts (at most 64 each) in
    // 10-bit fields
    const uint32_t c0 = static_cast<uint32_t>(__popcll(__ballot(h & 1u) & real));
    const uint32_t c1 = static_cast<uint32_t>(__popcll(__ballot(h & 2u) & real));
    const uint32_t c2 = static_cast<uint32_t>(__popcll(__ballot(h & 4u) & real));
    write_lane<q>(my_cnt, static_cast<int32_t>(c0 | (c1 << 10) | (c2 << 20)));
    cmask |= h << (3 * q);
    const int32_t jr[3] = {jr0, jr1, jr2};
#pragma unroll
    for (int kx = 0; kx < 3; ++kx) {
      *(global_int*)(slot + col4) = jr[kx];
      slot += slot_bytes;
      asm("" : "+s"(slot));
    }
  };
  for_each_index(kernel_row, std::make_integer_sequence<int, 9>{});
  if constexpr (IDENT) {
    if (bad) atomicOr(&counts[K], TSC_FLAG_ROWS_NOT_BITMAP);
  }
  if (col_masks) col_masks[col] = cmask;
  if (lane < 9) s_cnt[t / kWave][lane] = my_cnt;
  __syncthreads();
  if (t < K) {
    int32_t sum = 0;
#pragma unroll
    for (int w = 0; w < kRows / kWave; ++w) sum += (s_cnt[w][t / 3] >> (10 * (t % 3))) & 1023;
    if (blk_cnt)
      blk_cnt[(int64_t)t * nblk + blockIdx.x] = sum;
    else if (sum)
      atomicAdd(&counts[t], sum);
  }
}

// Row-order hit counts per (slot, block) of a row-major map, for the
// compaction offsets of the pair lists.
__global__ void __launch_bounds__(kRows) map_count_kernel(const int32_t* __restrict__ nbr, int64_t n,
                                                          int K, int32_t* __restrict__ blk_cnt,
                                                          int nblk) {
  __shared__ int32_t s_cnt[kRows / kWave][64];
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int64_t r = blockIdx.x * (int64_t)kRows + t;
  const bool valid = r < n;
  for (int k = 0; k < K; ++k) {
    const int32_t j = valid ? nbr[(int64_t)k * n + r] : -1;
    const uint64_t hits = __ballot(j >= 0);
    if (__lane_id() == 0) {
      if (k < 64)
        s_cnt[w][k] = __popcll(hits);
      else
        atomicAdd(&blk_cnt[(int64_t)k * nblk + blockIdx.x], (int)__popcll(hits));
    }
  }
  __syncthreads();
  if (t < K && t < 64) {
    int sum = 0;
#pragma unroll
    for (int ww = 0; ww < kRows / kWave; ++ww) sum += s_cnt[ww][t];
    blk_cnt[(int64_t)t * nblk + blockIdx.x] = sum;
  }
}

// nbr_rows[k][cols_row[t]] = nbr_cols[k][t]: the map back in row order.
// blockIdx.y is the slot, so the blocks in flight share one slot's rows.
__global__ void __launch_bounds__(256) map_to_rows_kernel(const int32_t* __restrict__ nbr_cols,
                                                          const int32_t* __restrict__ cols_row,
                                                          int64_t n_cols, int64_t n_rows,
                                                          int32_t* __restrict__ nbr_rows) {
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t >= n_cols) return;
  const int32_t r = cols_row[t];
  if (r < 0 || r >= n_rows) return;
  nbr_rows[(int64_t)blockIdx.y * n_rows + r] = nbr_cols[(int64_t)blockIdx.y * n_cols + t];
}

// Emits pairs_in/pairs_out for every slot from the neighbour map.  Rows keep
// ascending order inside a slot: blocks own consecutive row ranges (block
// offsets from the per-slot scan), waves own consecutive sub-ranges (offsets
// from per-wave counts) and lanes are ranked by ballot.
__global__ void __launch_bounds__(kRows) subm_fill_kernel(const int32_t* __restrict__ nbr, int64_t n,
                                                          int K,
                                                          const int32_t* __restrict__ blk_off,
                                                          int nblk, int64_t cap,
                                                          int32_t* __restrict__ pairs_in,
                                                          int32_t* __restrict__ pairs_out) {
  __shared__ int32_t s_wcnt[kRows / kWave][64];
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int64_t r = blockIdx.x * (int64_t)kRows + t;
  const bool valid = r < n;
  for (int kb = 0; kb < K; kb += 64) {
    const int kend = (K - kb) < 64 ? (K - kb) : 64;
    for (int kk = 0; kk < kend; ++kk) {
      const int32_t j = valid ? nbr[(int64_t)(kb + kk) * n + r] : -1;
      const uint64_t hits = __ballot(j >= 0);
      if (__lane_id() == 0) s_wcnt[w][kk] = __popcll(hits);
    }
    __syncthreads();
    for (int kk = 0; kk < kend; ++kk) {
      const int k = kb + kk;
      const int32_t j = valid ? nbr[(int64_t)k * n + r] : -1;
      const uint64_t hits = __ballot(j >= 0);
      int base = blk_off[(int64_t)k * nblk + blockIdx.x];
      for (int ww = 0; ww < w; ++ww) base += s_wcnt[ww][kk];
      const int64_t slot_pos = base + rank_in_wave(hits);
      if (j >= 0 && slot_pos < cap) {  // slot_pos < cap holds by construction
        pairs_in[(int64_t)k * cap + slot_pos] = j;
        pairs_out[(int64_t)k * cap + slot_pos] = static_cast<int32_t>(r);
      }
    }
    __syncthreads();
  }
}

// Block k: counts[k] = the sum of slot k's per-block counts (cnt [K][nblk];
// none: counts[k] as it is), copied into host memory (host[k]; block 0 also
// copies counts[K] and counts[K + 1]), then done[k] = 1 once they are
// visible there.
__global__ void __launch_bounds__(256) subm_counts_kernel(const int32_t* __restrict__ cnt,
                                                          int nblk, int K,
                                                          int32_t* __restrict__ counts,
                                                          int32_t* host, int32_t* done) {
  __shared__ int32_t s_part[256 / kWave];
  const int k = blockIdx.x;
  int32_t tot = 0;
  if (cnt) {
    int32_t acc = 0;
    for (int i = threadIdx.x; i < nblk; i += blockDim.x) acc += cnt[(int64_t)k * nblk + i];
    for (int off = kWave / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
    if (__lane_id() == 0) s_part[threadIdx.x / kWave] = acc;
    __syncthreads();
    for (int w = 0; w < 256 / kWave; ++w) tot += s_part[w];
  }
  if (threadIdx.x != 0) return;
  if (cnt)
    counts[k] = tot;
  else
    tot = counts[k];
  __hip_atomic_store(&host[k], tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (k == 0) {
    __hip_atomic_store(&host[K], counts[K], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(&host[K + 1], counts[K + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  // the values reach host memory before the word that announces them
  __hip_atomic_store(&done[k], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

}  // namespace

static int64_t subm_capacity(int64_t n) {
  int64_t cap = 1024;
  while (cap < 2 * n) cap <<= 1;
  return cap;
}

// The bitmap is used when its words number at most 64 per voxel plus 2^20.
// Its zeroing and scan cost about 7 ns per 1000 words and its per-voxel
// kernels about 0.2 ns per voxel, against about 0.9 ns per voxel for the hash
// once the table outgrows L2 (240 000 voxels in 4 x 41 x 1600 x 1408 cells:
// 127 us against 222 us), so the bitmap stays ahead up to about 100 words per
// voxel.  Its entries then take at most 512 bytes per voxel.
static bool subm_use_bitmap(int64_t n, int64_t cells) {
  return ceil_div(cells, 32) <= 64 * n + (int64_t(1) << 20);
}

// Cell keys fit the packed 32-bit hash words and the bitmap's column words
// below this many cells.
constexpr int64_t kNarrowCells = 0xffffffffll;

struct SubmWork {
  unsigned long long* table;  // packed (key << 32 | row) words, or the 64-bit keys
  int32_t* vals;              // rows of the 64-bit-key table
  uint2* wr;       // bitmap entries (word, rank)
  uint8_t* bytes;  // byte-per-cell occupancy (byte-marked bitmap builds)
  uint32_t* scan;  // bitmap scan scratch
  uint2* col;      // map columns: (row + 1, cell), 4 entries of padding
  uint8_t* touched;  // atomic-marked bitmaps: a byte per scan tile holding a row's cell
  int32_t *n_unique, *n_extra, *blk_cnt, *blk_off;
};

// How the build finds neighbours: hash table, or occupancy bitmap whose bits
// are set by atomics or packed from a byte per cell.
enum SubmMode { kSubmHash = 0, kSubmBitmap = 1, kSubmBytes = 2 };

static int64_t bitmap_words(int64_t cells) { return ceil_div(cells, 32); }

// marks_outside: the byte marks are the caller's (kept between builds), not
// part of the workspace.
static SubmWork subm_carve(void* ws, int64_t n, int K, int64_t cells, int mode, int64_t* used,
                           bool marks_outside = false) {
  Carver c(ws);
  const int64_t m = n > 0 ? n : 1;
  const int64_t nblk = ceil_div(m, kRows);
  SubmWork w{};
  if (mode != kSubmHash) {
    const int64_t nw = bitmap_words(cells);
    w.wr = c.take<uint2>(bitmap_entries(nw));
    if (mode == kSubmBytes) {
      if (!marks_outside) w.bytes = c.take<uint8_t>(marks_bytes(nw));
    } else {
      w.touched = c.take<uint8_t>(align_up(bitmap_tiles(nw), 16));
    }
    w.scan = c.take<uint32_t>(bitmap_scan_scratch_words(nw));
    w.col = c.take<uint2>(m + 4);
    w.n_unique = c.take<int32_t>(1);
    w.n_extra = c.take<int32_t>(1);
    w.blk_cnt = c.take<int32_t>(nblk * K);
  } else {
    w.table = c.take<unsigned long long>(subm_capacity(m));
    if (cells >= kNarrowCells) w.vals = c.take<int32_t>(subm_capacity(m));
    w.blk_cnt = c.take<int32_t>(nblk * K);
    w.blk_off = c.take<int32_t>(nblk * K);
  }
  if (used) *used = c.used;
  return w;
}

// Grids of at most this many cells mark through bytes however few rows they
// hold: packing a byte map of up to 4 MB costs less than the three launches
// of the atomic path's touched tiles (flag clear, touch, tile zeroing).
constexpr int64_t kSmallByteGrid = int64_t(1) << 22;

// Bitmap or hash: the bitmap while the grid is dense enough (and its cell ids
// fit 32 bits), marked through a byte map while that is at most 64 bytes per
// row or the grid is small; with a workspace limit, the first of these that
// fits.
static int subm_pick_mode(int64_t n, int K, int64_t cells, int64_t ws_limit) {
  if (!(cells < kNarrowCells && subm_use_bitmap(n, cells))) return kSubmHash;
  int64_t used = 0;
  if (cells <= 64 * n || cells <= kSmallByteGrid) {
    subm_carve(nullptr, n, K, cells, kSubmBytes, &used);
    if (used <= ws_limit) return kSubmBytes;
  }
  subm_carve(nullptr, n, K, cells, kSubmBitmap, &used);
  return used <= ws_limit ? kSubmBitmap : kSubmHash;
}

__global__ void iota_kernel(int32_t* p, int64_t n) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i < n) p[i] = static_cast<int32_t>(i);
}

}  // namespace tsc

using namespace tsc;

static int64_t subm_cells(int64_t n, int32_t k_vol, int32_t batch_size, const int32_t* spatial) {
  if (n < 0 || k_vol <= 0 || batch_size <= 0 || !spatial) return -1;
  if (spatial[0] <= 0 || spatial[1] <= 0 || spatial[2] <= 0 ||
      (int64_t)batch_size * spatial[0] * spatial[1] > (int64_t(1) << 62) / spatial[2])
    return -1;
  return (int64_t)batch_size * spatial[0] * spatial[1] * spatial[2];
}

extern "C" int64_t tsc_subm_workspace_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                            const int32_t spatial[3], int32_t marks_outside) {
  const int64_t cells = subm_cells(n, k_vol, batch_size, spatial);
  if (cells < 0) return -1;
  int64_t used = 0;
  subm_carve(nullptr, n, k_vol, cells, subm_pick_mode(n, k_vol, cells, INT64_MAX), &used,
             marks_outside != 0);
  return used;
}

extern "C" int64_t tsc_subm_marks_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                        const int32_t spatial[3]) {
  const int64_t cells = subm_cells(n, k_vol, batch_size, spatial);
  if (cells < 0) return -1;
  return subm_pick_mode(n, k_vol, cells, INT64_MAX) == kSubmBytes ? marks_bytes(bitmap_words(cells))
                                                                   : 0;
}

// The build on a given workspace.  ws_limit > 0: the workspace is that many
// bytes of fixed scratch (the bitmap is taken only when it fits, else the
// hash); 0: the caller's workspace, sized by tsc_subm_workspace_bytes.
int tsc::subm_pairs_ws(const int32_t* coords, int64_t n, int32_t batch_size,
                      const int32_t spatial[3], const int32_t ksize[3],
                      const int32_t dilation[3], void* ws, int64_t ws_bytes, int64_t ws_limit,
                      int32_t* cols_row, int32_t* nbr, int32_t* counts, tsc_stream_t stream,
                      const HostStatus* hs, int32_t* slot_blocks, int32_t* raster,
                      int32_t mask_row, uint8_t* marks, int64_t marks_size, int32_t gen) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "subm: n=%lld out of range", (long long)n);
  TSC_REQUIRE(batch_size > 0, "subm: batch_size must be positive");
  TSC_REQUIRE(spatial && ksize && dilation, "subm: null shape argument");
  const Box shape = box(spatial), ks = box(ksize), dil = box(dilation);
  TSC_REQUIRE(shape.z > 0 && shape.y > 0 && shape.x > 0, "subm: spatial shape must be positive");
  TSC_REQUIRE(ks.z > 0 && ks.y > 0 && ks.x > 0 && dil.z > 0 && dil.y > 0 && dil.x > 0,
              "subm: kernel size and dilation must be positive");
  TSC_REQUIRE((int64_t)batch_size * shape.z * shape.y <= (int64_t(1) << 62) / shape.x,
              "subm: batch*D*H*W exceeds 2^62 cells");
  const int64_t cells = (int64_t)batch_size * shape.z * shape.y * shape.x;
  const int K = ks.z * ks.y * ks.x;
  TSC_REQUIRE(K <= 4096, "subm: kernel volume %d too large", K);
  const int mode = subm_pick_mode(n, K, cells, ws_limit > 0 ? ws_limit : INT64_MAX);
  // the caller's byte marks, used when this build marks through bytes
  const bool outside = marks != nullptr && mode == kSubmBytes;
  if (outside) {
    TSC_REQUIRE(marks_size >= marks_bytes(bitmap_words(cells)),
                "subm: marks of %lld bytes, this grid needs %lld", (long long)marks_size,
                (long long)marks_bytes(bitmap_words(cells)));
    TSC_REQUIRE(gen >= 1 && gen <= 255, "subm: mark value %d outside 1..255", gen);
  }
  int64_t need = 0;
  subm_carve(nullptr, n, K, cells, mode, &need, outside);
  if (ws_limit > 0)
    TSC_REQUIRE(need <= ws_limit,
                "subm: this build needs %lld bytes of scratch, more than the %lld the "
                "no-allocation entry point holds (n=%lld, %lld cells); use tsc_subm_pairs with "
                "a workspace", (long long)need, (long long)ws_limit, (long long)n,
                (long long)cells);
  else
    TSC_REQUIRE(ws_bytes >= need, "subm: workspace too small");
  TSC_REQUIRE(counts != nullptr, "subm: counts is null");

  int rc = 0;
  if (raster) *raster = 0;
  if (n == 0) return fill_u32(reinterpret_cast<uint32_t*>(counts), K + 2, 0u, s);
  TSC_REQUIRE(coords && cols_row && nbr && ws, "subm: null pointer");
  // the checking kernel's flag and the next kernel's start, in host memory
  int32_t* host_flag = hs ? hs->dev + kHostFlag : nullptr;
  int32_t* started = hs ? hs->dev + kHostStarted : nullptr;

  const int nblk = static_cast<int>(ceil_div(n, kRows));
  SubmWork w = subm_carve(ws, n, K, cells, mode, nullptr, outside);
  if (outside) w.bytes = marks;
  const uint32_t mark_gen = outside ? static_cast<uint32_t>(gen) : 1u;
  int32_t* const blk_cnt = slot_blocks ? slot_blocks : w.blk_cnt;
  TSC_REQUIRE(!mask_row || K <= 32, "subm: a slot-mask row needs k_vol <= 32 (got %d)", K);
  // the column slot masks, as row K of the map (the bitmap path's probes
  // write them; the hash path's columns are the rows, which take no order)
  uint32_t* const col_masks = mask_row ? reinterpret_cast<uint32_t*>(nbr + (int64_t)K * n) : nullptr;
  const int4* c4 = reinterpret_cast<const int4*>(coords);
  if (w.wr) {
    const int64_t nw = bitmap_words(cells);
    SubmGeom g{batch_size, shape, ks, dil, 0u};
    uint32_t* const mwords = w.bytes ? mark_words(w.bytes, nw) : nullptr;
    // zero the marks: the byte marks (the scan then writes every bitmap
    // entry), or for atomic marks the touched-tile flags, whose tiles alone
    // are then zeroed.  Marks kept by the caller are not zeroed: this build's
    // generation value tells its marks apart, and the rank pass writes the
    // counters the init would clear.
    if (!outside) {
      const int64_t units = w.bytes ? marks_bytes(nw) / 16 : align_up(bitmap_tiles(nw), 16) / 16;
      uint4* zero = reinterpret_cast<uint4*>(w.bytes ? static_cast<void*>(w.bytes)
                                                     : static_cast<void*>(w.touched));
      const int64_t init_blocks = std::min<int64_t>(ceil_div(units, 256), 4096);
      subm_init_kernel<<<static_cast<unsigned>(init_blocks > 0 ? init_blocks : 1), 256, 0, s>>>(
          zero, units, counts, K, w.n_extra);
      TSC_LAUNCH_CHECK("subm_init");
    }
    if (w.bytes) {
      subm_mark_kernel<true><<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.wr, w.bytes, mwords,
                                                              mark_gen, counts + K, host_flag,
                                                              w.col, w.n_extra);
    } else {
      subm_touch_kernel<<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.touched);
      TSC_LAUNCH_CHECK("subm_touch");
      subm_zero_touched_kernel<<<static_cast<unsigned>(bitmap_tiles(nw)), 256, 0, s>>>(
          reinterpret_cast<uint4*>(w.wr), bitmap_entries(nw) / 2, w.touched);
      TSC_LAUNCH_CHECK("subm_zero_touched");
      subm_mark_kernel<false><<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.wr, nullptr, nullptr,
                                                               0u, counts + K, host_flag, w.col,
                                                               w.n_extra);
    }
    TSC_LAUNCH_CHECK("subm_mark");
    if (raster) *raster = 1;
    if ((rc = bitmap_scan(w.wr, nw, w.scan, w.n_unique, s, w.bytes, nullptr, started, w.touched,
                          mark_gen)))
      return rc;
    subm_rank_kernel<<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.wr, w.n_unique, w.col,
                                                      w.n_extra, mwords, mark_gen, counts, K);
    TSC_LAUNCH_CHECK("subm_rank");
    // slots from 64 on are added into the per-block table, which starts at 0
    if (K > 64 &&
        (rc = fill_u32(reinterpret_cast<uint32_t*>(blk_cnt), (int64_t)nblk * K, 0u, s)))
      return rc;
    if (ks.x == 3 && ks.y == 3 && ks.z == 3 && dil.x == 1 && n < kProbe333Rows) {
      if (w.touched)
        subm_probe_333_kernel<false, true><<<ceil_div(n, kRows), kRows, 0, s>>>(
            n, g, w.wr, nw, w.col, nullptr, w.n_unique, w.n_extra, cols_row, nbr, blk_cnt, nblk,
            counts, col_masks, w.touched);
      else
        subm_probe_333_kernel<false, false><<<ceil_div(n, kRows), kRows, 0, s>>>(
            n, g, w.wr, nw, w.col, nullptr, w.n_unique, w.n_extra, cols_row, nbr, blk_cnt, nblk,
            counts, col_masks, nullptr);
      TSC_LAUNCH_CHECK("subm_probe_333");
    } else if (ks.x == 3 && 2 * dil.x < 32 && ks.y == 3 && ks.z == 3) {
      subm_probe_rows_kernel<3, 3, 3, false><<<ceil_div(n, 256), 256, 0, s>>>(
          n, K, g, w.wr, nw, w.col, nullptr, w.n_unique, w.n_extra, cols_row, nbr, blk_cnt,
          nblk, counts, col_masks, w.touched);
      TSC_LAUNCH_CHECK("subm_probe_rows");
    } else if (ks.x == 3 && 2 * dil.x < 32) {
      subm_probe_rows_kernel<3, 0, 0, false><<<ceil_div(n, 256), 256, 0, s>>>(
          n, K, g, w.wr, nw, w.col, nullptr, w.n_unique, w.n_extra, cols_row, nbr, blk_cnt,
          nblk, counts, col_masks, w.touched);
      TSC_LAUNCH_CHECK("subm_probe_rows");
    } else {
      subm_probe_cols_kernel<<<ceil_div(n, 256), 256, 0, s>>>(n, K, g, w.wr, w.col, w.n_unique,
                                                              w.n_extra, cols_row, nbr, blk_cnt,
                                                              nblk, counts, col_masks, w.touched);
      TSC_LAUNCH_CHECK("subm_probe_cols");
    }
    if (!slot_blocks && (rc = sum_slot_blocks(blk_cnt, counts, K, nblk, s))) return rc;
  } else {
    if ((rc = fill_u32(reinterpret_cast<uint32_t*>(counts), K + 2, 0u, s))) return rc;
    const int64_t cap = subm_capacity(n);
    SubmGeom g{batch_size, shape, ks, dil, static_cast<uint32_t>(cap - 1)};
    if (K > 64 &&
        (rc = fill_u32(reinterpret_cast<uint32_t*>(blk_cnt), (int64_t)nblk * K, 0u, s)))
      return rc;
    if ((rc = fill_u64(w.table, cap, kEmpty, s))) return rc;
    iota_kernel<<<ceil_div(n, 256), 256, 0, s>>>(cols_row, n);
    TSC_LAUNCH_CHECK("subm_iota");
    if (w.vals) {
      if ((rc = fill_u32(reinterpret_cast<uint32_t*>(w.vals), cap, 0xffffffffu, s))) return rc;
      subm_insert_wide_kernel<<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.table, w.vals,
                                                               counts + K, host_flag);
      TSC_LAUNCH_CHECK("subm_insert_wide");
      subm_probe_wide_kernel<<<nblk, kRows, 0, s>>>(c4, n, K, g, w.table, w.vals, nbr, blk_cnt,
                                                    nblk, started);
      TSC_LAUNCH_CHECK("subm_probe_wide");
    } else {
      subm_insert_kernel<<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.table, counts + K,
                                                          host_flag);
      TSC_LAUNCH_CHECK("subm_insert");
      subm_probe_kernel<<<nblk, kRows, 0, s>>>(c4, n, K, g, w.table, nbr, blk_cnt, nblk, started);
      TSC_LAUNCH_CHECK("subm_probe");
    }
    if (!slot_blocks && (rc = sum_slot_blocks(blk_cnt, counts, K, nblk, s))) return rc;
  }
  return 0;
}

extern "C" int tsc_subm_pairs(const int32_t* coords, int64_t n, int32_t batch_size,
                              const int32_t spatial[3], const int32_t ksize[3],
                              const int32_t dilation[3], void* ws, int64_t ws_bytes,
                              int32_t* cols_row, int32_t* nbr, int32_t* counts,
                              tsc_stream_t stream) {
  return subm_pairs_ws(coords, n, batch_size, spatial, ksize, dilation, ws, ws_bytes, 0, cols_row,
                       nbr, counts, stream);
}

extern "C" int64_t tsc_subm_slot_blocks_len(int64_t n, int32_t k_vol) {
  if (n < 0 || k_vol <= 0) return -1;
  return ceil_div(n > 0 ? n : 1, kRows) * k_vol;
}

extern "C" int tsc_subm_pairs_checked(const int32_t* coords, int64_t n, int32_t batch_size,
                                      const int32_t spatial[3], const int32_t ksize[3],
                                      const int32_t dilation[3], void* ws, int64_t ws_bytes,
                                      void* marks, int64_t marks_size, int32_t gen,
                                      int32_t* cols_row, int32_t* nbr, int32_t* counts,
                                      int32_t* slot_blocks, int32_t mask_row, int32_t result[2],
                                      tsc_stream_t stream) {
  TSC_REQUIRE(result != nullptr, "subm: result is null");
  TSC_REQUIRE(slot_blocks != nullptr, "subm: slot_blocks is null");
  result[0] = result[1] = 0;
  HostStatus hs{};
  if (int rc = host_status(&hs)) return rc;
  hs.host[kHostFlag] = 0;
  hs.host[kHostStarted] = 0;
  int32_t raster = 0;
  if (int rc = subm_pairs_ws(coords, n, batch_size, spatial, ksize, dilation, ws, ws_bytes, 0,
                             cols_row, nbr, counts, stream, &hs, slot_blocks, &raster, mask_row,
                             static_cast<uint8_t*>(marks), marks_size, gen))
    return rc;
  result[1] = raster;
  if (n == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  int seen = 0;
  if (int rc = wait_host_word(hs.host + kHostStarted, s, &seen)) return rc;
  if (!seen || __atomic_load_n(hs.host + kHostFlag, __ATOMIC_ACQUIRE) != 0) {
    // a coordinate failed (or the stream drained before the word was seen):
    // the exact flags, from the device's status word
    hipError_t e = hipMemcpyAsync(&result[0], counts + ksize[0] * ksize[1] * ksize[2],
                                  sizeof(int32_t), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess)
      return set_error(-static_cast<int>(e), "subm: reading the status flags: %s",
                       hipGetErrorString(e));
  }
  return 0;
}

extern "C" int tsc_subm_counts(const int32_t* slot_blocks, int64_t n, int32_t k_vol,
                               int32_t* counts, int32_t* counts_host, tsc_stream_t stream) {
  TSC_REQUIRE(n >= 0 && n < (int64_t(1) << 31) && k_vol > 0 && k_vol <= 4096,
              "subm_counts: invalid sizes");
  TSC_REQUIRE(counts, "subm_counts: null pointer");
  TSC_REQUIRE(n == 0 || slot_blocks, "subm_counts: null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int32_t* cnt = n > 0 ? slot_blocks : nullptr;
  const int nblk = static_cast<int>(ceil_div(n > 0 ? n : 1, kRows));
  if (!counts_host) {
    if (!cnt) return 0;
    return sum_slot_blocks(cnt, counts, k_vol, nblk, s);
  }
  // the sums go to the device counts and, with counts[K] and counts[K+1],
  // straight into pinned host memory; a word per slot says its count is there
  HostStatus hs{};
  if (int rc = host_status(&hs)) return rc;
  for (int k = 0; k < k_vol; ++k) hs.host[kHostDone + k] = 0;
  subm_counts_kernel<<<k_vol, 256, 0, s>>>(cnt, nblk, k_vol, counts, hs.dev + kHostCounts,
                                           hs.dev + kHostDone);
  TSC_LAUNCH_CHECK("subm_counts");
  int seen = 1;
  for (int k = 0; k < k_vol && seen; ++k)
    if (int rc = wait_host_word(hs.host + kHostDone + k, s, &seen)) return rc;
  if (!seen) {
    // the stream drained without the words showing: read the device copy
    hipError_t e = hipMemcpyAsync(counts_host, counts, (k_vol + 2) * sizeof(int32_t),
                                  hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    return e == hipSuccess ? 0 : set_error(-static_cast<int>(e), "subm_counts: %s",
                                           hipGetErrorString(e));
  }
  for (int i = 0; i < k_vol + 2; ++i)
    counts_host[i] = __atomic_load_n(hs.host + kHostCounts + i, __ATOMIC_ACQUIRE);
  return 0;
}

extern "C" int tsc_subm_pairs_from_bitmap(const int32_t* coords, int64_t n, int32_t batch_size,
                                          const int32_t spatial[3], const int32_t ksize[3],
                                          const int32_t dilation[3], const void* bitmap,
                                          int64_t bitmap_entries_n, int32_t* cols_row, int32_t* nbr,
                                          int32_t* counts, int32_t mask_row, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "subm: n=%lld out of range", (long long)n);
  TSC_REQUIRE(batch_size > 0, "subm: batch_size must be positive");
  TSC_REQUIRE(spatial && ksize && dilation, "subm: null shape argument");
  const Box shape = box(spatial), ks = box(ksize), dil = box(dilation);
  TSC_REQUIRE(shape.z > 0 && shape.y > 0 && shape.x > 0, "subm: spatial shape must be positive");
  TSC_REQUIRE(ks.z > 0 && ks.y > 0 && dil.z > 0 && dil.y > 0 && dil.x > 0,
              "subm: kernel size and dilation must be positive");
  TSC_REQUIRE(ks.x == 3 && 2 * dil.x < 32,
              "subm: a build on a bitmap needs a kernel 3 cells wide in x with dilation < 16");
  const int64_t cells = (int64_t)batch_size * shape.z * shape.y * shape.x;
  TSC_REQUIRE(cells < kNarrowCells,
              "subm: a build on a bitmap needs fewer than 2^32 - 1 cells (batch*D*H*W = %lld)",
              (long long)cells);
  const int K = ks.z * ks.y * ks.x;
  TSC_REQUIRE(K <= 4096, "subm: kernel volume %d too large", K);
  const int64_t nw = bitmap_words(cells);
  TSC_REQUIRE(bitmap && bitmap_entries_n >= nw,
              "subm: bitmap of %lld entries, the grid needs %lld", (long long)bitmap_entries_n,
              (long long)nw);
  TSC_REQUIRE(counts != nullptr, "subm: counts is null");
  TSC_REQUIRE(!mask_row || K <= 32, "subm: a slot-mask row needs k_vol <= 32 (got %d)", K);
  uint32_t* const col_masks = mask_row ? reinterpret_cast<uint32_t*>(nbr + (int64_t)K * n) : nullptr;
  // counts[0..K] = 0 (counts[K]: no status flags), counts[K+1] = 1 (rows in
  // (b,z,y,x) order)
  subm_init_kernel<<<1, 256, 0, s>>>(nullptr, 0, counts, K, counts + K);
  TSC_LAUNCH_CHECK("subm_init");
  if (n == 0) return 0;
  TSC_REQUIRE(coords && cols_row && nbr, "subm: null pointer");
  SubmGeom g{batch_size, shape, ks, dil, 0u};
  const uint2* wr = static_cast<const uint2*>(bitmap);
  const int4* c4 = reinterpret_cast<const int4*>(coords);
  if (ks.y == 3 && ks.z == 3 && dil.x == 1 && n < kProbe333Rows)
    subm_probe_333_kernel<true, false><<<ceil_div(n, kRows), kRows, 0, s>>>(
        n, g, wr, nw, nullptr, c4, nullptr, nullptr, cols_row, nbr, nullptr, 0, counts, col_masks,
        nullptr);
  else if (ks.y == 3 && ks.z == 3)
    subm_probe_rows_kernel<3, 3, 3, true><<<ceil_div(n, 256), 256, 0, s>>>(
        n, K, g, wr, nw, nullptr, c4, nullptr, nullptr, cols_row, nbr, nullptr, 0, counts,
        col_masks, nullptr);
  else
    subm_probe_rows_kernel<3, 0, 0, true><<<ceil_div(n, 256), 256, 0, s>>>(
        n, K, g, wr, nw, nullptr, c4, nullptr, nullptr, cols_row, nbr, nullptr, 0, counts,
        col_masks, nullptr);
  TSC_LAUNCH_CHECK("subm_probe_rows");
  return 0;
}

extern "C" int tsc_map_to_rows(const int32_t* nbr_cols, const int32_t* cols_row, int64_t n_cols,
                               int64_t n_rows, int32_t k_vol, int32_t* nbr_rows,
                               tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(n_cols >= 0 && n_rows >= 0 && k_vol > 0 && k_vol <= 65535,
              "map_to_rows: invalid sizes");
  if (n_cols == 0 || n_rows == 0) return 0;
  TSC_REQUIRE(nbr_cols && cols_row && nbr_rows, "map_to_rows: null pointer");
  dim3 grid(static_cast<unsigned>(ceil_div(n_cols, 256)), static_cast<unsigned>(k_vol));
  map_to_rows_kernel<<<grid, 256, 0, s>>>(nbr_cols, cols_row, n_cols, n_rows, nbr_rows);
  TSC_LAUNCH_CHECK("map_to_rows");
  return 0;
}

extern "C" int64_t tsc_pairs_from_map_workspace_bytes(int64_t n, int32_t k_vol) {
  if (n < 0 || k_vol <= 0) return -1;
  Carver c(nullptr);
  const int64_t nblk = ceil_div(n > 0 ? n : 1, kRows);
  c.take<int32_t>(nblk * k_vol);  // block counts
  c.take<int32_t>(nblk * k_vol);  // block offsets
  c.take<int32_t>(k_vol);         // slot totals
  return c.used;
}

extern "C" int tsc_pairs_from_map(const int32_t* nbr, int64_t n, int32_t k_vol, int64_t cap,
                                  void* ws, int64_t ws_bytes, int32_t* pairs_in,
                                  int32_t* pairs_out, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(n >= 0 && n < (int64_t(1) << 31) && k_vol > 0 && k_vol <= 4096 && cap >= 0,
              "pairs_from_map: invalid sizes");
  TSC_REQUIRE(ws_bytes >= tsc_pairs_from_map_workspace_bytes(n, k_vol),
              "pairs_from_map: workspace too small");
  if (n == 0) return 0;
  TSC_REQUIRE(nbr && ws && pairs_in && pairs_out, "pairs_from_map: null pointer");
  const int nblk = static_cast<int>(ceil_div(n, kRows));
  Carver c(ws);
  auto* blk_cnt = c.take<int32_t>((int64_t)nblk * k_vol);
  auto* blk_off = c.take<int32_t>((int64_t)nblk * k_vol);
  auto* totals = c.take<int32_t>(k_vol);
  int rc;
  if (k_vol > 64 &&
      (rc = fill_u32(reinterpret_cast<uint32_t*>(blk_cnt), (int64_t)nblk * k_vol, 0u, s)))
    return rc;
  map_count_kernel<<<nblk, kRows, 0, s>>>(nbr, n, k_vol, blk_cnt, nblk);
  TSC_LAUNCH_CHECK("pairs_count");
  if ((rc = scan_slot_blocks(blk_cnt, blk_off, totals, k_vol, nblk, s))) return rc;
  subm_fill_kernel<<<nblk, kRows, 0, s>>>(nbr, n, k_vol, blk_off, nblk, cap, pairs_in, pairs_out);
  TSC_LAUNCH_CHECK("pairs_fill");
  return 0;
}
