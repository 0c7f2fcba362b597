// Submanifold indice pairs on the GPU.
//
// Reference algorithm: trispconv/pytorch/indices.py:67-140.  For slot k (kernel
// offsets in (kz,ky,kx) lexicographic order, measured from the kernel centre)
// and every output row r in ascending order, the pair (in = j, out = r) exists
// when coord(r) + offset_k lies inside the grid and is the coordinate of row j.
//
// MI355X design: the reference's dense grid-sized lookup table (:54-64) becomes
// one of two compact structures, chosen by how dense the active set is:
//   * occupancy bitmap (grids of up to about 32 cells per voxel): one bit per
//     cell, an exclusive popcount scan of its words (each occupied cell's rank
//     in (b,z,y,x) order) and rank -> row.  The neighbour lookups then run in
//     rank order — a wave handles 64 neighbouring occupied cells, so its
//     bitmap and rank reads share cache lines — and write the map rows they
//     own; a row-order pass copies the entries of duplicate rows;
//   * open-addressing hash of 2N..4N 64-bit slots otherwise, probed in row
//     order.
// Both write the slot-major [K][N] neighbour map the convolution consumes and
// per-(slot, block) hit counts; a per-slot scan of those counts gives each
// block its write offset, and a fill kernel emits every slot's pair list in
// ascending output-row order with wave ballots, so the lists come out in
// exactly the reference's order.  Repeated coordinates resolve to the later
// row, as the reference's table scatter leaves them.
#include "common.hpp"

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

__global__ void __launch_bounds__(256) subm_insert_kernel(const int4* __restrict__ coords,
                                                          int64_t n, SubmGeom g,
                                                          unsigned long long* table,
                                                          int32_t* status) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int4 c = coords[r];  // (b, z, y, x)
  if (!in_grid(g, c.x, c.y, c.z, c.w)) {
    atomicOr(status, (c.x < 0 || c.x >= g.B) ? TSC_FLAG_BATCH_OUT_OF_RANGE
                                              : TSC_FLAG_COORD_OUT_OF_GRID);
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
                                                           int nblk) {
  __shared__ int32_t s_cnt[kRows / kWave][64];  // per wave, per slot (slots < 64)
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

// ------------------------------------------------------------ bitmap path --
// Sets each row's cell bit; rows outside the grid only raise a status flag.
__global__ void __launch_bounds__(256) subm_mark_kernel(const int4* __restrict__ coords, int64_t n,
                                                        SubmGeom g, uint32_t* words,
                                                        int32_t* status) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int4 c = coords[r];
  if (!in_grid(g, c.x, c.y, c.z, c.w)) {
    atomicOr(status, (c.x < 0 || c.x >= g.B) ? TSC_FLAG_BATCH_OUT_OF_RANGE
                                              : TSC_FLAG_COORD_OUT_OF_GRID);
    return;
  }
  const uint32_t cell = cell_key(g, c.x, c.y, c.z, c.w);
  atomicOr(&words[cell >> 5], 1u << (cell & 31));
}

// Rank of an occupied cell: occupied cells before it in (b,z,y,x) order.
__device__ __forceinline__ uint32_t cell_rank(uint32_t word, uint32_t word_rank, uint32_t cell) {
  return word_rank + __popc(word & ((1u << (cell & 31)) - 1u));
}

// rank_row[rank of the row's cell] = the largest row with that cell.
__global__ void __launch_bounds__(256) subm_rank_kernel(const int4* __restrict__ coords, int64_t n,
                                                        SubmGeom g,
                                                        const uint32_t* __restrict__ words,
                                                        const uint32_t* __restrict__ word_rank,
                                                        int32_t* rank_row) {
  const int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (r >= n) return;
  const int4 c = coords[r];
  if (!in_grid(g, c.x, c.y, c.z, c.w)) return;
  const uint32_t cell = cell_key(g, c.x, c.y, c.z, c.w);
  atomicMax(&rank_row[cell_rank(words[cell >> 5], word_rank[cell >> 5], cell)],
            static_cast<int32_t>(r));
}

// One thread per occupied cell, in rank order: the thread's row (the cell's
// last row) gets its K neighbours.  Eight slots' bitmap and prefix reads are
// in flight together, then their rank -> row reads.
constexpr int kLook = 8;

__global__ void __launch_bounds__(256) subm_probe_rank_kernel(
    const int4* __restrict__ coords, int64_t n, int K, SubmGeom g,
    const uint32_t* __restrict__ words, const uint32_t* __restrict__ word_rank,
    const int32_t* __restrict__ rank_row, const int32_t* __restrict__ n_unique,
    int32_t* __restrict__ nbr) {
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (t >= *n_unique) return;
  const int32_t row = rank_row[t];
  const int4 c = coords[row];
  for (int k0 = 0; k0 < K; k0 += kLook) {
    uint32_t cell[kLook], wv[kLook], wr[kLook];
    bool look[kLook];
#pragma unroll
    for (int i = 0; i < kLook; ++i) {
      const int k = k0 + i;
      int kz, ky, kx;
      slot_to_zyx(k < K ? k : 0, g.ks, kz, ky, kx);
      const int z = c.y + (kz - g.ks.z / 2) * g.dil.z;
      const int y = c.z + (ky - g.ks.y / 2) * g.dil.y;
      const int x = c.w + (kx - g.ks.x / 2) * g.dil.x;
      look[i] = k < K && in_grid(g, c.x, z, y, x);
      cell[i] = look[i] ? cell_key(g, c.x, z, y, x) : 0u;
      wv[i] = words[cell[i] >> 5];  // word 0 exists: unconditional reads
      wr[i] = word_rank[cell[i] >> 5];
    }
    int32_t jr[kLook];
#pragma unroll
    for (int i = 0; i < kLook; ++i) {
      const bool hit = look[i] && ((wv[i] >> (cell[i] & 31)) & 1u);
      jr[i] = rank_row[hit ? cell_rank(wv[i], wr[i], cell[i]) : 0u];  // rank 0 exists
      if (!hit) jr[i] = -1;
    }
#pragma unroll
    for (int i = 0; i < kLook; ++i)
      if (k0 + i < K) nbr[(int64_t)(k0 + i) * n + row] = jr[i];
  }
}

// Row order: rows that share a cell with a later row copy that row's map
// entries, rows outside the grid get -1 (the call reports them), and every
// block counts its hits per slot for the compaction offsets.
__global__ void __launch_bounds__(kRows) subm_finish_kernel(
    const int4* __restrict__ coords, int64_t n, int K, SubmGeom g,
    const uint32_t* __restrict__ words, const uint32_t* __restrict__ word_rank,
    const int32_t* __restrict__ rank_row, int32_t* __restrict__ nbr, int32_t* __restrict__ blk_cnt,
    int nblk) {
  __shared__ int32_t s_cnt[kRows / kWave][64];
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int64_t r = blockIdx.x * (int64_t)kRows + t;
  const bool valid = r < n;
  const int4 c = valid ? coords[r] : make_int4(-1, 0, 0, 0);
  const bool ok = valid && in_grid(g, c.x, c.y, c.z, c.w);
  int64_t src = r;
  if (ok) {
    const uint32_t cell = cell_key(g, c.x, c.y, c.z, c.w);
    src = rank_row[cell_rank(words[cell >> 5], word_rank[cell >> 5], cell)];
  }
  const bool copy = ok && src != r;
  for (int k = 0; k < K; ++k) {
    int32_t j = -1;
    if (ok) j = nbr[(int64_t)k * n + src];
    if (valid && (copy || !ok)) nbr[(int64_t)k * n + r] = j;
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

}  // namespace

static int64_t subm_capacity(int64_t n) {
  int64_t cap = 1024;
  while (cap < 2 * n) cap <<= 1;
  return cap;
}

// The bitmap is used when its words number at most 8 per voxel plus 2^20
// (4 MiB): its zeroing and scan then cost about as much as the hash would.
static bool subm_use_bitmap(int64_t n, int64_t cells) {
  return ceil_div(cells, 32) <= 8 * n + (int64_t(1) << 20);
}

struct SubmWork {
  unsigned long long* table;
  uint32_t *words, *word_rank, *scan_scratch;
  int32_t *rank_row, *n_unique, *blk_cnt, *blk_off;
};

static SubmWork subm_carve(void* ws, int64_t n, int K, int64_t cells, int64_t* used) {
  Carver c(ws);
  const int64_t m = n > 0 ? n : 1;
  const int64_t nblk = ceil_div(m, kRows);
  SubmWork w{};
  if (subm_use_bitmap(n, cells)) {
    const int64_t nw = ceil_div(cells, 32);
    w.words = c.take<uint32_t>(nw);
    w.word_rank = c.take<uint32_t>(nw);
    w.scan_scratch = c.take<uint32_t>(scan_scratch_words(nw));
    w.rank_row = c.take<int32_t>(m);
    w.n_unique = c.take<int32_t>(1);
  } else {
    w.table = c.take<unsigned long long>(subm_capacity(m));
  }
  w.blk_cnt = c.take<int32_t>(nblk * K);
  w.blk_off = c.take<int32_t>(nblk * K);
  if (used) *used = c.used;
  return w;
}

}  // namespace tsc

using namespace tsc;

extern "C" int64_t tsc_subm_workspace_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                            const int32_t spatial[3]) {
  if (n < 0 || k_vol <= 0 || batch_size <= 0 || !spatial) return -1;
  const int64_t cells = (int64_t)batch_size * spatial[0] * spatial[1] * spatial[2];
  if (cells <= 0) return -1;
  int64_t used = 0;
  subm_carve(nullptr, n, k_vol, cells, &used);
  return used;
}

extern "C" int tsc_subm_pairs(const int32_t* coords, int64_t n, int32_t batch_size,
                              const int32_t spatial[3], const int32_t ksize[3],
                              const int32_t dilation[3], void* ws, int64_t ws_bytes, int32_t* nbr,
                              int32_t* pairs_in, int32_t* pairs_out, int32_t* counts,
                              tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "subm: n=%lld out of range", (long long)n);
  TSC_REQUIRE(batch_size > 0, "subm: batch_size must be positive");
  TSC_REQUIRE(spatial && ksize && dilation, "subm: null shape argument");
  const Box shape = box(spatial), ks = box(ksize), dil = box(dilation);
  TSC_REQUIRE(shape.z > 0 && shape.y > 0 && shape.x > 0, "subm: spatial shape must be positive");
  TSC_REQUIRE(ks.z > 0 && ks.y > 0 && ks.x > 0 && dil.z > 0 && dil.y > 0 && dil.x > 0,
              "subm: kernel size and dilation must be positive");
  const int64_t cells = (int64_t)batch_size * shape.z * shape.y * shape.x;
  TSC_REQUIRE(cells < 0xffffffffll,
              "subm: batch*D*H*W = %lld cells exceeds the 32-bit cell id range", (long long)cells);
  const int K = ks.z * ks.y * ks.x;
  TSC_REQUIRE(K <= 4096, "subm: kernel volume %d too large", K);
  TSC_REQUIRE(ws_bytes >= tsc_subm_workspace_bytes(n, K, batch_size, spatial),
              "subm: workspace too small");
  TSC_REQUIRE(counts != nullptr, "subm: counts is null");

  int rc = fill_u32(reinterpret_cast<uint32_t*>(counts), K + 1, 0u, s);
  if (rc) return rc;
  if (n == 0) return 0;
  TSC_REQUIRE(coords && nbr && pairs_in && pairs_out && ws, "subm: null pointer");

  const int nblk = static_cast<int>(ceil_div(n, kRows));
  const SubmWork w = subm_carve(ws, n, K, cells, nullptr);
  const int4* c4 = reinterpret_cast<const int4*>(coords);
  if (K > 64 && (rc = fill_u32(reinterpret_cast<uint32_t*>(w.blk_cnt), (int64_t)nblk * K, 0u, s)))
    return rc;
  if (w.words) {
    const int64_t nw = ceil_div(cells, 32);
    SubmGeom g{batch_size, shape, ks, dil, 0u};
    if ((rc = fill_u32(w.words, nw, 0u, s))) return rc;
    subm_mark_kernel<<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.words, counts + K);
    TSC_LAUNCH_CHECK("subm_mark");
    if ((rc = exclusive_scan_u32(w.words, 0, nw, w.word_rank, w.n_unique, w.scan_scratch, s)))
      return rc;
    if ((rc = fill_u32(reinterpret_cast<uint32_t*>(w.rank_row), n, 0xffffffffu, s))) return rc;
    subm_rank_kernel<<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.words, w.word_rank, w.rank_row);
    TSC_LAUNCH_CHECK("subm_rank");
    subm_probe_rank_kernel<<<ceil_div(n, 256), 256, 0, s>>>(c4, n, K, g, w.words, w.word_rank,
                                                            w.rank_row, w.n_unique, nbr);
    TSC_LAUNCH_CHECK("subm_probe_rank");
    subm_finish_kernel<<<nblk, kRows, 0, s>>>(c4, n, K, g, w.words, w.word_rank, w.rank_row, nbr,
                                              w.blk_cnt, nblk);
    TSC_LAUNCH_CHECK("subm_finish");
  } else {
    const int64_t cap = subm_capacity(n);
    SubmGeom g{batch_size, shape, ks, dil, static_cast<uint32_t>(cap - 1)};
    if ((rc = fill_u64(w.table, cap, kEmpty, s))) return rc;
    subm_insert_kernel<<<ceil_div(n, 256), 256, 0, s>>>(c4, n, g, w.table, counts + K);
    TSC_LAUNCH_CHECK("subm_insert");
    subm_probe_kernel<<<nblk, kRows, 0, s>>>(c4, n, K, g, w.table, nbr, w.blk_cnt, nblk);
    TSC_LAUNCH_CHECK("subm_probe");
  }
  if ((rc = scan_slot_blocks(w.blk_cnt, w.blk_off, counts, K, nblk, s))) return rc;
  subm_fill_kernel<<<nblk, kRows, 0, s>>>(nbr, n, K, w.blk_off, nblk, n, pairs_in, pairs_out);
  TSC_LAUNCH_CHECK("subm_fill");
  return 0;
}
