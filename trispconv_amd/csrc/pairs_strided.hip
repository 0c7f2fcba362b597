// Strided indice pairs on the GPU.
//
// Reference algorithm: trispconv/pytorch/indices.py:143-259.  For slot
// k = (kz,ky,kx) in product order and each input row i in ascending order,
// c = coord(i) + pad - k*dil is a candidate when, on every axis, c is a
// multiple of the stride and 0 <= c/stride < out_dim; its output is
// o = (b_i, c/stride).  The output set is the sorted unique set of all
// candidate cells; a pair's output id is its cell's rank in that set.
//
// MI355X design: instead of concatenating candidates and running a sort-based
// unique (indices.py:215-229), every candidate sets one bit in an occupancy
// bitmap over the output grid (B*oD*oH*oW bits: 1/64 of the reference's
// int64-per-cell dense table).  An exclusive scan of the words' popcounts then
// gives each cell's rank in sorted order directly, so output coordinates come
// out sorted by (b,z,y,x) and ranks need no sort and no search.  Pair lists are
// compacted per slot in ascending input order with the same block-offset +
// wave-ballot scheme as the submanifold builder.  Two calls, count and fill;
// the fill reads the output count from the device, so it is queued right
// behind the count and the counts reach the host while it runs.
#include "common.hpp"

#include <algorithm>

namespace tsc {
namespace {

constexpr int kRows = 256;

struct StridedGeom {
  int32_t B;
  Box ks, st, pad, dil, out;
};

// Candidate output cell of input coordinate c for slot (kz,ky,kx); -1 if none.
__device__ __forceinline__ int64_t candidate(const StridedGeom& g, const int4& c, int kz, int ky,
                                             int kx) {
  const int cz = c.y + g.pad.z - kz * g.dil.z;
  const int cy = c.z + g.pad.y - ky * g.dil.y;
  const int cx = c.w + g.pad.x - kx * g.dil.x;
  // divisibility does not depend on the sign, and c < 0 gives c/s < 0 (out of
  // range) under floor division, so testing c >= 0 first is equivalent to the
  // reference's floor-mod / floor-div test
  if (cz < 0 || cy < 0 || cx < 0) return -1;
  if (cz % g.st.z || cy % g.st.y || cx % g.st.x) return -1;
  const int oz = cz / g.st.z, oy = cy / g.st.y, ox = cx / g.st.x;
  if (oz >= g.out.z || oy >= g.out.y || ox >= g.out.x) return -1;
  return ((static_cast<int64_t>(c.x) * g.out.z + oz) * g.out.y + oy) * g.out.x + ox;
}

// The slots' candidate cells of one input row.  KZ/KY/KX > 0: the kernel
// shape is known at compile time, each axis's candidate output coordinates
// are computed once (KZ + KY + KX divisions instead of 3 per slot) and every
// slot index is a constant; 0: runtime shape, one candidate() per slot.
template <int KZ, int KY, int KX>
struct Cands {
  static constexpr int K = KZ * KY * KX;
  int oz[KZ], oy[KY], ox[KX];
  int b;
  bool ok;
  __device__ __forceinline__ Cands(const StridedGeom& g, const int4& c, bool valid) {
    b = c.x;
    ok = valid;
#pragma unroll
    for (int a = 0; a < KZ; ++a) oz[a] = axis(c.y + g.pad.z - a * g.dil.z, g.st.z, g.out.z);
#pragma unroll
    for (int a = 0; a < KY; ++a) oy[a] = axis(c.z + g.pad.y - a * g.dil.y, g.st.y, g.out.y);
#pragma unroll
    for (int a = 0; a < KX; ++a) ox[a] = axis(c.w + g.pad.x - a * g.dil.x, g.st.x, g.out.x);
  }
  static __device__ __forceinline__ int axis(int v, int st, int out) {
    if (v < 0 || v % st) return -1;
    const int q = v / st;
    return q < out ? q : -1;
  }
  // slot k = (kz*KY + ky)*KX + kx with k a compile-time constant after unrolling
  __device__ __forceinline__ int64_t cell(const StridedGeom& g, int k) const {
    const int kz = k / (KY * KX), ky = (k / KX) % KY, kx = k % KX;
    if (!ok || oz[kz] < 0 || oy[ky] < 0 || ox[kx] < 0) return -1;
    return ((static_cast<int64_t>(b) * g.out.z + oz[kz]) * g.out.y + oy[ky]) * g.out.x + ox[kx];
  }
};

template <>
struct Cands<0, 0, 0> {
  int4 c;
  bool ok;
  __device__ __forceinline__ Cands(const StridedGeom&, const int4& c_, bool valid)
      : c(c_), ok(valid) {}
  __device__ __forceinline__ int64_t cell(const StridedGeom& g, int k) const {
    if (!ok) return -1;
    int kz, ky, kx;
    slot_to_zyx(k, g.ks, kz, ky, kx);
    return candidate(g, c, kz, ky, kx);
  }
};

// Marks every candidate output cell and counts each slot's pairs per block.
// BYTES: byte marks (common.hpp): each candidate cell's byte, and for a row
// whose batch index is out of range the status word kMarkBatch, receive the
// build's generation value gen by plain stores (every writer stores the same
// value); the scan packs the bytes equal to gen into the bitmap and writes
// the status flags.  Otherwise the cells' bits are set with device-scope
// atomics, which on this part are carried out beyond the XCD's L2: several
// times the cost of the byte stores plus the packing pass, so they are kept
// for sparse output grids only; bad rows then raise their flag in *status.
template <int KZ, int KY, int KX, bool BYTES>
__global__ void __launch_bounds__(kRows) strided_mark_kernel(const int4* __restrict__ coords,
                                                             int64_t n, int K, StridedGeom g,
                                                             uint2* wr, uint8_t* __restrict__ bytes,
                                                             uint32_t* __restrict__ mark_words,
                                                             uint32_t gen,
                                                             int32_t* __restrict__ blk_cnt,
                                                             int nblk, int32_t* status,
                                                             int32_t* __restrict__ paired) {
  // paired: [nblk] per-block counts of rows with a pair
  __shared__ int32_t s_cnt[kRows / kWave][64];
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int64_t i = blockIdx.x * (int64_t)kRows + t;
  const bool valid = i < n;
  const int4 c = valid ? coords[i] : make_int4(-1, 0, 0, 0);
  const bool ok = valid && c.x >= 0 && c.x < g.B;
  if (valid && !ok) {
    if constexpr (BYTES)
      mark_words[kMarkBatch] = gen;
    else
      atomicOr(status, TSC_FLAG_BATCH_OUT_OF_RANGE);
  }
  const Cands<KZ, KY, KX> cand(g, c, ok);
  constexpr int KC = KZ * KY * KX;
  if constexpr (BYTES) {
    const uint8_t mark = static_cast<uint8_t>(gen);
#pragma unroll
    for (int k = 0; k < (KC ? KC : K); ++k) {
      const int64_t cell = cand.cell(g, k);
      if (cell >= 0) bytes[cell] = mark;
    }
  } else if constexpr (KC > 0) {
    // One atomic per bitmap word a (kz, ky) row of candidates touches, not
    // one per candidate: the row's cells share (b, oz, oy) and their x
    // positions are a few cells apart, so they fall in one or two words.
#pragma unroll
    for (int r = 0; r < KZ * KY; ++r) {
      int64_t w0 = -1;
      uint32_t m0 = 0, m1 = 0;
#pragma unroll
      for (int kx = 0; kx < KX; ++kx) {
        const int64_t cell = cand.cell(g, r * KX + kx);
        if (cell < 0) continue;
        if (w0 < 0) w0 = cell >> 5;
        const uint32_t bit = 1u << (cell & 31);
        if ((cell >> 5) == w0)
          m0 |= bit;
        else if ((cell >> 5) == w0 + 1)
          m1 |= bit;
        else
          atomicOr(&wr[cell >> 5].x, bit);
      }
      if (m0) atomicOr(&wr[w0].x, m0);
      if (m1) atomicOr(&wr[w0 + 1].x, m1);
    }
  }
  bool any = false;  // this input row has a pair through some slot
#pragma unroll
  for (int k = 0; k < (KC ? KC : K); ++k) {
    const int64_t cell = cand.cell(g, k);
    if (!BYTES && KC == 0 && cell >= 0) atomicOr(&wr[cell >> 5].x, 1u << (cell & 31));
    any |= cell >= 0;
    const uint64_t hits = __ballot(cell >= 0);
    if (__lane_id() == 0) {
      if (k < 64)
        s_cnt[w][k] = __popcll(hits);
      else
        atomicAdd(&blk_cnt[(int64_t)k * nblk + blockIdx.x], (int)__popcll(hits));
    }
  }
  // rows with some pair: per block into row K of the count table (one
  // counter bumped by every wave would serialize them all)
  const uint64_t with_pairs = __ballot(any);
  __shared__ int32_t s_paired[kRows / kWave];
  if (__lane_id() == 0) s_paired[w] = static_cast<int32_t>(__popcll(with_pairs));
  __syncthreads();
  if (t == 0) {
    int32_t sum = 0;
#pragma unroll
    for (int ww = 0; ww < kRows / kWave; ++ww) sum += s_paired[ww];
    paired[blockIdx.x] = sum;
  }
  if (t < K && t < 64) {
    int sum = 0;
#pragma unroll
    for (int ww = 0; ww < kRows / kWave; ++ww) sum += s_cnt[ww][t];
    blk_cnt[(int64_t)t * nblk + blockIdx.x] = sum;
  }
}

// The output count the count pass left on the device, or 0 when it exceeds
// the capacity the caller sized the output coordinates and the map for (then
// neither is written; the caller reads the count and fills again).
__device__ __forceinline__ int64_t outputs_within(const int32_t* n_out_dev, int64_t out_cap) {
  const int64_t n_out = *n_out_dev;
  return n_out <= out_cap ? n_out : 0;
}

// One thread per bitmap entry: decode every set bit, in ascending order, into
// its (b, z, y, x) row at the entry's rank.
// Blocks from emit_blocks on instead fill the map [K][n_out] with -1 (one
// launch for both).
__global__ void __launch_bounds__(256) strided_emit_kernel(const uint2* __restrict__ wr,
                                                           int64_t nwords, StridedGeom g,
                                                           int4* __restrict__ out_coords,
                                                           const int32_t* __restrict__ n_out_dev,
                                                           int64_t out_cap, int emit_blocks,
                                                           uint32_t* __restrict__ map, int K) {
  const int64_t n_out = outputs_within(n_out_dev, out_cap);
  if (static_cast<int>(blockIdx.x) >= emit_blocks) {
    const int64_t nb = gridDim.x - emit_blocks;
    const int64_t map_words = n_out * K;
    for (int64_t i = (blockIdx.x - emit_blocks) * (int64_t)blockDim.x + threadIdx.x; i < map_words;
         i += nb * blockDim.x)
      map[i] = 0xffffffffu;
    return;
  }
  const int64_t wi = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (wi >= nwords || n_out == 0) return;
  const uint2 e = wr[wi];
  uint32_t bits = e.x;
  if (!bits) return;
  uint32_t rank = e.y;
  // the word's first cell, decomposed once; later cells step along x with
  // carries into y, z and the batch
  const int64_t plane = (int64_t)g.out.y * g.out.x;
  const int64_t vol = plane * g.out.z;
  const int64_t cell0 = wi << 5;
  int bb = static_cast<int>(cell0 / vol);
  const int64_t rem = cell0 - bb * vol;
  int z = static_cast<int>(rem / plane);
  const int64_t r2 = rem - z * plane;
  int y = static_cast<int>(r2 / g.out.x);
  int x = static_cast<int>(r2 - (int64_t)y * g.out.x);
  int at = 0;  // bit index of (bb, z, y, x)
  while (bits) {
    const int b = __ffs(bits) - 1;
    bits &= bits - 1;
    x += b - at;
    at = b;
    while (x >= g.out.x) {
      x -= g.out.x;
      if (++y == g.out.y) {
        y = 0;
        if (++z == g.out.z) {
          z = 0;
          ++bb;
        }
      }
    }
    if (rank < n_out) out_coords[rank] = make_int4(bb, z, y, x);
    ++rank;
  }
}

// Pair lists in ascending input row per slot (block offsets from the per-slot
// scan, wave offsets from per-wave counts, lanes ranked by ballot) and the
// output-major map [K][n_out] (n_out read from the device; the map is left
// unwritten when n_out exceeds out_cap).  Slots are taken 64 at a time (one
// LDS count row each).
template <int KZ, int KY, int KX>
__global__ void __launch_bounds__(kRows) strided_fill_kernel(const int4* __restrict__ coords,
                                                             int64_t n, int K, StridedGeom g,
                                                             const uint2* __restrict__ wr,
                                                             const int32_t* __restrict__ blk_off,
                                                             int nblk, int64_t cap,
                                                             const int32_t* __restrict__ n_out_dev,
                                                             int64_t out_cap,
                                                             int32_t* __restrict__ nbr,
                                                             int32_t* __restrict__ pairs_in,
                                                             int32_t* __restrict__ pairs_out,
                                                             int32_t* __restrict__ in_ids) {
  __shared__ int32_t s_wcnt[kRows / kWave][64];
  __shared__ int32_t s_paired[kRows / kWave];
  const int64_t n_out = *n_out_dev;
  const bool to_map = n_out <= out_cap;
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int64_t i = blockIdx.x * (int64_t)kRows + t;
  const bool valid = i < n;
  const int4 c = valid ? coords[i] : make_int4(-1, 0, 0, 0);
  const bool ok = valid && c.x >= 0 && c.x < g.B;
  const Cands<KZ, KY, KX> cand(g, c, ok);
  constexpr int KC = KZ * KY * KX;
  // The row's id among the input rows with a pair (the inverse's output
  // rows, in ascending row order): the mark counted them per block into row
  // K of the count table, whose scan gives each block's first id; within the
  // block, waves in order, lanes by ballot.
  auto write_id = [&](bool any, uint64_t with_pairs) {
    int32_t id = blk_off[(int64_t)K * nblk + blockIdx.x];
    for (int ww = 0; ww < w; ++ww) id += s_paired[ww];
    if (valid) in_ids[i] = any ? id + rank_in_wave(with_pairs) : -1;
  };
  if constexpr (KC > 0 && KC <= 64) {
    // Fixed kernel shape: every slot's bitmap entry is loaded before any is
    // used (one straight-line batch of loads, no branch per slot), then the
    // ranks and the stores.
    int64_t cell[KC];
    uint2 e[KC];
    bool any = false;
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      cell[k] = cand.cell(g, k);
      any |= cell[k] >= 0;
      const uint64_t hits = __ballot(cell[k] >= 0);
      if (__lane_id() == 0) s_wcnt[w][k] = __popcll(hits);
      e[k] = wr[cell[k] >= 0 ? cell[k] >> 5 : 0];  // entry 0 exists
    }
    const uint64_t with_pairs = __ballot(any);
    if (__lane_id() == 0) s_paired[w] = static_cast<int32_t>(__popcll(with_pairs));
    __syncthreads();
    if (in_ids) write_id(any, with_pairs);
    // s_wcnt[w][k] becomes the block offset of wave w's slot-k pairs
    if (t < KC) {
      int run = blk_off[(int64_t)t * nblk + blockIdx.x];
#pragma unroll
      for (int ww = 0; ww < kRows / kWave; ++ww) {
        const int cnt = s_wcnt[ww][t];
        s_wcnt[ww][t] = run;
        run += cnt;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const uint64_t hits = __ballot(cell[k] >= 0);
      const int base = s_wcnt[w][k];
      const int32_t rank =
          static_cast<int32_t>(e[k].y + __popc(e[k].x & ((1u << (cell[k] & 31)) - 1u)));
      const int64_t slot_pos = base + rank_in_wave(hits);
      // both bounds hold by construction; the test keeps a bad count from
      // turning into an out-of-bounds write
      if (cell[k] >= 0 && slot_pos < cap && rank < n_out) {
        pairs_in[(int64_t)k * cap + slot_pos] = static_cast<int32_t>(i);
        pairs_out[(int64_t)k * cap + slot_pos] = rank;
        if (to_map) nbr[(int64_t)k * n_out + rank] = static_cast<int32_t>(i);
      }
    }
    return;
  }
  const int KR = KC ? KC : K;
  if (in_ids) {
    bool any = false;
    for (int k = 0; k < KR; ++k) any |= cand.cell(g, k) >= 0;
    const uint64_t with_pairs = __ballot(any);
    if (__lane_id() == 0) s_paired[w] = static_cast<int32_t>(__popcll(with_pairs));
    __syncthreads();
    write_id(any, with_pairs);
  }
  for (int kb = 0; kb < KR; kb += 64) {
    const int kend = (KR - kb) < 64 ? (KR - kb) : 64;
#pragma unroll
    for (int kk = 0; kk < (KC ? (KC < 64 ? KC : 64) : kend); ++kk) {
      if (kk >= kend) break;
      const uint64_t hits = __ballot(cand.cell(g, kb + kk) >= 0);
      if (__lane_id() == 0) s_wcnt[w][kk] = __popcll(hits);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < (KC ? (KC < 64 ? KC : 64) : kend); ++kk) {
      if (kk >= kend) break;
      const int k = kb + kk;
      const int64_t cell = cand.cell(g, k);
      const uint64_t hits = __ballot(cell >= 0);
      int base = blk_off[(int64_t)k * nblk + blockIdx.x];
      for (int ww = 0; ww < w; ++ww) base += s_wcnt[ww][kk];
      if (cell >= 0) {
        const uint2 e = wr[cell >> 5];
        const int32_t rank =
            static_cast<int32_t>(e.y + __popc(e.x & ((1u << (cell & 31)) - 1u)));
        const int64_t slot_pos = base + rank_in_wave(hits);
        // both bounds hold by construction; the test keeps a bad count from
        // turning into an out-of-bounds write
        if (slot_pos < cap && rank < n_out) {
          pairs_in[(int64_t)k * cap + slot_pos] = static_cast<int32_t>(i);
          pairs_out[(int64_t)k * cap + slot_pos] = rank;
          if (to_map) nbr[(int64_t)k * n_out + rank] = static_cast<int32_t>(i);
        }
      }
    }
    __syncthreads();
  }
}

struct Layout {
  int64_t cells, nwords, nblk;
  bool bytes;  // output cells marked through a byte map
};

// The byte map costs its size twice (zeroing and packing); the atomics cost
// about one device-scope atomic per (kz, ky) candidate row.  Bytes win up to
// a few hundred output cells per input row.
constexpr int64_t kBytesPerRow = 256;

Layout layout(int64_t n, int32_t batch, const int32_t* out) {
  Layout L;
  L.cells = (int64_t)batch * out[0] * out[1] * out[2];
  L.nwords = ceil_div(L.cells > 0 ? L.cells : 1, 32);
  L.nblk = ceil_div(n > 0 ? n : 1, kRows);
  L.bytes = n > 0 && L.cells <= kBytesPerRow * n;
  return L;
}

struct Buffers {
  uint2* wr;       // output-cell bitmap entries (word, rank)
  uint32_t* scan;  // bitmap scan scratch
  int32_t* blk_cnt;
  int32_t* blk_off;
  uint8_t* bytes;  // byte marks (byte-marked builds whose marks the caller does not keep)
};

// The byte marks come last, so the other buffers sit at the same offsets
// whether or not the workspace holds them (the fill never reads them).
Buffers carve(void* ws, const Layout& L, int K, int64_t* used, bool marks_outside = false) {
  Carver c(ws);
  Buffers b;
  b.wr = c.take<uint2>(bitmap_entries(L.nwords));
  b.scan = c.take<uint32_t>(bitmap_scan_scratch_words(L.nwords));
  b.blk_cnt = c.take<int32_t>(L.nblk * (K + 1));  // row K: rows with a pair, per block
  b.blk_off = c.take<int32_t>(L.nblk * (K + 1));
  b.bytes = L.bytes && !marks_outside ? c.take<uint8_t>(marks_bytes(L.nwords)) : nullptr;
  if (used) *used = c.used;
  return b;
}

// ---------------------------------------------------------------------------
// Narrow builds of the fixed kernel shapes: output grids of fewer than 2^30
// cells and every axis with out < 2^24 and out * stride^2 < 2^32 (with fewer
// than 2^29 input rows).  All of a row's candidate arithmetic is then 32-bit.
// An axis value v = c + pad - a * dil is a candidate iff v < out * stride as
// an unsigned number (a negative v fails too) and v is a multiple of the
// stride; its output coordinate v / stride is one multiply-high by the
// axis's rounded-up reciprocal, exact for v * stride < 2^32.  An axis value
// that is no candidate carries kFar = 2^30, so a slot's cell is one
// three-way add, and a candidate iff it is below kFar (up to three kFar terms
// plus a cell below 2^30 stay below 2^32).  The general kernels above spend
// most of their time on 64-bit multiplies and the divisions, and with every
// lane busy these builds are bound by their vector instructions.
constexpr uint32_t kFar = 1u << 30;

struct NarrowGeom {
  uint32_t mag[3];  // z, y, x: ceil(2^32 / stride), 0 for stride 1
  uint32_t lim[3];  // out * stride
  uint32_t plane;   // oH * oW
  uint32_t vol;     // oD * oH * oW
};

bool narrow_geom(const StridedGeom& g, int64_t n, const Layout& L, NarrowGeom* ng) {
  if (L.cells >= kFar || n >= (int64_t(1) << 29)) return false;
  const int32_t st[3] = {g.st.z, g.st.y, g.st.x}, out[3] = {g.out.z, g.out.y, g.out.x};
  for (int a = 0; a < 3; ++a) {
    if (out[a] >= (1 << 24) || (uint64_t)out[a] * st[a] * st[a] >= (uint64_t(1) << 32))
      return false;
    ng->mag[a] = st[a] == 1 ? 0u
                            : static_cast<uint32_t>(((uint64_t(1) << 32) + st[a] - 1) / st[a]);
    ng->lim[a] = static_cast<uint32_t>(out[a]) * static_cast<uint32_t>(st[a]);
  }
  ng->plane = static_cast<uint32_t>(out[1]) * static_cast<uint32_t>(out[2]);
  ng->vol = static_cast<uint32_t>(out[0]) * ng->plane;
  return true;
}

// Output coordinate of axis value v (v < lim: v * stride < 2^32), or kFar
// for no candidate; the output coordinate is then scaled by `scale` and
// `base` is added (the row's cell offset along that axis).
__device__ __forceinline__ uint32_t narrow_axis(int v, int st, uint32_t mag, uint32_t lim,
                                                uint32_t scale, uint32_t base, bool ok) {
  const uint32_t u = static_cast<uint32_t>(v);
  const uint32_t q = mag ? __umulhi(u, mag) : u;  // u / st for u < lim
  const bool cand = ok && u < lim && u == __umul24(q, static_cast<uint32_t>(st));
  return cand ? base + q * scale : kFar;
}

template <int KZ, int KY, int KX>
struct NarrowCands {
  static constexpr int K = KZ * KY * KX;
  uint32_t zt[KZ], yt[KY], xt[KX];
  bool any;  // some slot has a candidate
  __device__ __forceinline__ NarrowCands(const StridedGeom& g, const NarrowGeom& ng,
                                         const int4& c, bool ok) {
    const uint32_t row = static_cast<uint32_t>(c.x) * ng.vol;  // batch b's first cell
    uint32_t mz = kFar, my = kFar, mx = kFar;
#pragma unroll
    for (int a = 0; a < KZ; ++a) {
      zt[a] = narrow_axis(c.y + g.pad.z - a * g.dil.z, g.st.z, ng.mag[0], ng.lim[0], ng.plane,
                          row, ok);
      mz = min(mz, zt[a]);
    }
#pragma unroll
    for (int a = 0; a < KY; ++a) {
      yt[a] = narrow_axis(c.z + g.pad.y - a * g.dil.y, g.st.y, ng.mag[1], ng.lim[1],
                          static_cast<uint32_t>(g.out.x), 0u, true);  // q * oW < 2^30
      my = min(my, yt[a]);
    }
#pragma unroll
    for (int a = 0; a < KX; ++a) {
      xt[a] = narrow_axis(c.w + g.pad.x - a * g.dil.x, g.st.x, ng.mag[2], ng.lim[2], 1u, 0u,
                          true);
      mx = min(mx, xt[a]);
    }
    any = mz < kFar && my < kFar && mx < kFar;
  }
  // slot k = (kz*KY + ky)*KX + kx, k a compile-time constant
  template <int k>
  __device__ __forceinline__ uint32_t cell() const {
    return zt[k / (KY * KX)] + yt[(k / KX) % KY] + xt[k % KX];
  }
};

// Per-wave slot counts, three 10-bit fields per lane (lane k / 3 holds slots
// 3(k/3) .. 3(k/3) + 2): one lane write per three slots.
template <int k, int KC>
__device__ __forceinline__ void count_slot(int32_t& lanes, uint32_t& packed, bool hit) {
  packed |= static_cast<uint32_t>(__popcll(__ballot(hit))) << (10 * (k % 3));
  if constexpr (k % 3 == 2 || k == KC - 1) {
    write_lane<k / 3>(lanes, static_cast<int32_t>(packed));
    packed = 0;
  }
}

__device__ __forceinline__ int32_t count_field(int32_t packed, int k) {
  return (packed >> (10 * (k % 3))) & 1023;
}

// strided_mark_kernel's byte-marking form for narrow builds: the same marks,
// counts and per-block paired rows.
template <int KZ, int KY, int KX>
__global__ void __launch_bounds__(kRows) strided_mark_narrow_kernel(
    const int4* __restrict__ coords, int64_t n, StridedGeom g, NarrowGeom ng,
    uint8_t* __restrict__ bytes, uint32_t* __restrict__ mark_words, uint32_t gen,
    int32_t* __restrict__ blk_cnt, int nblk, int32_t* __restrict__ paired) {
  constexpr int KC = KZ * KY * KX;
  constexpr int NW = (KC + 2) / 3;
  __shared__ int32_t s_cnt[kRows / kWave][NW];
  __shared__ int32_t s_paired[kRows / kWave];
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = t & (kWave - 1);
  const int64_t i = blockIdx.x * (int64_t)kRows + t;
  const bool valid = i < n;
  const int4 c = valid ? coords[i] : make_int4(-1, 0, 0, 0);
  const bool ok = valid && c.x >= 0 && c.x < g.B;
  if (valid && !ok) mark_words[kMarkBatch] = gen;
  const NarrowCands<KZ, KY, KX> cand(g, ng, c, ok);
  const uint8_t mark = static_cast<uint8_t>(gen);
  int32_t cnt = 0;
  uint32_t packed = 0;
  for_each_index(
      [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const uint32_t cell = cand.template cell<k>();
        const bool hit = cell < kFar;
        if (hit) ((global_char*)bytes)[cell] = mark;
        count_slot<k, KC>(cnt, packed, hit);
      },
      std::make_integer_sequence<int, KC>{});
  const uint64_t with_pairs = __ballot(cand.any);
  if (lane == 0) s_paired[w] = static_cast<int32_t>(__popcll(with_pairs));
  if (lane < NW) s_cnt[w][lane] = cnt;
  __syncthreads();
  if (t == 0) {
    int32_t sum = 0;
#pragma unroll
    for (int ww = 0; ww < kRows / kWave; ++ww) sum += s_paired[ww];
    paired[blockIdx.x] = sum;
  }
  if (t < KC) {
    int32_t sum = 0;
#pragma unroll
    for (int ww = 0; ww < kRows / kWave; ++ww) sum += count_field(s_cnt[ww][t / 3], t);
    blk_cnt[(int64_t)t * nblk + blockIdx.x] = sum;
  }
}

// strided_fill_kernel for narrow builds: the same lists, map and ids.  The
// stores address per-slot scalar bases plus 32-bit lane offsets.
template <int KZ, int KY, int KX>
__global__ void __launch_bounds__(kRows) strided_fill_narrow_kernel(
    const int4* __restrict__ coords, int64_t n, int K, StridedGeom g, NarrowGeom ng,
    const uint2* __restrict__ wr, const int32_t* __restrict__ blk_off, int nblk, int64_t cap,
    const int32_t* __restrict__ n_out_dev, int64_t out_cap, int32_t* __restrict__ nbr,
    int32_t* __restrict__ pairs_in, int32_t* __restrict__ pairs_out,
    int32_t* __restrict__ in_ids) {
  constexpr int KC = KZ * KY * KX;
  constexpr int NW = (KC + 2) / 3;
  __shared__ int32_t s_cnt[kRows / kWave][NW];
  __shared__ int32_t s_off[kRows / kWave][KC];
  __shared__ int32_t s_paired[kRows / kWave];
  const int32_t n_out = *n_out_dev;
  const bool to_map = n_out <= out_cap;
  const int t = threadIdx.x;
  const int w = t / kWave;
  const int lane = t & (kWave - 1);
  const int64_t i = blockIdx.x * (int64_t)kRows + t;
  const bool valid = i < n;
  const int4 c = valid ? coords[i] : make_int4(-1, 0, 0, 0);
  const bool ok = valid && c.x >= 0 && c.x < g.B;
  const NarrowCands<KZ, KY, KX> cand(g, ng, c, ok);
  // every slot's bitmap entry is loaded before any is used
  uint2 e[KC];
  int32_t cnt = 0;
  uint32_t packed = 0;
  for_each_index(
      [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const uint32_t cell = cand.template cell<k>();
        const bool hit = cell < kFar;
        e[k] = wr[hit ? cell >> 5 : 0u];  // entry 0 exists
        count_slot<k, KC>(cnt, packed, hit);
      },
      std::make_integer_sequence<int, KC>{});
  const uint64_t with_pairs = __ballot(cand.any);
  if (lane == 0) s_paired[w] = static_cast<int32_t>(__popcll(with_pairs));
  if (lane < NW) s_cnt[w][lane] = cnt;
  __syncthreads();
  if (in_ids) {
    // the row's id among the input rows with a pair: the block's first id
    // from the scan of the mark's per-block counts, then waves, then lanes
    int32_t id = blk_off[(int64_t)K * nblk + blockIdx.x];
    for (int ww = 0; ww < w; ++ww) id += s_paired[ww];
    if (valid) in_ids[i] = cand.any ? id + rank_in_wave(with_pairs) : -1;
  }
  if (t < KC) {
    // block offset of each wave's slot-t pairs
    int32_t run = blk_off[(int64_t)t * nblk + blockIdx.x];
#pragma unroll
    for (int ww = 0; ww < kRows / kWave; ++ww) {
      s_off[ww][t] = run;
      run += count_field(s_cnt[ww][t / 3], t);
    }
  }
  __syncthreads();
  const uint32_t row = static_cast<uint32_t>(i);
  const uint32_t ucap = static_cast<uint32_t>(cap), un_out = static_cast<uint32_t>(n_out);
  global_char* pin = (global_char*)pairs_in;
  global_char* pout = (global_char*)pairs_out;
  global_char* pmap = (global_char*)nbr;
  const uint64_t list_bytes = static_cast<uint64_t>(cap) * sizeof(int32_t);
  const uint64_t map_bytes = static_cast<uint64_t>(n_out) * sizeof(int32_t);
  for_each_index(
      [&](auto kc) {
        constexpr int k = decltype(kc)::value;
        const uint32_t cell = cand.template cell<k>();
        const bool hit = cell < kFar;
        const uint64_t hits = __ballot(hit);
        const uint32_t base = static_cast<uint32_t>(s_off[w][k]);
        const uint32_t rank = e[k].y + __popc(e[k].x & ~(0xffffffffu << (cell & 31u)));
        const uint32_t pos = __builtin_amdgcn_mbcnt_hi(
            static_cast<uint32_t>(hits >> 32),
            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(hits), base));
        // both bounds hold by construction; the test keeps a bad count from
        // turning into an out-of-bounds write
        if (hit && pos < ucap && rank < un_out) {
          *(global_int*)(pin + (pos << 2)) = static_cast<int32_t>(row);
          *(global_int*)(pout + (pos << 2)) = static_cast<int32_t>(rank);
          if (to_map) *(global_int*)(pmap + (rank << 2)) = static_cast<int32_t>(row);
        }
        pin += list_bytes;
        pout += list_bytes;
        pmap += map_bytes;
        asm("" : "+s"(pin), "+s"(pout), "+s"(pmap));
      },
      std::make_integer_sequence<int, KC>{});
}

// Runs F<KZ, KY, KX> for the common kernel shapes, F<0, 0, 0> otherwise.
template <template <int, int, int> class F, typename... A>
int by_shape(const Box& ks, A... a) {
  if (ks.z == 3 && ks.y == 3 && ks.x == 3) return F<3, 3, 3>::run(a...);
  if (ks.z == 2 && ks.y == 2 && ks.x == 2) return F<2, 2, 2>::run(a...);
  if (ks.z == 3 && ks.y == 1 && ks.x == 1) return F<3, 1, 1>::run(a...);
  if (ks.z == 1 && ks.y == 1 && ks.x == 1) return F<1, 1, 1>::run(a...);
  return F<0, 0, 0>::run(a...);
}

template <int KZ, int KY, int KX>
struct LaunchMark {
  static int run(const int4* c, int64_t n, int K, StridedGeom g, const NarrowGeom* ng, uint2* wr,
                 uint8_t* bytes, uint32_t* mwords, uint32_t gen, int32_t* blk_cnt, int nblk,
                 int32_t* status, int32_t* paired, hipStream_t s) {
    if constexpr (KZ * KY * KX > 0) {
      if (bytes && ng) {
        strided_mark_narrow_kernel<KZ, KY, KX><<<nblk, kRows, 0, s>>>(
            c, n, g, *ng, bytes, mwords, gen, blk_cnt, nblk, paired);
        TSC_LAUNCH_CHECK("strided_mark");
        return 0;
      }
    }
    if (bytes)
      strided_mark_kernel<KZ, KY, KX, true><<<nblk, kRows, 0, s>>>(
          c, n, K, g, wr, bytes, mwords, gen, blk_cnt, nblk, status, paired);
    else
      strided_mark_kernel<KZ, KY, KX, false><<<nblk, kRows, 0, s>>>(
          c, n, K, g, wr, nullptr, nullptr, 0u, blk_cnt, nblk, status, paired);
    TSC_LAUNCH_CHECK("strided_mark");
    return 0;
  }
};

template <int KZ, int KY, int KX>
struct LaunchFill {
  static int run(const int4* c, int64_t n, int K, StridedGeom g, const NarrowGeom* ng,
                 const uint2* wr, const int32_t* blk_off, int nblk, int64_t cap,
                 const int32_t* n_out_dev, int64_t out_cap, int32_t* nbr, int32_t* pin,
                 int32_t* pout, int32_t* in_ids, hipStream_t s) {
    if constexpr (KZ * KY * KX > 0) {
      if (ng) {
        strided_fill_narrow_kernel<KZ, KY, KX><<<nblk, kRows, 0, s>>>(
            c, n, K, g, *ng, wr, blk_off, nblk, cap, n_out_dev, out_cap, nbr, pin, pout, in_ids);
        TSC_LAUNCH_CHECK("strided_fill");
        return 0;
      }
    }
    strided_fill_kernel<KZ, KY, KX><<<nblk, kRows, 0, s>>>(c, n, K, g, wr, blk_off, nblk, cap,
                                                           n_out_dev, out_cap, nbr, pin, pout,
                                                           in_ids);
    TSC_LAUNCH_CHECK("strided_fill");
    return 0;
  }
};

int check_geom(int64_t n, int32_t batch, const int32_t* spatial, const int32_t* ksize,
               const int32_t* stride, const int32_t* padding, const int32_t* dilation,
               const int32_t* out_spatial, StridedGeom* g) {
  TSC_REQUIRE(n >= 0 && n < (int64_t(1) << 31), "strided: n=%lld out of range", (long long)n);
  TSC_REQUIRE(batch > 0, "strided: batch_size must be positive");
  for (int a = 0; a < 3; ++a) {
    TSC_REQUIRE(spatial[a] > 0 && ksize[a] > 0 && stride[a] > 0 && dilation[a] > 0 &&
                    padding[a] >= 0,
                "strided: invalid geometry on axis %d", a);
    const int num = spatial[a] + 2 * padding[a] - dilation[a] * (ksize[a] - 1) - 1;
    TSC_REQUIRE(num >= 0, "strided: kernel extent exceeds the padded input on axis %d", a);
    const int expect = num / stride[a] + 1;
    TSC_REQUIRE(out_spatial[a] == expect,
                "strided: output shape %d on axis %d, expected %d", out_spatial[a], a, expect);
  }
  const int64_t cells = (int64_t)batch * out_spatial[0] * out_spatial[1] * out_spatial[2];
  TSC_REQUIRE(cells <= (int64_t(1) << 37),
              "strided: output grid of %lld cells exceeds the 2^37-cell bitmap limit",
              (long long)cells);
  *g = StridedGeom{batch, box(ksize), box(stride), box(padding), box(dilation), box(out_spatial)};
  return 0;
}

}  // namespace
}  // namespace tsc

using namespace tsc;

extern "C" int64_t tsc_strided_workspace_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                               const int32_t out_spatial[3],
                                               int32_t marks_outside) {
  int64_t used = 0;
  carve(nullptr, layout(n, batch_size, out_spatial), k_vol, &used, marks_outside != 0);
  return used;
}

extern "C" int64_t tsc_strided_marks_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                           const int32_t out_spatial[3]) {
  (void)k_vol;
  const Layout L = layout(n, batch_size, out_spatial);
  return L.bytes ? marks_bytes(L.nwords) : 0;
}

extern "C" int tsc_strided_count(const int32_t* coords, int64_t n, int32_t batch_size,
                                 const int32_t spatial[3], const int32_t ksize[3],
                                 const int32_t stride[3], const int32_t padding[3],
                                 const int32_t dilation[3], const int32_t out_spatial[3], void* ws,
                                 int64_t ws_bytes, void* marks, int64_t marks_size, int32_t gen,
                                 int32_t* counts, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  StridedGeom g;
  int rc = check_geom(n, batch_size, spatial, ksize, stride, padding, dilation, out_spatial, &g);
  if (rc) return rc;
  const int K = ksize[0] * ksize[1] * ksize[2];
  TSC_REQUIRE(K <= 4096, "strided: kernel volume %d too large", K);
  const Layout L = layout(n, batch_size, out_spatial);
  // the caller's byte marks, used when this build marks through bytes
  const bool outside = marks != nullptr && L.bytes;
  if (outside) {
    TSC_REQUIRE(marks_size >= marks_bytes(L.nwords),
                "strided: marks of %lld bytes, this grid needs %lld", (long long)marks_size,
                (long long)marks_bytes(L.nwords));
    TSC_REQUIRE(gen >= 1 && gen <= 255, "strided: mark value %d outside 1..255", gen);
  }
  int64_t need = 0;
  carve(nullptr, L, K, &need, outside);
  TSC_REQUIRE(ws && ws_bytes >= need, "strided: workspace too small (%lld < %lld)",
              (long long)ws_bytes, (long long)need);
  TSC_REQUIRE(counts != nullptr, "strided: counts is null");
  Buffers b = carve(ws, L, K, nullptr, outside);
  uint8_t* const bytes = outside ? static_cast<uint8_t*>(marks) : b.bytes;
  uint32_t* const mwords = bytes ? mark_words(bytes, L.nwords) : nullptr;
  const uint32_t mark_gen = outside ? static_cast<uint32_t>(gen) : 1u;
  // zero the counters and the marks (the byte marks, which the scan turns
  // into every bitmap entry, or the bitmap entries), in one launch.  Marks
  // the caller keeps are not zeroed (this build's generation value tells its
  // marks apart), and every counter is then written by the scan: no launch.
  if (!outside) {
    uint32_t* zero = reinterpret_cast<uint32_t*>(bytes ? static_cast<void*>(bytes)
                                                       : static_cast<void*>(b.wr));
    const int64_t zero_words = bytes ? marks_bytes(L.nwords) / 4 : 2 * bitmap_entries(L.nwords);
    if ((rc = fill2_u32(reinterpret_cast<uint32_t*>(counts), K + 3, 0u, zero, zero_words, 0u, s)))
      return rc;
  }
  if (n == 0) return 0;  // (outside needs n > 0: the fill above zeroed the counts)
  TSC_REQUIRE(coords != nullptr, "strided: coords is null");
  if (K > 64 && (rc = fill_u32(reinterpret_cast<uint32_t*>(b.blk_cnt), L.nblk * K, 0u, s)))
    return rc;
  NarrowGeom ng;
  const bool narrow = narrow_geom(g, n, L, &ng);
  if ((rc = by_shape<LaunchMark>(g.ks, reinterpret_cast<const int4*>(coords), n, K, g,
                                 narrow ? &ng : static_cast<const NarrowGeom*>(nullptr), b.wr,
                                 bytes, mwords, mark_gen, b.blk_cnt, (int)L.nblk, counts + K + 1,
                                 b.blk_cnt + (int64_t)K * L.nblk, s)))
    return rc;
  // the per-slot scan of the block counts rides in the bitmap scan's first
  // launch; with byte marks it also writes the status flags
  SlotScan slots{b.blk_cnt, b.blk_off, counts, K, (int)L.nblk, counts + K + 2};
  if (mwords) {
    slots.mark_words = mwords;
    slots.gen = mark_gen;
    slots.status = counts + K + 1;
  }
  return bitmap_scan(b.wr, L.nwords, b.scan, counts + K, s, bytes, &slots, nullptr, nullptr,
                     mark_gen);
}

extern "C" int tsc_strided_fill(const int32_t* coords, int64_t n, int32_t batch_size,
                                const int32_t spatial[3], const int32_t ksize[3],
                                const int32_t stride[3], const int32_t padding[3],
                                const int32_t dilation[3], const int32_t out_spatial[3], void* ws,
                                int64_t ws_bytes, const int32_t* counts, int64_t out_cap,
                                int32_t* out_coords, int32_t* nbr, int32_t* pairs_in,
                                int32_t* pairs_out, int32_t* in_ids, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  StridedGeom g;
  int rc = check_geom(n, batch_size, spatial, ksize, stride, padding, dilation, out_spatial, &g);
  if (rc) return rc;
  const int K = ksize[0] * ksize[1] * ksize[2];
  const Layout L = layout(n, batch_size, out_spatial);
  int64_t need = 0;
  carve(nullptr, L, K, &need, true);  // the fill reads no marks
  TSC_REQUIRE(ws && ws_bytes >= need, "strided: workspace too small");
  TSC_REQUIRE(counts != nullptr, "strided: counts is null");
  TSC_REQUIRE(out_cap >= 0 && out_cap < (int64_t(1) << 31), "strided: out_cap=%lld invalid",
              (long long)out_cap);
  if (n == 0) return 0;
  TSC_REQUIRE(coords && pairs_in && pairs_out && (out_cap == 0 || (out_coords && nbr)),
              "strided: null pointer");
  Buffers b = carve(ws, L, K, nullptr, true);
  // the output coordinates, and the map's -1 fill, in one launch; both take
  // n_out from counts[K] on the device, so this call needs no host read
  const int emit_blocks = static_cast<int>(ceil_div(L.nwords, 256));
  const int fill_blocks = static_cast<int>(
      std::min<int64_t>(std::max<int64_t>(ceil_div(out_cap * K, 256), 1), 4096));
  strided_emit_kernel<<<emit_blocks + fill_blocks, 256, 0, s>>>(
      b.wr, L.nwords, g, reinterpret_cast<int4*>(out_coords), counts + K, out_cap, emit_blocks,
      reinterpret_cast<uint32_t*>(nbr), K);
  TSC_LAUNCH_CHECK("strided_emit");
  NarrowGeom ng;
  const bool narrow = narrow_geom(g, n, L, &ng);
  return by_shape<LaunchFill>(g.ks, reinterpret_cast<const int4*>(coords), n, K, g,
                              narrow ? &ng : static_cast<const NarrowGeom*>(nullptr),
                              static_cast<const uint2*>(b.wr), static_cast<const int32_t*>(b.blk_off),
                              (int)L.nblk, n, counts + K, out_cap, nbr, pairs_in, pairs_out, in_ids,
                              s);
}
