// Inverse (transposed) indice pairs on the GPU.
//
// Reference algorithm: trispconv/pytorch/modules.py:175-212.  The inverse of a
// strided layer reuses its pairs with roles swapped: output rows are the
// forward input rows that took part in at least one forward pair, kept in
// ascending row order (the sorted unique of the concatenated pairs_in,
// :178-182), and slot k maps forward output pairs_out[k][j] to the compact id
// of forward input pairs_in[k][j] (:193-194).
//
// MI355X design: no unique() — a participation flag per forward input row, an
// exclusive scan of the flags (the compact ids, already in ascending row
// order), then one pass that writes the remapped ids, the output-major
// neighbour map and the gathered output coordinates.
#include "common.hpp"

#include <algorithm>

namespace tsc {
namespace {

__global__ void __launch_bounds__(256) inverse_mark_kernel(const int32_t* __restrict__ fwd_pin,
                                                           const int32_t* __restrict__ fwd_cnt,
                                                           int64_t cap, uint32_t* flags) {
  const int k = blockIdx.y;
  const int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (j >= fwd_cnt[k]) return;
  flags[fwd_pin[(int64_t)k * cap + j]] = 1u;
}

__global__ void __launch_bounds__(256) inverse_emit_kernel(const uint32_t* __restrict__ flags,
                                                           const uint32_t* __restrict__ id_map,
                                                           const int4* __restrict__ in_coords,
                                                           int64_t n, int4* __restrict__ out_coords,
                                                           int64_t n_out) {
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n || !flags[i]) return;
  if (id_map[i] < n_out) out_coords[id_map[i]] = in_coords[i];  // holds by construction
}

__global__ void __launch_bounds__(256) inverse_fill_kernel(const int32_t* __restrict__ fwd_pin,
                                                           const int32_t* __restrict__ fwd_pout,
                                                           const int32_t* __restrict__ fwd_cnt,
                                                           int64_t cap, int K, int64_t n_out,
                                                           const uint32_t* __restrict__ id_map,
                                                           int32_t* __restrict__ nbr,
                                                           int32_t* __restrict__ inv_pout) {
  const int k = blockIdx.y;
  const int64_t j = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (j >= fwd_cnt[k]) return;
  const int64_t e = (int64_t)k * cap + j;
  const int32_t o = static_cast<int32_t>(id_map[fwd_pin[e]]);
  inv_pout[e] = o;
  if (o < n_out) nbr[(int64_t)k * n_out + o] = fwd_pout[e];  // holds by construction
}

// The fill's first launch for ids made by the forward build: blocks below
// emit_blocks write out_coords[id] = the row's coordinates for the rows with
// an id; the others fill the map with -1.
__global__ void __launch_bounds__(256) inverse_emit_ids_kernel(const int32_t* __restrict__ in_ids,
                                                               const int4* __restrict__ in_coords,
                                                               int64_t n, int4* __restrict__ out_coords,
                                                               int64_t n_out, int emit_blocks,
                                                               uint32_t* __restrict__ nbr,
                                                               int64_t nbr_words) {
  if (static_cast<int>(blockIdx.x) >= emit_blocks) {
    for (int64_t j = (blockIdx.x - emit_blocks) * (int64_t)blockDim.x + threadIdx.x; j < nbr_words;
         j += (int64_t)(gridDim.x - emit_blocks) * blockDim.x)
      nbr[j] = 0xffffffffu;
    return;
  }
  const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int32_t id = in_ids[i];
  if (id >= 0 && id < n_out) out_coords[id] = in_coords[i];  // id < n_out holds by construction
}

struct Buffers {
  uint32_t* flags;
  uint32_t* id_map;
  uint32_t* scratch;
};

Buffers carve(void* ws, int64_t n, int64_t* used) {
  Carver c(ws);
  Buffers b;
  const int64_t m = n > 0 ? n : 1;
  b.flags = c.take<uint32_t>(m);
  b.id_map = c.take<uint32_t>(m);
  b.scratch = c.take<uint32_t>(scan_scratch_words(m));
  if (used) *used = c.used;
  return b;
}

}  // namespace
}  // namespace tsc

using namespace tsc;

extern "C" int64_t tsc_inverse_workspace_bytes(int64_t n_fwd_in) {
  int64_t used = 0;
  carve(nullptr, n_fwd_in, &used);
  return used;
}

extern "C" int tsc_inverse_count(const int32_t* fwd_pairs_in, const int32_t* fwd_counts,
                                 int32_t k_vol, int64_t cap, int64_t n_fwd_in, void* ws,
                                 int64_t ws_bytes, int32_t* counts, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(k_vol > 0 && k_vol <= 65535, "inverse: invalid kernel volume %d", k_vol);
  TSC_REQUIRE(n_fwd_in >= 0 && n_fwd_in < (int64_t(1) << 31) && cap >= n_fwd_in,
              "inverse: invalid sizes");
  TSC_REQUIRE(ws && ws_bytes >= tsc_inverse_workspace_bytes(n_fwd_in),
              "inverse: workspace too small");
  TSC_REQUIRE(counts && fwd_counts, "inverse: null counts");
  Buffers b = carve(ws, n_fwd_in, nullptr);
  int rc;
  if ((rc = fill_u32(reinterpret_cast<uint32_t*>(counts), 1, 0u, s))) return rc;
  if (n_fwd_in == 0) return 0;
  TSC_REQUIRE(fwd_pairs_in != nullptr, "inverse: null pair table");
  if ((rc = fill_u32(b.flags, n_fwd_in, 0u, s))) return rc;
  if (cap > 0) {
    dim3 grid(static_cast<unsigned>(ceil_div(cap, 256)), static_cast<unsigned>(k_vol));
    inverse_mark_kernel<<<grid, 256, 0, s>>>(fwd_pairs_in, fwd_counts, cap, b.flags);
    TSC_LAUNCH_CHECK("inverse_mark");
  }
  return exclusive_scan_u32(b.flags, 1, n_fwd_in, b.id_map, counts, b.scratch, s);
}

extern "C" int tsc_inverse_fill(const int32_t* fwd_pairs_in, const int32_t* fwd_pairs_out,
                                const int32_t* fwd_counts, int32_t k_vol, int64_t cap,
                                const int32_t* fwd_in_coords, int64_t n_fwd_in, void* ws,
                                int64_t ws_bytes, int64_t n_out, int32_t* out_coords, int32_t* nbr,
                                int32_t* inv_pairs_out, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(k_vol > 0 && k_vol <= 65535, "inverse: invalid kernel volume %d", k_vol);
  TSC_REQUIRE(n_fwd_in >= 0 && cap >= n_fwd_in && n_out >= 0 && n_out <= n_fwd_in,
              "inverse: invalid sizes");
  TSC_REQUIRE(ws && ws_bytes >= tsc_inverse_workspace_bytes(n_fwd_in),
              "inverse: workspace too small");
  if (n_out == 0) return 0;
  TSC_REQUIRE(fwd_pairs_in && fwd_pairs_out && fwd_counts && fwd_in_coords && out_coords && nbr &&
                  inv_pairs_out,
              "inverse: null pointer");
  Buffers b = carve(ws, n_fwd_in, nullptr);
  int rc;
  inverse_emit_kernel<<<ceil_div(n_fwd_in, 256), 256, 0, s>>>(
      b.flags, b.id_map, reinterpret_cast<const int4*>(fwd_in_coords), n_fwd_in,
      reinterpret_cast<int4*>(out_coords), n_out);
  TSC_LAUNCH_CHECK("inverse_emit");
  if ((rc = fill_u32(reinterpret_cast<uint32_t*>(nbr), n_out * k_vol, 0xffffffffu, s))) return rc;
  dim3 grid(static_cast<unsigned>(ceil_div(cap, 256)), static_cast<unsigned>(k_vol));
  inverse_fill_kernel<<<grid, 256, 0, s>>>(fwd_pairs_in, fwd_pairs_out, fwd_counts, cap, k_vol,
                                           n_out, b.id_map, nbr, inv_pairs_out);
  TSC_LAUNCH_CHECK("inverse_fill");
  return 0;
}

extern "C" int tsc_inverse_fill_ids(const int32_t* fwd_pairs_in, const int32_t* fwd_pairs_out,
                                    const int32_t* fwd_counts, int32_t k_vol, int64_t cap,
                                    const int32_t* in_ids, const int32_t* fwd_in_coords,
                                    int64_t n_fwd_in, int64_t n_out, int32_t* out_coords,
                                    int32_t* nbr, int32_t* inv_pairs_out, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(k_vol > 0 && k_vol <= 65535, "inverse: invalid kernel volume %d", k_vol);
  TSC_REQUIRE(n_fwd_in >= 0 && n_fwd_in < (int64_t(1) << 31) && cap >= n_fwd_in && n_out >= 0 &&
                  n_out <= n_fwd_in,
              "inverse: invalid sizes");
  if (n_out == 0) return 0;
  TSC_REQUIRE(fwd_pairs_in && fwd_pairs_out && fwd_counts && in_ids && fwd_in_coords &&
                  out_coords && nbr && inv_pairs_out,
              "inverse: null pointer");
  const int emit_blocks = static_cast<int>(ceil_div(n_fwd_in, 256));
  const int64_t nbr_words = n_out * k_vol;
  const int fill_blocks =
      static_cast<int>(std::min<int64_t>(std::max<int64_t>(ceil_div(nbr_words, 256), 1), 4096));
  inverse_emit_ids_kernel<<<emit_blocks + fill_blocks, 256, 0, s>>>(
      in_ids, reinterpret_cast<const int4*>(fwd_in_coords), n_fwd_in,
      reinterpret_cast<int4*>(out_coords), n_out, emit_blocks, reinterpret_cast<uint32_t*>(nbr),
      nbr_words);
  TSC_LAUNCH_CHECK("inverse_emit_ids");
  // every row a forward pair names has an id (it has that pair), so the ids
  // read through pairs_in are never -1
  dim3 grid(static_cast<unsigned>(ceil_div(cap, 256)), static_cast<unsigned>(k_vol));
  inverse_fill_kernel<<<grid, 256, 0, s>>>(fwd_pairs_in, fwd_pairs_out, fwd_counts, cap, k_vol,
                                           n_out, reinterpret_cast<const uint32_t*>(in_ids), nbr,
                                           inv_pairs_out);
  TSC_LAUNCH_CHECK("inverse_fill");
  return 0;
}
