/*
 * trispconv_abi.h — C ABI of libtrispconv_hip.so, the MI355X (gfx950) backend
 * behind the unchanged `trispconv.pytorch` API.
 *
 * Conventions
 *   - Every pointer is caller-owned device memory (a torch tensor's data_ptr)
 *     unless the comment says "host".  The library allocates nothing: each
 *     builder has a *_workspace_bytes query and the caller passes that much
 *     scratch.
 *   - `stream` is a hipStream_t (torch.cuda.current_stream().cuda_stream).
 *     All work is enqueued on it; no entry point synchronises.
 *   - Return value: 0 = success, > 0 = invalid argument (message in
 *     tsc_last_error()), < 0 = -(hipError_t) of a failed launch.
 *   - Coordinates are int32 rows (b, z, y, x).  A slot k numbers the kernel
 *     offsets (kz, ky, kx) lexicographically: k = (kz*kH + ky)*kW + kx.
 *   - Pair tables are "padded": slot k owns entries [k*cap, k*cap + cnt[k]).
 *   - A neighbour map `nbr` is slot-major [K][n_out] int32: entry (k, o) is
 *     the input row that feeds output row o through slot k, or -1.
 *
 * Re-entrant; the only global state is the thread-local error string.
 */
#ifndef TRISPCONV_ABI_H
#define TRISPCONV_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define TSC_API __attribute__((visibility("default")))
#else
#define TSC_API
#endif

typedef void* tsc_stream_t; /* hipStream_t */

enum tsc_status { TSC_OK = 0, TSC_EINVAL = 1, TSC_ERANGE = 2, TSC_EUNSUPPORTED = 3 };
enum tsc_dtype { TSC_F32 = 0, TSC_F16 = 1, TSC_BF16 = 2 };
/* bits of the device-side status word written by the builders */
enum tsc_flags {
  TSC_FLAG_COORD_OUT_OF_GRID = 1,
  TSC_FLAG_BATCH_OUT_OF_RANGE = 2,
  TSC_FLAG_ROWS_NOT_BITMAP = 4 /* tsc_subm_pairs_from_bitmap: rows are not the bitmap's cells */
};

/* Thread-local description of the last non-zero return. */
TSC_API const char* tsc_last_error(void);
/* Bumped whenever a signature below changes. */
TSC_API int tsc_abi_version(void);

/* ------------------------------------------------------------------------
 * Submanifold pairs.  Replaces generate_subm_indice_pairs
 * (trispconv/pytorch/indices.py:67-140) including its dense lookup table
 * (:54-64), which becomes an occupancy bitmap with per-word ranks (grids of
 * up to about 2048 cells per voxel) or an open-addressing hash of 2N..4N slots.
 * The workspace depends on the grid (batch_size * D * H * W cells).
 *
 * Writes the neighbour map as columns: nbr [K][n], column t belongs to row
 * cols_row[t] (a permutation of the rows when every coordinate is in the
 * grid; -1 marks unused columns).  counts [K+2]: counts[k] = pairs in slot k
 * (pair_num), counts[K] = status flags, counts[K+1] = 1 when the columns are
 * in (b,z,y,x) order (bitmap path), 0 when they are the rows in order (hash
 * path, cols_row[t] = t).  The reference's pair lists follow from the map
 * with tsc_map_to_rows and tsc_pairs_from_map.
 *
 * Byte marks.  On dense grids the bitmap build marks each occupied cell with
 * a byte first.  A caller that builds repeatedly on one stream can keep
 * those bytes between builds (tsc_*_marks_bytes of them, zeroed once when
 * allocated) and pass them with a generation value gen in 1..255, a new one
 * per build: a build writes gen and reads only gen, so nothing zeroes the
 * marks before a build (one launch and one pass over the grid fewer).  The
 * caller zeroes them again before reusing a value.  Marks serve one
 * sequence of builds: builds on other streams, and builds that other host
 * threads launch on the same stream (their launches may interleave with
 * these), need marks of their own.  The workspace is then
 * the size given with marks_outside = 1.  tsc_*_marks_bytes returns 0 when
 * a build of that shape does not mark through bytes (it then ignores marks).
 * ------------------------------------------------------------------------ */
TSC_API int64_t tsc_subm_workspace_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                         const int32_t spatial[3] /* host */,
                                         int32_t marks_outside);
TSC_API int64_t tsc_subm_marks_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                     const int32_t spatial[3] /* host */);
TSC_API int tsc_subm_pairs(const int32_t* coords, int64_t n, int32_t batch_size,
                           const int32_t spatial[3] /* host */, const int32_t ksize[3] /* host */,
                           const int32_t dilation[3] /* host */, void* ws, int64_t ws_bytes,
                           int32_t* cols_row, int32_t* nbr, int32_t* counts, tsc_stream_t stream);

/* tsc_subm_pairs with the reference's synchronous coordinate check, but no
 * wait for the map.  The same launches and map; the call returns once the
 * kernel that checks the coordinates has finished (the rest of the build is
 * still queued on the stream) and reports result[0] = the status flags
 * (TSC_FLAG_* bits, 0 when every row is in the grid) and result[1] = 1 when
 * the columns are in (b,z,y,x) order.  The per-slot pair counts are not
 * summed: the probe's per-(slot, block) counts go to slot_blocks
 * (tsc_subm_slot_blocks_len(n, K) int32), and tsc_subm_counts turns them
 * into counts[0..K) when the caller wants them; counts[K] and counts[K+1]
 * are written as by tsc_subm_pairs.  Replaces the host read the reference's
 * build makes before it returns (pair_num is a CPU tensor, indices.py:131; a
 * coordinate outside the grid raises there) with a wait on the check alone.
 * It blocks the calling thread until then (spinning on a word of pinned host
 * memory, one per host thread and device, allocated on first use), so it is
 * not for code under graph capture: use tsc_subm_pairs there.  mask_row != 0
 * (K <= 32): nbr has K + 1 rows and, when the columns come out in (b,z,y,x)
 * order (result[1] = 1), row K receives each column's slot mask (bit k: the
 * column's row has a neighbour through slot k), which tsc_conv_forward reads
 * with nbr_ordered = 2.  marks (may be null), marks_size, gen: byte marks
 * kept by the caller (above). */
TSC_API int64_t tsc_subm_slot_blocks_len(int64_t n, int32_t k_vol);
TSC_API int tsc_subm_pairs_checked(const int32_t* coords, int64_t n, int32_t batch_size,
                                   const int32_t spatial[3] /* host */,
                                   const int32_t ksize[3] /* host */,
                                   const int32_t dilation[3] /* host */, void* ws,
                                   int64_t ws_bytes, void* marks, int64_t marks_size,
                                   int32_t gen, int32_t* cols_row, int32_t* nbr,
                                   int32_t* counts, int32_t* slot_blocks, int32_t mask_row,
                                   int32_t result[2] /* host */, tsc_stream_t stream);
/* counts[k] = sum of slot_blocks[k][*] for the n rows of a
 * tsc_subm_pairs_checked build (pair_num, indices.py:131), on the build's
 * stream.  counts_host (may be null): counts[0..K+2) are also copied there
 * and the call waits for the stream. */
TSC_API int tsc_subm_counts(const int32_t* slot_blocks, int64_t n, int32_t k_vol,
                            int32_t* counts, int32_t* counts_host /* host */,
                            tsc_stream_t stream);

/* tsc_subm_pairs without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference.  The
 * scratch is a fixed device array of tsc_subm_pairs_noalloc_limit() bytes
 * (64 MiB) in this library, one copy per GPU held until the process ends;
 * the bitmap is used only when it fits there, else the hash, and a build
 * that fits in neither is refused (TSC_EINVAL, nothing launched).  Outputs
 * are those of tsc_subm_pairs for the same choice of structure.  Calls that
 * overlap on one GPU (two streams or threads) share the array and race;
 * calls in stream order do not.  Nothing is allocated. */
TSC_API int64_t tsc_subm_pairs_noalloc_limit(void);
TSC_API int tsc_subm_pairs_noalloc(const int32_t* coords, int64_t n, int32_t batch_size,
                                   const int32_t spatial[3] /* host */,
                                   const int32_t ksize[3] /* host */,
                                   const int32_t dilation[3] /* host */, int32_t* cols_row,
                                   int32_t* nbr, int32_t* counts, tsc_stream_t stream);

/* The same build for rows that are the occupied cells of an existing
 * occupancy bitmap in rank order: one (word, rank) 8-byte entry per 32 cells
 * of the batch x spatial grid (the rank is read only for words with a set
 * bit), row t the cell of rank t, no repeats.  That is
 * exactly a strided build's output: its coordinates, and its workspace,
 * which begins with those entries (tsc_strided_count/fill).  So a
 * submanifold layer after a strided layer (indices.py:67-140 on the output of
 * :143-259) skips zeroing, marking, scanning and ranking and runs only the
 * probe.  Writes cols_row[t] = t, nbr [K][n] by row, counts [K+2] as
 * tsc_subm_pairs (counts[K+1] = 1).  Kernels 3 cells wide in x, dilation
 * < 16 in x.  The rows must be the bitmap's first n occupied cells in rank
 * order; otherwise TSC_FLAG_ROWS_NOT_BITMAP is set in counts[K]: a row whose
 * own cell is empty or has another rank than the row (a permuted, foreign or
 * out-of-grid row), or a neighbour whose rank is not below n (that neighbour
 * is left out of the map).  mask_row != 0 (K <= 32): nbr has K + 1 rows and row K
 * receives each column's slot mask, as in tsc_subm_pairs_checked. */
TSC_API int tsc_subm_pairs_from_bitmap(const int32_t* coords, int64_t n, int32_t batch_size,
                                       const int32_t spatial[3] /* host */,
                                       const int32_t ksize[3] /* host */,
                                       const int32_t dilation[3] /* host */, const void* bitmap,
                                       int64_t bitmap_entries_n, int32_t* cols_row, int32_t* nbr,
                                       int32_t* counts, int32_t mask_row, tsc_stream_t stream);

/* ------------------------------------------------------------------------
 * Pair lists from a neighbour map (the reference's IndiceData.pairs_in /
 * pairs_out, indices.py:123-124).
 *   tsc_map_to_rows: nbr_rows[k][cols_row[t]] = nbr_cols[k][t] for the
 *     n_cols columns (entries of rows no column names are left untouched).
 *   tsc_pairs_from_map: padded pairs_in/pairs_out [K][cap] from a row-major
 *     map [K][n]: slot k lists its pairs in ascending output row.
 * ------------------------------------------------------------------------ */
TSC_API int tsc_map_to_rows(const int32_t* nbr_cols, const int32_t* cols_row, int64_t n_cols,
                            int64_t n_rows, int32_t k_vol, int32_t* nbr_rows,
                            tsc_stream_t stream);
TSC_API int64_t tsc_pairs_from_map_workspace_bytes(int64_t n, int32_t k_vol);
TSC_API int tsc_pairs_from_map(const int32_t* nbr, int64_t n, int32_t k_vol, int64_t cap,
                               void* ws, int64_t ws_bytes, int32_t* pairs_in,
                               int32_t* pairs_out, tsc_stream_t stream);

/* ------------------------------------------------------------------------
 * Strided pairs.  Replaces generate_strided_indice_pairs
 * (trispconv/pytorch/indices.py:143-259): candidate generation (:177-195),
 * unique(sorted) of output keys (:215-229) and the per-slot split (:235-244).
 * Two phases; the counts are read to the host once, after both are queued:
 *   count: counts [K+3]: counts[k] = pairs in slot k, counts[K] = n_out,
 *          counts[K+1] = status flags, counts[K+2] = input rows with at
 *          least one pair (the row count of this layer's inverse, known
 *          with the same host read).
 *   The workspace begins with the output grid's occupancy bitmap, one
 *   (word, rank) 8-byte entry per 32 cells, ranks = output rows, which
 *   tsc_subm_pairs_from_bitmap can build on.  marks (may be null),
 *   marks_size, gen: byte marks kept by the caller, as for the submanifold
 *   build (tsc_strided_marks_bytes; the workspace sized with marks_outside).
 *   fill:  out_coords [n_out][4] sorted by (b,z,y,x); nbr [K][n_out];
 *          pairs_in/pairs_out [K][n] (slot k: input rows ascending, output
 *          rank of each); in_ids [n] (may be null): each input row's id
 *          among the rows with a pair (ascending), -1 for the others, which
 *          tsc_inverse_fill_ids takes.  The workspace and counts must be
 *          the ones `count` filled, and fill runs behind it on the same
 *          stream: its kernels read n_out from counts[K] on the device, so
 *          it can be launched before the counts reach the host.  out_cap
 *          is the number of rows out_coords and the map have room for (the
 *          map's row stride is n_out, not out_cap).  When n_out > out_cap
 *          neither out_coords nor nbr is written (the pair lists and in_ids
 *          still are): read the counts and call fill again with room for
 *          n_out rows.
 * ------------------------------------------------------------------------ */
TSC_API int64_t tsc_strided_workspace_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                    const int32_t out_spatial[3] /* host */,
                                    int32_t marks_outside);
TSC_API int64_t tsc_strided_marks_bytes(int64_t n, int32_t k_vol, int32_t batch_size,
                                        const int32_t out_spatial[3] /* host */);
TSC_API int tsc_strided_count(const int32_t* coords, int64_t n, int32_t batch_size,
                      const int32_t spatial[3], const int32_t ksize[3], const int32_t stride[3],
                      const int32_t padding[3], const int32_t dilation[3],
                      const int32_t out_spatial[3], void* ws, int64_t ws_bytes, void* marks,
                      int64_t marks_size, int32_t gen, int32_t* counts, tsc_stream_t stream);
TSC_API int tsc_strided_fill(const int32_t* coords, int64_t n, int32_t batch_size,
                     const int32_t spatial[3], const int32_t ksize[3], const int32_t stride[3],
                     const int32_t padding[3], const int32_t dilation[3],
                     const int32_t out_spatial[3], void* ws, int64_t ws_bytes,
                     const int32_t* counts, int64_t out_cap, int32_t* out_coords, int32_t* nbr,
                     int32_t* pairs_in, int32_t* pairs_out, int32_t* in_ids,
                     tsc_stream_t stream);

/* ------------------------------------------------------------------------
 * Inverse pairs.  Replaces the pair swap of SparseInverseConv3d
 * (trispconv/pytorch/modules.py:175-212).  Input: the forward layer's padded
 * tables (cap = forward n_in) and device pair counts.
 *   count: counts[0] = number of participating forward inputs (= n_out).
 *   fill:  out_coords [n_out][4] = forward input coords of participating
 *          rows in ascending row order; nbr [K][n_out];
 *          inv_pairs_out [K][cap] = compact id of each forward input
 *          (the inverse's pairs_in are the forward's pairs_out, unchanged).
 * ------------------------------------------------------------------------ */
TSC_API int64_t tsc_inverse_workspace_bytes(int64_t n_fwd_in);
TSC_API int tsc_inverse_count(const int32_t* fwd_pairs_in, const int32_t* fwd_counts, int32_t k_vol,
                      int64_t cap, int64_t n_fwd_in, void* ws, int64_t ws_bytes, int32_t* counts,
                      tsc_stream_t stream);
TSC_API int tsc_inverse_fill(const int32_t* fwd_pairs_in, const int32_t* fwd_pairs_out,
                     const int32_t* fwd_counts, int32_t k_vol, int64_t cap,
                     const int32_t* fwd_in_coords, int64_t n_fwd_in, void* ws, int64_t ws_bytes,
                     int64_t n_out, int32_t* out_coords, int32_t* nbr, int32_t* inv_pairs_out,
                     tsc_stream_t stream);
/* The fill, for a forward built by tsc_strided_fill with in_ids: its ids
 * are the compact ids that the count phase derives (n_out = that build's
 * counts[K+2]), so neither the count nor a workspace is needed.  Same
 * outputs as tsc_inverse_fill. */
TSC_API int tsc_inverse_fill_ids(const int32_t* fwd_pairs_in, const int32_t* fwd_pairs_out,
                                 const int32_t* fwd_counts, int32_t k_vol, int64_t cap,
                                 const int32_t* in_ids, const int32_t* fwd_in_coords,
                                 int64_t n_fwd_in, int64_t n_out, int32_t* out_coords,
                                 int32_t* nbr, int32_t* inv_pairs_out, tsc_stream_t stream);

/* ------------------------------------------------------------------------
 * Execution order for the convolution: output rows in spatial order, cut into
 * regions of region_rows rows, each region sorted (stably) by the set of
 * slots that feed its rows — rows processed together then need the same
 * weight slices and gather nearby inputs.  No reference counterpart (the
 * reference runs slot by slot); the order never changes any output value.
 *   nbr [K][n_out] is a map by columns: column t belongs to row cols_row[t]
 *   (cols_row == NULL: column t is row t).  raster != 0 says the columns are
 *   already in (b,z,y,x) order (the submanifold builder's bitmap path);
 *   otherwise they are put in Morton order of out_coords [n_out][4] when
 *   there is more than one region (region_rows < n_out; with one region the
 *   column order breaks ties and out_coords may be NULL).
 *   order [n_out] receives the processing order (rows); nbr_ordered
 *   [K][n_out] (may be NULL) the map permuted into that order: entry (k, t)
 *   belongs to row order[t], so the convolution reads it contiguously;
 *   pos_masks [n_out] (may be NULL; K <= 32) the slot mask of each position
 *   (bit k: row order[t] has a neighbour through slot k).  Placed right
 *   after nbr_ordered (as its row K), it lets the convolution skip reading
 *   every entry of a tile to learn which slots the tile uses
 *   (nbr_ordered = 2 in tsc_conv_forward).
 * ------------------------------------------------------------------------ */
TSC_API int64_t tsc_plan_workspace_bytes(int64_t n_out, int32_t k_vol);
TSC_API int tsc_conv_plan(const int32_t* nbr, const int32_t* cols_row, int32_t raster,
                          const int32_t* out_coords, int64_t n_out, int32_t k_vol,
                          int32_t batch_size, const int32_t out_spatial[3] /* host */,
                          int64_t region_rows, void* ws, int64_t ws_bytes, int32_t* order,
                          int32_t* nbr_ordered, int32_t* pos_masks, tsc_stream_t stream);

/* ------------------------------------------------------------------------
 * Weights.  Replaces normalize_spconv_weight (trispconv/pytorch/weight.py:8-50)
 * and the fp32 upcast of the GPU branch (functional.py:34-36): reads the
 * module's parameter and writes the kernel's layout in one pass.
 *   layout 0 (KRSC):  W[k][ci][co] = w[((co*K + k)*c_in + ci)]
 *   layout 1 (flat):  W[k][ci][co] = w[((k*c_in + ci)*c_out + co)]
 *                     (the internal (K, C_in, C_out) layout, and the 1x1x1
 *                      fold quirk, which re-reads KRSC storage this way)
 * The packed layout and size depend on (k_vol, c_in, c_out, dtype), which
 * choose the convolution kernel; pack once per such tuple.
 * ------------------------------------------------------------------------ */
TSC_API int64_t tsc_packed_weight_bytes(int32_t k_vol, int32_t c_in, int32_t c_out, int32_t dtype);
TSC_API int tsc_pack_weight(const void* w, int32_t w_dtype, int32_t layout, int32_t k_vol, int32_t c_in,
                    int32_t c_out, int32_t dtype, void* packed, tsc_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused gather -> GEMM -> scatter over all slots in one launch.  Replaces
 * sparse_conv_forward (trispconv/pytorch/functional.py:14-51) and the Triton
 * per-slot kernel (triton_kernels.py:16-135).  Output-stationary: each
 * output row accumulates sum_k feat[nbr[k][o]] @ W[k] in fp32 with k
 * ascending (layers with C_in % 4 == 0 and C_out % 16 == 0 that are not
 * 32x32-tile shapes sum 16 bytes of (slot, channel) products per lane quad
 * and matrix-core step instead; the smallest 32x32-tile layers sum the slots
 * of each residue mod 4 apart, then the four partial sums in order), adds
 * bias in fp32 and is rounded once to `dtype`.  No atomics; results are
 * bitwise reproducible and independent of `order`.
 *   nbr == NULL means the identity map with k_vol == 1 (1x1x1 layers).
 *   order == NULL means rows in index order.
 *   nbr_ordered != 0 means nbr is the plan's permuted map (entry (k, t)
 *   belongs to output row order[t]); 2 means its row K (nbr + K * n_out)
 *   holds the plan's pos_masks as well (K <= 32).
 *   bias may be NULL; bias_dtype is its element type.
 * ------------------------------------------------------------------------ */
TSC_API int tsc_conv_forward(const void* feat, int32_t dtype, int64_t n_in, int32_t c_in,
                     const void* packed_w, const void* bias, int32_t bias_dtype,
                     const int32_t* nbr, const int32_t* order, int32_t nbr_ordered,
                     int64_t n_out, int32_t k_vol, int32_t c_out, void* out,
                     tsc_stream_t stream);

/* ------------------------------------------------------------------------
 * The same convolution with the layers that follow it in a SparseSequential
 * chain (trispconv/pytorch/modules.py:320-329, which runs them as separate
 * torch ops on the features) folded into the store: an eval-mode
 * BatchNorm1d and a ReLU.  After the bias, in fp32, when bn_mean is not NULL:
 *   v = v * s + (beta[c] - mean[c] * s),  s = gamma[c] / sqrt(var[c] + eps)
 * i.e. (v - mean) / sqrt(var + eps) * gamma + beta, read from the running
 * statistics on every call (nothing is cached, so updated statistics take
 * effect at once).  bn_mean and bn_var come together; bn_weight (gamma) and
 * bn_bias (beta) may be NULL for 1 and 0; all four have c_out entries of
 * bn_dtype.  Then v = max(v, 0) when relu != 0 (NaN stays NaN), then one
 * rounding to `dtype`.  With bn_mean == NULL and relu == 0 it computes
 * exactly what tsc_conv_forward computes.
 * ------------------------------------------------------------------------ */
TSC_API int tsc_conv_forward_ep(const void* feat, int32_t dtype, int64_t n_in, int32_t c_in,
                                const void* packed_w, const void* bias, int32_t bias_dtype,
                                const void* bn_mean, const void* bn_var, const void* bn_weight,
                                const void* bn_bias, int32_t bn_dtype, float bn_eps,
                                int32_t relu, const int32_t* nbr, const int32_t* order,
                                int32_t nbr_ordered, int64_t n_out, int32_t k_vol, int32_t c_out,
                                void* out, tsc_stream_t stream);

/* ------------------------------------------------------------------------
 * tsc_conv_forward with the column tile width chosen by the caller instead
 * of by the layer's size: column_tile = 32, 64 or 128 (dividing c_out) runs
 * the 256-row 32x32-tile kernel with that width, always its register-gather
 * form; 0 chooses as tsc_conv_forward does (which may pick the direct-to-LDS
 * form of the same kernel).  Every width and both forms sum each output in
 * the same order, so all return the same bits.  No counterpart in the reference (its Triton
 * path autotunes block sizes, triton_kernels.py:16-30); for tests that
 * compare the widths.  Any other width, or a layer the 32x32 tile does not
 * serve, is an argument error.
 * ------------------------------------------------------------------------ */
TSC_API int tsc_conv_forward_tile(const void* feat, int32_t dtype, int64_t n_in, int32_t c_in,
                                  const void* packed_w, const void* bias, int32_t bias_dtype,
                                  const int32_t* nbr, const int32_t* order, int32_t nbr_ordered,
                                  int64_t n_out, int32_t k_vol, int32_t c_out,
                                  int32_t column_tile, void* out, tsc_stream_t stream);

/* Name of the kernel tsc_conv_forward launches for a layer of this shape
 * ("conv_mfma_kernel", "conv_dma_kernel", "conv_split_kernel",
 * "conv_narrow_kernel" or "conv_valu_kernel"; "" for invalid sizes): what a
 * kernel trace lists it under.  No counterpart in the reference; for profilers and benchmarks. */
TSC_API const char* tsc_conv_kernel_name(int32_t dtype, int32_t c_in, int32_t c_out,
                                         int32_t k_vol, int64_t n_out);

/* ------------------------------------------------------------------------
 * Sparse -> dense.  Replaces SparseConvTensor.dense (trispconv/pytorch/
 * tensor.py:72-99): writes out, zero-filled, of shape (B, C, D, H, W) when
 * channels_first != 0 else (B, D, H, W, C), with row r's C features at its
 * coordinate.  elem_bytes is the feature element size (1, 2, 4 or 8: any
 * dtype; the values are copied bit for bit).  A row whose coordinate lies outside [0,B) x [0,D) x
 * [0,H) x [0,W) is not written and sets *status to 1 (device int32, the
 * reference's range assertions).  out must be 16-byte aligned.
 * ------------------------------------------------------------------------ */
TSC_API int tsc_dense_scatter(const void* feat, int32_t elem_bytes, int64_t n, int32_t c,
                              const int32_t* coords, int32_t batch_size,
                              const int32_t spatial[3] /* host */, int32_t channels_first,
                              void* out, int32_t* status, tsc_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* TRISPCONV_ABI_H */
