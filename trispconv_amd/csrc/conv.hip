// Fused sparse convolution: gather -> GEMM -> scatter over all kernel slots in
// one launch, plus the weight packer that feeds it.
//
// Reference semantics (trispconv/pytorch/functional.py:27-51, GPU branch):
// out = 0; for k ascending: out[pairs_out[k]] += feat[pairs_in[k]] @ W[k] in
// fp32 (fp16/bf16 inputs upcast, :34-36); then + bias; then one rounding to the
// input dtype (:51).  The reference launches one Triton kernel per slot with an
// atomic-add scatter (triton_kernels.py:31-92).
//
// MI355X design: output-stationary implicit GEMM.  A workgroup owns a tile of
// output rows (in the order the plan chose) and one column tile; it keeps the
// fp32 accumulators in registers across all slots, gathers each slot's input
// rows straight into MFMA operand registers, stages the slot's weight slice in
// LDS (double-buffered), and writes each output row exactly once.  No atomics:
// every output element is a fixed sequence of fp32 operations, so results are
// bitwise reproducible and independent of the tile order.
//
// Three code shapes share that structure:
//   * mfma: f32/f16/bf16 with C_in a multiple of 16, C_out of 32 and K <= 64
//     — v_mfma_f32_32x32x16_{f16,bf16} or v_mfma_f32_32x32x2_f32, 4 waves x
//     (64 rows x BN cols) per tile.
//   * narrow: the other layers with C_in % 4 == 0 and C_out % 16 == 0 (a
//     LiDAR encoder's 4 -> 16 first layer, 16-wide outputs, K > 64) —
//     v_mfma_f32_16x16x32_{f16,bf16} or v_mfma_f32_16x16x4_f32 over (slot,
//     channel) pairs, 16 rows per wave.
//   * valu: everything else (C_in not a multiple of 4 or C_out not of 16) —
//     one output row per lane and CO columns per thread, weights read with
//     wave-uniform addresses, slots skipped when no lane of the wave needs
//     them.
//
// The epilogue adds the bias and, when asked, an eval-mode batch norm and a
// ReLU (a BatchNorm1d and ReLU following the convolution in a
// SparseSequential), all in fp32 before the one rounding.  The batch norm is
// read from its running statistics and affine parameters on every launch, so
// no folded copy of them can go stale.
#include "common.hpp"

#include <type_traits>

namespace tsc {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum Path { kValu = 0, kMfma = 1, kNarrow = 2 };

// Input-channel chunk of one stage: 64 bytes of every gathered row per lane
// half (64 channels of f16/bf16, 32 of f32), or half that when the channels
// do not divide.  With C_in an odd multiple of 16 the last chunk's upper half
// is padding: those lanes read the zero row and the packed weight holds zeros.
int pick_ck(int dtype, int c_in) {
  if (dtype == TSC_F32) return 32;
  return c_in % 64 == 0 ? 64 : 32;
}
int pick_bn(int c_out) { return c_out % 128 == 0 ? 128 : (c_out % 64 == 0 ? 64 : 32); }
int64_t mfma_chunks(int c_in, int ck) { return ceil_div(c_in, ck); }

// MFMA for every dtype when C_in is a multiple of 16 and C_out of 32 (the
// slot table of K <= 64 slots fits LDS); the narrow MFMA kernel for the other
// layers whose channels come in 4-channel pieces and 16-column tiles; VALU
// otherwise.
Path pick_path(int dtype, int c_in, int c_out, int K) {
  if (c_in % 16 == 0 && c_out % 32 == 0 && K <= 64) return kMfma;
  if (c_in % 4 == 0 && c_out % 16 == 0) return kNarrow;
  return kValu;
}

// Steps of the narrow kernel: 16 bytes of reduction values (slot, channel)
// per lane quad, i.e. 32 values for f16/bf16 and 16 for f32; the last step is
// padded with zero weights.
int64_t narrow_steps(int dtype, int K, int c_in) {
  return ceil_div((int64_t)K * c_in, 4 * (16 / dtype_bytes(dtype)));
}

// ----------------------------------------------------------- weight pack --
__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  if (dt == TSC_F32) return static_cast<const float*>(p)[i];
  if (dt == TSC_F16) return __half2float(static_cast<const __half*>(p)[i]);
  return __bfloat162float(static_cast<const __hip_bfloat16*>(p)[i]);
}

// Entry i of a per-channel parameter (bias, batch-norm statistics) as fp32
// without a branch on the dtype: two 16-bit reads that are in bounds for every
// dtype (the halves of an fp32, or the same 16-bit entry twice), then selects.
// A three-way branch here, in the epilogue, once led the compiler to leave the
// output address undefined on the bf16 arm.
__device__ __forceinline__ float load_param(const void* p, int dt, int64_t i) {
  const uint16_t* q = static_cast<const uint16_t*>(p);
  const bool wide = dt == TSC_F32;
  const uint32_t lo = q[wide ? 2 * i : i];
  const uint32_t hi = q[wide ? 2 * i + 1 : i];
  const uint32_t bits = wide ? (lo | (hi << 16)) : (dt == TSC_BF16 ? lo << 16 : 0u);
  const float h = __half2float(__ushort_as_half(static_cast<unsigned short>(lo)));
  return dt == TSC_F16 ? h : __uint_as_float(bits);
}

// What happens to an output element after the slot sum: v = acc + bias[c];
// with a batch norm v = (v - mean[c]) / sqrt(var[c] + eps) * gamma[c] +
// beta[c]; with relu v = max(v, 0) (NaN stays NaN); then one rounding.
struct Epilogue {
  const void* bias;     // per output channel, bias_dt, or null
  int bias_dt;
  const void* mean;     // batch-norm running mean and variance, or null for none
  const void* var;
  const void* gamma;    // its affine weight and bias, each null for 1 and 0
  const void* beta;
  int bn_dt;            // dtype of mean, var, gamma and beta
  float eps;
  int relu;
};

// The batch norm of channel c as v * sc + sh: sc = gamma / sqrt(var + eps),
// sh = beta - mean * sc (the linear-plus-constant form torch's CPU batch norm
// evaluates).  1 and 0 without a batch norm.
__device__ __forceinline__ void channel_affine(const Epilogue& ep, int64_t c, float& sc,
                                               float& sh) {
  sc = 1.f;
  sh = 0.f;
  if (!ep.mean) return;
  float s = 1.f / sqrtf(load_param(ep.var, ep.bn_dt, c) + ep.eps);
  if (ep.gamma) s *= load_param(ep.gamma, ep.bn_dt, c);
  const float b = ep.beta ? load_param(ep.beta, ep.bn_dt, c) : 0.f;
  sc = s;
  sh = b - load_param(ep.mean, ep.bn_dt, c) * s;
}

__device__ __forceinline__ float finish(float v, float scale, float shift, bool affine, bool relu) {
  if (affine) v = fmaf(v, scale, shift);
  if (relu) v = v < 0.f ? 0.f : v;
  return v;
}

__device__ __forceinline__ float src_weight(const void* w, int dt, int layout, int K, int c_in,
                                            int c_out, int k, int ci, int co) {
  const int64_t idx = layout == 0 ? ((int64_t)co * K + k) * c_in + ci
                                  : ((int64_t)k * c_in + ci) * c_out + co;
  return load_any(w, dt, idx);
}

__global__ void pack_valu_kernel(const void* w, int w_dt, int layout, int K, int c_in, int c_out,
                                 float* packed) {
  const int64_t total = (int64_t)K * c_in * c_out;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int co = e % c_out;
    const int ci = (e / c_out) % c_in;
    const int k = e / ((int64_t)c_in * c_out);
    packed[e] = src_weight(w, w_dt, layout, K, c_in, c_out, k, ci, co);
  }
}

// MFMA layout: [k][chunk][c_out/32][u][lane][16/sizeof(T)].  Lane l of a
// 32-column block n supplies column n*32 + l%32, and for lane half h = l/32
// the channels c*CK + h*CK/2 + u*(16/sizeof(T)) + 0.. of chunk c: the same
// channel split the A operand uses, so that each lane's A data is a
// contiguous CK/2-channel (64-byte) run of a row.  An f16/bf16 MFMA step
// (32x32x16) takes one 16-byte vector per lane; an f32 step (32x32x2) one
// element of it.
template <typename T>
__global__ void pack_mfma_kernel(const void* w, int w_dt, int layout, int K, int c_in, int c_out,
                                 int ck, T* packed) {
  constexpr int VPL = 16 / sizeof(T);  // values per 16-byte vector
  const int ub = (ck / 2) / VPL;      // vectors per lane per chunk
  const int nbt = c_out / 32;
  const int nch = (c_in + ck - 1) / ck;  // the last chunk may be half padding
  const int64_t total = (int64_t)K * nch * ck * c_out;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int i = e % VPL;
    const int lane = (e / VPL) & 63;
    int64_t r = e / (VPL * 64);
    const int u = r % ub;
    r /= ub;
    const int nb = r % nbt;
    r /= nbt;
    const int c = r % nch;
    const int k = r / nch;
    const int ci = c * ck + (lane >> 5) * (ck / 2) + u * VPL + i;
    const int co = nb * 32 + (lane & 31);
    packed[e] = from_f32<T>(ci < c_in ? src_weight(w, w_dt, layout, K, c_in, c_out, k, ci, co)
                                      : 0.f);
  }
}

// The direct-to-LDS kernel's output rows are written once and not read
// again by the launch: when a row is whole 128-byte lines (nt), non-temporal
// stores keep them from displacing the gathered input rows in the caches.
// Measured: headline 128->128 layer 310-312 -> 306-308 us, two such layers
// in sequence (the second gathering the first's output) no slower, the
// encoder's 64->64 layers 28.5 -> 28.0 us, the LiDAR 64->64 fp32 layer 137
// -> 135 us.  Not for the register-gather kernel: the 674k-row 32->64 bf16
// strided layer's output (86 MB) is the next inverse layer's input, which
// then misses the Infinity Cache (that layer 56 -> 61 us).
__device__ __forceinline__ void store_out(void* dst, uint4 v, bool nt) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  if (nt) {
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, static_cast<u32x4*>(dst));
  } else {
    *static_cast<uint4*>(dst) = v;
  }
}

// Operand source for absent neighbours: lanes whose output row has no input
// through the current slot read zeros from here instead of branching around
// their loads (64 bytes per lane are read at most).
__device__ __attribute__((aligned(256))) uint4 g_zero_row[16];

// Narrow layout: [step i][c_out/16][lane][LV], LV = 16 / sizeof(T) values.
// Lane l of 16-column tile n supplies column n*16 + l%16 and the reduction
// values r = 4*LV*i + LV*(l/16) + 0..LV-1, r = k * C_in + c for slot k and
// channel c (zero past K * C_in): the values the A operand's lane l gathers
// for its row.
template <typename T>
__global__ void pack_narrow_kernel(const void* w, int w_dt, int layout, int K, int c_in,
                                   int c_out, int64_t nsteps, T* packed) {
  constexpr int LV = 16 / (int)sizeof(T);
  const int nt_all = c_out / 16;
  const int64_t total = nsteps * nt_all * 64 * LV;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int v = e % LV;
    const int lane = (e / LV) % 64;
    const int nt = (e / (64 * LV)) % nt_all;
    const int64_t i = e / (64 * LV * (int64_t)nt_all);
    const int64_t r = 4 * LV * i + LV * (lane / 16) + v;
    const int k = static_cast<int>(r / c_in);
    const int ci = static_cast<int>(r % c_in);
    const int co = nt * 16 + lane % 16;
    packed[e] = from_f32<T>(k < K ? src_weight(w, w_dt, layout, K, c_in, c_out, k, ci, co) : 0.f);
  }
}

// ---------------------------------------------------------------- VALU --
// VB: bytes of one feature load (16 or 8 when every row is a whole number of
// such vectors and the features are aligned to them, else one element).
template <int VB> struct VecOf;
template <> struct VecOf<16> { using type = uint4; };
template <> struct VecOf<8> { using type = uint2; };
template <> struct VecOf<4> { using type = uint32_t; };
template <> struct VecOf<2> { using type = uint16_t; };

template <typename T, int CO, int VB>
__global__ void __launch_bounds__(256) conv_valu_kernel(
    const T* __restrict__ feat, int c_in, const float* __restrict__ W, Epilogue ep,
    const int32_t* __restrict__ nbr, const int32_t* __restrict__ order, int nbr_ordered,
    int64_t n_out, int K, int c_out, T* __restrict__ out) {
  using Vec = typename VecOf<VB>::type;
  constexpr int NV = VB / (int)sizeof(T);  // values per load
  static_assert(NV >= 1 && NV * (int)sizeof(T) == VB, "vector of whole elements");
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int co0 = blockIdx.y * CO;
  const bool valid = t < n_out;
  __shared__ float s_scale[CO], s_shift[CO];  // the batch norm of this block's columns
  if (threadIdx.x < CO)
    channel_affine(ep, co0 + threadIdx.x, s_scale[threadIdx.x], s_shift[threadIdx.x]);
  __syncthreads();
  const int64_t o = valid ? (order ? order[t] : t) : 0;
  float acc[CO];
#pragma unroll
  for (int c = 0; c < CO; ++c) acc[c] = 0.f;
  // Slots go in groups of G: the group's map entries are loaded together, then
  // for each NV-channel piece the G gathers are issued before any is used, so
  // a row waits on about K/G load round trips instead of K.
  constexpr int G = 9;
  const int64_t col = nbr_ordered ? t : o;  // the map's column of this row
  for (int k0 = 0; k0 < K; k0 += G) {
    int32_t j[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const int k = k0 + u;
      j[u] = valid && k < K ? (nbr ? nbr[(int64_t)k * n_out + col] : static_cast<int32_t>(o)) : -1;
    }
    uint32_t live = 0;  // slots of the group that some lane of the wave uses
#pragma unroll
    for (int u = 0; u < G; ++u) live |= (__ballot(j[u] >= 0) != 0ull ? 1u : 0u) << u;
    if (live == 0) continue;
    for (int ci0 = 0; ci0 < c_in; ci0 += NV) {
      Vec v[G];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        // one vector load through a selected pointer (a conditional load of
        // the vector gets split into per-element loads)
        const Vec* src = j[u] >= 0
                             ? reinterpret_cast<const Vec*>(feat + (int64_t)j[u] * c_in) + ci0 / NV
                             : reinterpret_cast<const Vec*>(g_zero_row);
        v[u] = *src;
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (!((live >> u) & 1u)) continue;
        const float* wk = W + ((int64_t)(k0 + u) * c_in + ci0) * c_out + co0;
        const T* vals = reinterpret_cast<const T*>(&v[u]);
#pragma unroll
        for (int q = 0; q < NV; ++q) {
          const float xv = to_f32<T>(vals[q]);
          const float* wr = wk + (int64_t)q * c_out;
#pragma unroll
          for (int c = 0; c < CO; ++c) acc[c] = fmaf(xv, wr[c], acc[c]);
        }
      }
    }
  }
  if (!valid) return;
  T* dst = out + o * c_out + co0;
#pragma unroll
  for (int c = 0; c < CO; ++c) {
    const float b = ep.bias ? load_param(ep.bias, ep.bias_dt, co0 + c) : 0.f;
    dst[c] = from_f32<T>(finish(acc[c] + b, s_scale[c], s_shift[c], ep.mean != nullptr,
                                ep.relu != 0));
  }
}

// ---------------------------------------------------------------- MFMA --
template <typename T> struct MfmaOp;
template <> struct MfmaOp<__half> {
  using V = f16x8;
  static __device__ __forceinline__ f32x16 run(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct MfmaOp<__hip_bfloat16> {
  using V = bf16x8;
  static __device__ __forceinline__ f32x16 run(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct MfmaOp<float> {
  using V = float;
  static __device__ __forceinline__ f32x16 run(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

constexpr int kTileRows = kConvTileRows;  // 4 waves x 64 rows
constexpr int kSplitRows = 64;            // rows of a small-layer tile (its 4 waves split the slots)


template <int N> using Slot = std::integral_constant<int, N>;

// XCD placement: workgroups are dispatched round-robin over the 8 XCDs, in
// grid order.  Row tiles are dealt round-robin too (the execution order puts
// the tiles with the most slots first, so every XCD gets an even share of the
// heavy ones), and all column tiles of a row tile run one after another on the
// same XCD, sharing its L2 for the gathered rows.  Returns the work item
// (row tile * ncol + column tile) of workgroup lin.
__device__ __forceinline__ uint32_t dealt_item(uint32_t lin, uint32_t grid, uint32_t ncol) {
  const uint32_t dealt = (grid / (8 * ncol)) * (8 * ncol);  // whole rounds of 8 row tiles
  const uint32_t x = lin % 8, j = lin / 8;
  return lin < dealt ? ((j / ncol) * 8 + x) * ncol + j % ncol : lin;
}

// Output rows each wave stages per epilogue pass: 32 rows of up to 256 bytes,
// else 16, so the staging area stays within 35 KB for two workgroups per CU.
constexpr int mfma_stage_rows(int row_bytes) { return row_bytes <= 256 ? 32 : 16; }

// One workgroup (4 waves, one per SIMD) per CU; each wave owns 64 rows x BN
// columns of a 256-row tile.  The work of a tile is a sequence of stages
// (slot k present in the tile, 64- or 32-channel input chunk c).  Gathered
// input rows are loaded straight into MFMA operand registers RING-1 stages
// ahead (a ring of RING register buffers, so RING-1 stages of gathers are in
// flight while one computes); the stage's weight slab is loaded into registers
// one stage ahead and written to an LDS double buffer after the MFMAs, so all
// four waves share one copy.  fp32 accumulators live in AGPRs.
template <typename T, int BN, int CK>
__global__ void __launch_bounds__(256, 2) conv_mfma_kernel(
    const T* __restrict__ feat, int c_in, const T* __restrict__ W, Epilogue ep,
    const int32_t* __restrict__ nbr, const int32_t* __restrict__ order, int nbr_ordered,
    int64_t n_out, int K, int c_out, T* __restrict__ out) {
  using Op = MfmaOp<T>;
  using V = typename Op::V;
  constexpr int RING = 2;                        // operand buffers: this stage and the next
  constexpr bool F32 = std::is_same<T, float>::value;
  constexpr int VPL = 16 / (int)sizeof(T);       // values per 16-byte vector
  constexpr int UB = (CK / 2) / VPL;             // vectors per lane per row and stage
  static_assert(UB * VPL * 2 == CK && UB >= 1, "chunk must split into 16-byte runs");
  constexpr int NB = BN / 32;                    // 32-wide column blocks
  constexpr int SLAB_VECS = BN * CK * (int)sizeof(T) / 16;  // 16-byte vectors of one weight stage
  constexpr int WV = SLAB_VECS >= 256 ? SLAB_VECS / 256 : 1;
  constexpr bool FULL = SLAB_VECS % 256 == 0;
  static_assert(WV <= 4, "weight slab too large for the register stage");

  __shared__ __attribute__((aligned(16))) uint4 s_w[2][SLAB_VECS];
  __shared__ __attribute__((aligned(16))) int32_t s_orow[kTileRows];
  __shared__ float s_bias[BN];        // this column tile's bias in fp32 (0 without one)
  __shared__ float s_scale[BN];       // its affine epilogue (1 and 0 without one)
  __shared__ float s_shift[BN];
  __shared__ uint64_t s_mask[4];      // per wave: slots its rows use (K <= 64)
  extern __shared__ int32_t s_nbr[];  // [K][kTileRows]; output staging at the end

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int h = lane >> 5;
  const uint32_t ncol = static_cast<uint32_t>(c_out / BN);
  // the launch keeps the grid below 2^31 workgroups
  const uint32_t item = dealt_item(blockIdx.x, gridDim.x, ncol);
  const int64_t tile0 = static_cast<int64_t>(item / ncol) * kTileRows;
  const int nbt = static_cast<int>(item % ncol);
  const int nch = (c_in + CK - 1) / CK;  // C_in % 16 == 0: the last chunk may be half padding

  // ---- tile set-up: output rows, their slot lists and slot masks.  The map
  // entries are read 32 slots at a time, all in flight before any is used
  // (rows past the end read column 0 and are then discarded).  A map permuted
  // into the execution order is indexed by processing position, so its first
  // batch goes out before the order lookup: one memory round trip, not two.
  {
    const int64_t tr = tile0 + t;
    const bool in = tr < n_out;
    uint64_t m = 0;
    int32_t jv[32];
    auto issue = [&](int k0, int64_t src_row, int32_t self) {
      if (nbr) {
        const int32_t* col = nbr + src_row;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int k = k0 + i < K ? k0 + i : K - 1;
          jv[i] = col[(int64_t)k * n_out];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) jv[i] = self;
      }
    };
    auto consume = [&](int k0, int32_t orow) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int k = k0 + i;
        const int32_t j = orow >= 0 ? jv[i] : -1;
        if (k < K) {
          s_nbr[k * kTileRows + t] = j;
          m |= (j >= 0 ? uint64_t(1) : uint64_t(0)) << k;
        }
      }
    };
    // column of the map holding this row: its processing position when the map
    // was permuted into the execution order (contiguous reads), else the row
    int32_t orow;
    if (nbr && nbr_ordered) {
      issue(0, in ? tr : 0, 0);
      orow = in ? (order ? order[tr] : static_cast<int32_t>(tr)) : -1;
    } else {
      orow = in ? (order ? order[tr] : static_cast<int32_t>(tr)) : -1;
      issue(0, orow >= 0 ? orow : 0, orow >= 0 ? orow : 0);
    }
    s_orow[t] = orow;
    if (t < BN) {
      const int64_t col = (int64_t)nbt * BN + t;
      s_bias[t] = ep.bias ? load_param(ep.bias, ep.bias_dt, col) : 0.f;
      channel_affine(ep, col, s_scale[t], s_shift[t]);
    }
    consume(0, orow);
    for (int k0 = 32; k0 < K; k0 += 32) {
      issue(k0, nbr_ordered ? (in ? tr : 0) : (orow >= 0 ? orow : 0), orow >= 0 ? orow : 0);
      consume(k0, orow);
    }
    // OR over the wave (two 32-bit halves)
    uint32_t lo = static_cast<uint32_t>(m), hi = static_cast<uint32_t>(m >> 32);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo |= __shfl_xor(lo, off, kWave);
      hi |= __shfl_xor(hi, off, kWave);
    }
    if (lane == 0) s_mask[wave] = (static_cast<uint64_t>(hi) << 32) | lo;
  }
  __syncthreads();
  // the tile's slots, wave-uniform (scalar registers)
  const uint64_t umask_v = s_mask[0] | s_mask[1] | s_mask[2] | s_mask[3];
  const uint64_t umask =
      (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(umask_v >> 32))) << 32) |
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(umask_v));
  // the slots this wave's own rows use
  const uint64_t wmask_v = s_mask[wave];
  const uint64_t wmask =
      (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(wmask_v >> 32))) << 32) |
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(wmask_v));
  const int r0 = wave * 64 + (lane & 31);  // tile rows of this lane's A operands
  const int r1 = r0 + 32;

  // stage (k, c) -> the next stage: the next chunk of slot k, else chunk 0
  // of the tile's next slot; k == K marks the end.  Branch-free (bit scan),
  // so a loop body is one scheduling region.  k may start at -1.
  auto advance = [&](int& k, int& c) {
    const bool done = k >= K;
    const bool more_c = c + 1 < nch;
    const uint64_t above = k + 1 < 64 ? umask >> (k + 1) : 0;
    const int nk = above ? k + 1 + __builtin_ctzll(above) : K;
    const int k2 = done ? K : (more_c ? k : nk);
    c = done ? c : (more_c ? c + 1 : 0);
    k = k2;
  };

  const uint4* Wv = reinterpret_cast<const uint4*>(W);
  const int nbt_all = c_out / 32;
  // the zero row's address, held in scalar registers for the whole kernel
  // (otherwise it is reloaded from the GOT, with a wait, in every stage)
  uint64_t zero_addr = reinterpret_cast<uint64_t>(g_zero_row);
  asm volatile("" : "+s"(zero_addr));
  const uint64_t feat_addr = reinterpret_cast<uint64_t>(feat);
  const uint32_t row_bytes = static_cast<uint32_t>(c_in) * static_cast<uint32_t>(sizeof(T));

  f32x16 acc[2][NB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][nb][i] = 0.f;

  uint4 ring[RING][2][UB];  // gathered operands: this stage and the next
  uint4 w0, w1, w2, w3;        // this thread's share of the next weight slab

  // Loads are issued whether or not the stage exists (past the last stage they
  // re-read stage 0 or the zero row), keeping the loop body straight-line.
  auto load_w = [&](int k, int c) {
    if (k >= K) k = c = 0;
    const uint4* src = Wv + (((int64_t)k * nch + c) * nbt_all + (int64_t)nbt * NB) * UB * 64 + t;
    if (FULL || t < SLAB_VECS) w0 = src[0];
    if constexpr (WV > 1) w1 = src[256];
    if constexpr (WV > 2) w2 = src[512];
    if constexpr (WV > 3) w3 = src[768];
  };
  auto store_w = [&](uint4* dst) {
    if (FULL || t < SLAB_VECS) dst[t] = w0;
    if constexpr (WV > 1) dst[256 + t] = w1;
    if constexpr (WV > 2) dst[512 + t] = w2;
    if constexpr (WV > 3) dst[768 + t] = w3;
  };
  auto load_a = [&](auto slot, int k, int c) {
    constexpr int S = decltype(slot)::value;
    const bool live = k < K;
    const int kk = live ? k : K - 1;  // reads stay in the table; dead stages use -1
    const int32_t e0 = s_nbr[kk * kTileRows + r0];
    const int32_t e1 = s_nbr[kk * kTileRows + r1];
    const int32_t j0 = live ? e0 : -1;
    const int32_t j1 = live ? e1 : -1;
    const int coff = c * CK + h * (CK / 2);
    const bool pad = coff >= c_in;  // the upper half of a half-filled last chunk
    // one 64-bit multiply-add per row, the zero row by a lane-mask select
    const uint64_t base = feat_addr + static_cast<uint64_t>(coff) * sizeof(T);
    const uint64_t a0 = static_cast<uint64_t>(static_cast<uint32_t>(j0)) * static_cast<uint64_t>(row_bytes) + base;
    const uint64_t a1 = static_cast<uint64_t>(static_cast<uint32_t>(j1)) * static_cast<uint64_t>(row_bytes) + base;
    const uint4* p0 = global_ptr<uint4>(select_lanes64(__ballot(j0 >= 0 && !pad), a0, zero_addr));
    const uint4* p1 = global_ptr<uint4>(select_lanes64(__ballot(j1 >= 0 && !pad), a1, zero_addr));
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      ring[S][0][u] = p0[u];
      ring[S][1][u] = p1[u];
    }
  };
  // Every wave takes part in every stage of its tile (the waves share the
  // weight slab through LDS), but it issues the stage's MFMAs only when one of
  // its own rows has an input through the stage's slot: the matrix core then
  // serves the other workgroup's wave on the same SIMD.  Inside a computed
  // stage, rows without input through the slot multiply the zero row and add
  // exact zeros, so skipping a stage leaves every finite result unchanged.
  auto compute = [&](auto slot, const uint4* sw, int k) {
    constexpr int S = decltype(slot)::value;
    if (k >= K || !((wmask >> k) & 1)) return;
#pragma unroll
    for (int u = 0; u < UB; ++u) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint4 bv = sw[(nb * UB + u) * 64 + lane];
        if constexpr (F32) {
          // four 32x32x2 steps per vector: step i uses element i of A and B
          const float4 a0 = __builtin_bit_cast(float4, ring[S][0][u]);
          const float4 a1 = __builtin_bit_cast(float4, ring[S][1][u]);
          const float4 b4 = __builtin_bit_cast(float4, bv);
          acc[0][nb] = Op::run(a0.x, b4.x, acc[0][nb]);
          acc[1][nb] = Op::run(a1.x, b4.x, acc[1][nb]);
          acc[0][nb] = Op::run(a0.y, b4.y, acc[0][nb]);
          acc[1][nb] = Op::run(a1.y, b4.y, acc[1][nb]);
          acc[0][nb] = Op::run(a0.z, b4.z, acc[0][nb]);
          acc[1][nb] = Op::run(a1.z, b4.z, acc[1][nb]);
          acc[0][nb] = Op::run(a0.w, b4.w, acc[0][nb]);
          acc[1][nb] = Op::run(a1.w, b4.w, acc[1][nb]);
        } else {
          const V b = __builtin_bit_cast(V, bv);
          acc[0][nb] = Op::run(__builtin_bit_cast(V, ring[S][0][u]), b, acc[0][nb]);
          acc[1][nb] = Op::run(__builtin_bit_cast(V, ring[S][1][u]), b, acc[1][nb]);
        }
      }
    }
  };

  // current stage (kc, cc) and the next one (kn, cn)
  int kc = -1, cc = nch - 1;
  advance(kc, cc);  // the tile's first slot
  int kn = kc, cn = cc;
  advance(kn, cn);
  load_w(kc, cc);
  load_a(Slot<0>{}, kc, cc);
  store_w(s_w[0]);
  __syncthreads();

  // Two waves per SIMD (two workgroups per CU): while one wave waits for its
  // gathers or at the barrier, the other's MFMAs keep the matrix core busy.
  // The next stage's loads are issued before this stage's MFMAs, the weights
  // first (they are waited for before the barrier, the gathered operands only
  // in the next stage); the scheduling barrier keeps the compiler from sinking
  // the loads below the MFMAs.
  auto body = [&](auto slot) {
    constexpr int S = decltype(slot)::value;
    load_w(kn, cn);                           // next stage's weights
    load_a(Slot<(S + 1) % RING>{}, kn, cn);   // next stage's operands
    __builtin_amdgcn_sched_barrier(0);
    compute(Slot<S>{}, s_w[S], kc);
    store_w(s_w[(S + 1) % RING]);
    __syncthreads();
    kc = kn;
    cc = cn;
    advance(kn, cn);
  };
  while (kc < K) {
    body(Slot<0>{});
    body(Slot<1>{});
  }

  // ---- epilogue: + bias (and the affine map and ReLU when asked), round
  // once, store each output element once.
  const bool affine = ep.mean != nullptr;
  const bool relu = ep.relu != 0;
  // Each wave transposes its accumulators through LDS, PR rows at a time, so
  // that lanes write 16-byte pieces of output rows instead of single
  // elements.  32x32 accumulator layout: register i of lane l holds row
  // (i/4)*8 + (l/32)*4 + i%4 and column l%32 of the block.
  constexpr int ROW_BYTES = BN * (int)sizeof(T);
  constexpr int STRIDE = ROW_BYTES + 16;            // padded LDS row
  constexpr int CHUNKS = ROW_BYTES / 16;            // 16-byte pieces per row
  constexpr int PR = mfma_stage_rows(ROW_BYTES);    // rows staged per wave and pass
  char* stage = reinterpret_cast<char*>(s_nbr) + wave * PR * STRIDE;
  // this lane's columns' bias and batch norm, read once: the staging stores
  // go through a pointer the compiler cannot tell apart from these arrays, so
  // read in the loop they would be loaded again after every store
  float cbias[NB], cscale[NB], cshift[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int cl = nb * 32 + (lane & 31);
    cbias[nb] = s_bias[cl];
    cscale[nb] = s_scale[cl];
    cshift[nb] = s_shift[cl];
  }
#pragma unroll
  for (int pass = 0; pass < 64 / PR; ++pass) {
    __syncthreads();                                // the staging area is free
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rblk = rb * 32 + (i >> 2) * 8;    // + h*4 + i%4 stays within 8 rows
        if (rblk / PR != pass) continue;
        const int row = rblk % PR + h * 4 + (i & 3);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int cl = nb * 32 + (lane & 31);
          *reinterpret_cast<T*>(stage + row * STRIDE + cl * (int)sizeof(T)) =
              from_f32<T>(finish(acc[rb][nb][i] + cbias[nb], cscale[nb], cshift[nb], affine,
                                 relu));
        }
      }
    __syncthreads();
    // every LDS read of the pass is issued before the first store waits
    constexpr int NQ = PR * CHUNKS / 64;
    int32_t orows[NQ];
    uint4 vals[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int piece = q * 64 + lane;
      const int row = piece / CHUNKS, ch = piece % CHUNKS;
      orows[q] = s_orow[wave * 64 + pass * PR + row];
      vals[q] = *reinterpret_cast<const uint4*>(stage + row * STRIDE + ch * 16);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int ch = (q * 64 + lane) % CHUNKS;
      if (orows[q] >= 0)
        *reinterpret_cast<uint4*>(out + (int64_t)orows[q] * c_out + nbt * BN + ch * (16 / (int)sizeof(T))) = vals[q];
    }
  }
}

// ------------------------------------------------------ LDS DMA variant --
// The same tile schedule as conv_mfma_kernel, for layers whose stages are
// 128 bytes of every row (64 channels of f16/bf16 with C_in a multiple of 64,
// 32 of f32 with C_in a multiple of 32) and with a neighbour map (K > 1).
// A wave computes RB blocks of 32 rows: 64 rows (256-row tiles) on large
// layers, 32 (128-row tiles) on layers whose time is one heavy tile's chain
// of stages rather than the sum of all tiles' work.  Its operands reach LDS through direct-to-LDS loads
// (global_load_lds_dwordx4: each lane names a global address, the 16 bytes
// land at M0 + 16 * lane), which changes how the gathered rows pass the
// vector L1:
//   - each quad of lanes reads one row's 64 contiguous bytes, which the L1
//     serves as one access (an MFMA operand layout, 32 rows in 32 lanes,
//     costs one access per lane);
//   - the data skips the registers, so no transpose is needed to reach the
//     operand layout: the MFMA reads its operands from LDS in that layout.
// The weight slab and the map entries of each stage come the same way, so no
// load the compiler can see remains in the main loop.  The DMA instructions
// are issued from inline assembly: the compiler does not know they write LDS
// and adds no waits for them (given the builtin, it waits for every
// outstanding DMA before any LDS read).  The kernel waits with explicit
// s_waitcnt at three points (below).  Nothing else in these kernels reads M0.
__device__ __attribute__((aligned(16))) int32_t g_no_row[4] = {-1, -1, -1, -1};

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));  // low 32 bits of a shared pointer
}
__device__ __forceinline__ void dma_b128(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(m0) : "memory");
}
__device__ __forceinline__ void dma_b32(const void* g, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" : : "v"(g), "s"(m0) : "memory");
}

// Dynamic LDS of conv_dma_kernel: two weight slabs, each wave's operand rows
// of one stage (32 * RB rows x 128 bytes) and two stages of its map entries.
template <typename T, int BN, int RB>
constexpr size_t dma_pool_bytes() {
  return (size_t)2 * BN * 128 + (size_t)4 * 32 * RB * 128 + (size_t)4 * 2 * 256;
}

template <typename T, int BN, int RB>
__global__ void __launch_bounds__(256, 2) conv_dma_kernel(
    const T* __restrict__ feat, int c_in, const T* __restrict__ W, Epilogue ep,
    const int32_t* __restrict__ nbr, const int32_t* __restrict__ order, int nbr_ordered,
    int64_t n_out, int K, int c_out, T* __restrict__ out) {
  using Op = MfmaOp<T>;
  using V = typename Op::V;
  constexpr bool F32 = std::is_same<T, float>::value;
  constexpr int CK = 128 / (int)sizeof(T);   // channels of a stage: 128 bytes of each row
  constexpr int UB = 4;                      // 16-byte vectors per lane per row and stage
  constexpr int NB = BN / 32;
  constexpr int SLAB_VECS = BN * CK * (int)sizeof(T) / 16;
  constexpr int WD = SLAB_VECS / 256;        // slab DMA instructions per wave
  static_assert(SLAB_VECS % 256 == 0, "a slab splits into 1 KB pieces per wave");
  constexpr int SLAB_BYTES = SLAB_VECS * 16;
  constexpr int WR = 32 * RB;                // rows of a wave: RB blocks of 32
  constexpr int TR = 4 * WR;                 // rows of a tile
  constexpr int A_BYTES = WR * CK * (int)sizeof(T);  // one wave's rows of one stage (4 or 8 KB)
  static_assert(RB == 1 || RB == 2, "one or two 32-row blocks per wave");
  static_assert(A_BYTES == 4096 * RB && (size_t)2 * SLAB_BYTES + 4 * A_BYTES + 2048 == dma_pool_bytes<T, BN, RB>(),
                "pool layout");
  // pool: slabs [2][SLAB_BYTES] | operand rows [4 waves][A_BYTES] |
  // map entries [4 waves][2][64]; the output staging at the end
  extern __shared__ __attribute__((aligned(16))) char pool[];
  __shared__ __attribute__((aligned(16))) int32_t s_orow[TR];
  __shared__ float s_bias[BN];
  __shared__ float s_scale[BN];
  __shared__ float s_shift[BN];
  __shared__ uint64_t s_bmask[TR / 32];  // slots used by each 32-row block

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int h = lane >> 5;
  const uint32_t wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t ncol = static_cast<uint32_t>(c_out / BN);
  const uint32_t item = dealt_item(blockIdx.x, gridDim.x, ncol);
  const int64_t tile0 = static_cast<int64_t>(item / ncol) * TR;
  const int nbt = static_cast<int>(item % ncol);
  const int nch = c_in / CK;

  // ---- tile set-up: output rows and slot masks (the entries themselves are
  // loaded again stage by stage), as in conv_mfma_kernel; thread t < TR
  // takes tile row t, which wave t / WR computes
  {
    const int64_t tr = tile0 + t;
    const bool in = t < TR && tr < n_out;
    uint64_t m = 0;
    int32_t jv[32];
    auto issue = [&](int k0, int64_t src_row) {
      const int32_t* col = nbr + src_row;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int k = k0 + i < K ? k0 + i : K - 1;
        jv[i] = col[(int64_t)k * n_out];
      }
    };
    auto consume = [&](int k0, int32_t orow) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int k = k0 + i;
        if (k < K && orow >= 0 && jv[i] >= 0) m |= uint64_t(1) << k;
      }
    };
    int32_t orow;
    if (nbr_ordered == 2) {
      // the plan's slot mask of each position follows the map as its row K
      // (K <= 32): one word per row instead of all of its entries
      const uint32_t pm = reinterpret_cast<const uint32_t*>(nbr)[(int64_t)K * n_out + (in ? tr : 0)];
      orow = in ? order[tr] : -1;
      m = orow >= 0 ? pm : 0u;
    } else if (nbr_ordered) {
      issue(0, in ? tr : 0);
      orow = in ? (order ? order[tr] : static_cast<int32_t>(tr)) : -1;
    } else {
      orow = in ? (order ? order[tr] : static_cast<int32_t>(tr)) : -1;
      issue(0, orow >= 0 ? orow : 0);
    }
    if (t < TR) s_orow[t] = orow;
    if (t < BN) {
      const int64_t col = (int64_t)nbt * BN + t;
      s_bias[t] = ep.bias ? load_param(ep.bias, ep.bias_dt, col) : 0.f;
      channel_affine(ep, col, s_scale[t], s_shift[t]);
    }
    if (nbr_ordered != 2) {
      consume(0, orow);
      for (int k0 = 32; k0 < K; k0 += 32) {
        issue(k0, nbr_ordered ? (in ? tr : 0) : (orow >= 0 ? orow : 0));
        consume(k0, orow);
      }
    }
    uint32_t lo = static_cast<uint32_t>(m), hi = static_cast<uint32_t>(m >> 32);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {  // within each 32-lane half: one 32-row block
      lo |= __shfl_xor(lo, off, kWave);
      hi |= __shfl_xor(hi, off, kWave);
    }
    if (t < TR && t % 32 == 0) s_bmask[t / 32] = (static_cast<uint64_t>(hi) << 32) | lo;
  }
  __syncthreads();
  auto uniform64 = [](uint64_t v) {
    return (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32))) << 32) |
           __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  };
  uint64_t umask_v = 0;
#pragma unroll
  for (int b = 0; b < TR / 32; ++b) umask_v |= s_bmask[b];
  const uint64_t umask = uniform64(umask_v);
  uint64_t bmask[RB];  // slots used by each of this wave's 32-row blocks
  uint64_t wmask = 0;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    bmask[rb] = uniform64(s_bmask[wave * RB + rb]);
    wmask |= bmask[rb];
  }

  auto advance = [&](int& k, int& c) {
    const bool done = k >= K;
    const bool more_c = c + 1 < nch;
    const uint64_t above = k + 1 < 64 ? umask >> (k + 1) : 0;
    const int nk = above ? k + 1 + __builtin_ctzll(above) : K;
    const int k2 = done ? K : (more_c ? k : nk);
    c = done ? c : (more_c ? c + 1 : 0);
    k = k2;
  };
  auto uses = [&](int k) { return k < K && ((wmask >> k) & 1); };  // this wave computes slot k
  // block rb of this wave computes slot k (a block none of whose rows uses
  // slot k would only add exact zeros: its loads and MFMAs are skipped)
  auto buses = [&](int rb, int k) { return k < K && ((bmask[rb] >> k) & 1); };
  // blocks set of slot k: bit rb for block rb
  auto blocks = [&](int k) {
    int set = 0;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) set |= buses(rb, k) ? 1 << rb : 0;
    return set;
  };

  const uint4* Wv = reinterpret_cast<const uint4*>(W);
  const int nbt_all = c_out / 32;
  uint64_t zero_addr = reinterpret_cast<uint64_t>(g_zero_row);
  asm volatile("" : "+s"(zero_addr));
  const char* zero_row = reinterpret_cast<const char*>(zero_addr);
  uint64_t none_addr = reinterpret_cast<uint64_t>(g_no_row);
  asm volatile("" : "+s"(none_addr));
  const int32_t* no_row = reinterpret_cast<const int32_t*>(none_addr);

  // LDS offsets for M0 (wave-uniform) and the same places as pointers
  const uint32_t w_lds = lds_offset(pool);                                   // slab P: + P * SLAB_BYTES
  const uint32_t a_lds = w_lds + 2 * SLAB_BYTES + wave_u * A_BYTES;
  const uint32_t e_lds = w_lds + 2 * SLAB_BYTES + 4 * A_BYTES + wave_u * 512;  // entries P: + P * 256
  const uint4* s_w = reinterpret_cast<const uint4*>(pool);
  const char* s_a = pool + 2 * SLAB_BYTES + wave * A_BYTES;
  const int32_t* s_e = reinterpret_cast<const int32_t*>(pool + 2 * SLAB_BYTES + 4 * A_BYTES + wave * 512);

  // Map entries: lane l < WR loads the entry of its wave's row l (lanes
  // past WR load -1 from the no-row array).  Operand rows:
  // DMA instruction 2g + hh covers rows 16g..16g+15 of the wave and channel
  // half hh; the quad of lanes 4q..4q+3 reads row 16g + q, lane 4q + j its
  // 16-byte piece j ^ (q >> 2), which lands in LDS at (4q + j) * 16 of the
  // instruction's 1 KB.  So piece p of row 16g + q sits at (4q + (p ^ (q >>
  // 2))) * 16, and the MFMA's reads (lanes 0..15: rows q = 0..15, one piece)
  // hit sixteen different 16-byte bank groups.
  const int32_t orow_l = lane < WR ? s_orow[wave * WR + lane] : -1;
  const int64_t col_l = nbr_ordered ? tile0 + wave * WR + lane : (int64_t)orow_l;
  const int q = lane >> 2;
  const int piece = (lane & 3) ^ (q >> 2);

  auto dma_slab = [&](int P, int k, int c) {  // the slab of stage (k, c) into buffer P
    const uint4* src = Wv + (((int64_t)k * nch + c) * nbt_all + (int64_t)nbt * NB) * UB * 64 + t;
#pragma unroll
    for (int m = 0; m < WD; ++m)
      dma_b128(src + m * 256, w_lds + P * SLAB_BYTES + (m * 256 + wave_u * 64) * 16);
  };
  // DMA addresses.  A present row's is one 64-bit multiply-add (row times
  // row bytes plus the lane's base), an absent row's the zero row, chosen by a
  // lane-mask select: written as a C++ select, the compiler branches around
  // the multiply, an exec-masked block with its own 64-bit arithmetic per DMA.
  // Channel half hh of a stage is the same address plus 64 bytes, added in the
  // address register: the DMA's immediate offset would move its LDS
  // destination too.
  const uint64_t row_bytes = static_cast<uint64_t>(c_in) * sizeof(T);
  const uint64_t feat_lane = reinterpret_cast<uint64_t>(feat) + piece * 16;
  const uint64_t zero_lane = reinterpret_cast<uint64_t>(zero_row) + piece * 16;
  const uint64_t live_entries = __ballot(orow_l >= 0);
  const uint64_t entry_lane = reinterpret_cast<uint64_t>(nbr + col_l);  // slot 0's entry
  const uint64_t none_lane = reinterpret_cast<uint64_t>(no_row);
  auto lane_select = [](uint64_t m, uint64_t a, uint64_t b) {
    return reinterpret_cast<const char*>(select_lanes64(m, a, b));
  };
  auto dma_entries = [&](int P, int k) {  // slot k's entries of the wave's rows into buffer P
    const uint64_t a = entry_lane + static_cast<uint64_t>(k) * static_cast<uint64_t>(n_out) * 4u;
    dma_b32(lane_select(live_entries, a, none_lane), e_lds + P * 256);
  };
  // chunk c of the rows named by entry buffer P, for the blocks in set (four
  // DMAs per 32-row block)
  auto dma_rows = [&](int P, int c, int set) {
    int32_t j[2 * RB];
#pragma unroll
    for (int g = 0; g < 2 * RB; ++g) j[g] = s_e[P * 64 + 16 * g + q];
    const uint64_t base = feat_lane + static_cast<uint64_t>(c) * (CK * sizeof(T));
#pragma unroll
    for (int g = 0; g < 2 * RB; ++g) {
      if (!((set >> (g / 2)) & 1)) continue;
      const uint64_t a = static_cast<uint64_t>(static_cast<uint32_t>(j[g])) * row_bytes + base;
      const char* src = lane_select(__ballot(j[g] >= 0), a, zero_lane);
      dma_b128(src, a_lds + (2 * g) * 1024);
      dma_b128(src + 64, a_lds + (2 * g + 1) * 1024);
    }
  };
  auto wait_vm0 = [] { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); };
  // all but the youngest 4 * nblk: the row DMAs of the next stage, for nblk
  // blocks (the count must be exact: anything older, the slab and the
  // entries, has to have landed)
  auto wait_rows = [](int nblk) {
    if (nblk == 2)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (nblk == 1)
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  auto wait_lgkm0 = [] { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); };
  const int qr = lane & 15;
  auto a_read = [&](int rb, int u) {  // operand u of row block rb (rows rb*32 + lane%32)
    const int g = rb * 2 + ((lane & 31) >> 4);
    return *reinterpret_cast<const uint4*>(s_a + (2 * g + h) * 1024 + (4 * qr + (u ^ (qr >> 2))) * 16);
  };

  f32x16 acc[RB][NB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][nb][i] = 0.f;

  // stages s (kc, cc), s + 1 (kn, cn) and s + 2 (kp, cp)
  int kc = -1, cc = nch - 1;
  advance(kc, cc);
  int kn = kc, cn = cc;
  advance(kn, cn);
  int kp = kn, cp = cn;
  advance(kp, cp);
  if (kc < K) {
    dma_entries(0, kc);
    dma_slab(0, kc, cc);
  }
  if (kn < K) dma_entries(1, kn);
  wait_vm0();
  dma_rows(0, cc, blocks(kc));
  wait_vm0();
  __syncthreads();

  // Stage s (slab and entry buffers S = s % 2), with the three waits:
  //  1. vmcnt(0): this wave's rows of s have landed (issued in stage s - 1);
  //  2. the slab of s + 1 and the entries of s + 2 go out; the rows of s and
  //     the entries of s + 1 are read; lgkmcnt(0): the reads are done, so the
  //     rows of s + 1 may overwrite the wave's one operand buffer;
  //  3. MFMAs of s; vmcnt(4 * RB) (or 0 when no rows went out): the slab and
  //     the entries have landed, the 4 * RB row loads of s + 1 may still be in
  //     flight; the barrier then publishes the slab to every wave.
  auto body = [&](auto slot) {
    constexpr int S = decltype(slot)::value;
    wait_vm0();
    if (kn < K) dma_slab(S ^ 1, kn, cn);
    if (kp < K) dma_entries(S, kp);
    const int cur = blocks(kc);
    uint4 a[RB][UB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      if ((cur >> rb) & 1) {
#pragma unroll
        for (int u = 0; u < UB; ++u) a[rb][u] = a_read(rb, u);
      }
    }
    wait_lgkm0();
    const int nxt = blocks(kn);
    dma_rows(S ^ 1, cn, nxt);
    // the MFMAs of the blocks that use slot kc (a wave-uniform branch per
    // block; one loop, so the register allocation is that of a full wave)
    if (cur) {
      const uint4* sw = s_w + S * SLAB_VECS;
#pragma unroll
      for (int u = 0; u < UB; ++u) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const uint4 bv = sw[(nb * UB + u) * 64 + lane];
          if constexpr (F32) {
            // four 32x32x2 steps per vector: step e uses element e of A and B
            const float4 b4 = __builtin_bit_cast(float4, bv);
            const float bs[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
              for (int rb = 0; rb < RB; ++rb) {
                if ((cur >> rb) & 1) {
                  const float4 a4 = __builtin_bit_cast(float4, a[rb][u]);
                  const float as[4] = {a4.x, a4.y, a4.z, a4.w};
                  acc[rb][nb] = Op::run(as[e], bs[e], acc[rb][nb]);
                }
              }
          } else {
            const V b = __builtin_bit_cast(V, bv);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb)
              if ((cur >> rb) & 1)
                acc[rb][nb] = Op::run(__builtin_bit_cast(V, a[rb][u]), b, acc[rb][nb]);
          }
        }
      }
    }
    wait_rows(__builtin_popcount(nxt));
    __syncthreads();
    kc = kn;
    cc = cn;
    kn = kp;
    cn = cp;
    advance(kp, cp);
  };
  while (kc < K) {
    body(Slot<0>{});
    body(Slot<1>{});
  }
  wait_vm0();
  __syncthreads();

  // ---- epilogue, as in conv_mfma_kernel, staged in the pool
  const bool affine = ep.mean != nullptr;
  const bool relu = ep.relu != 0;
  const bool whole_lines = ((int64_t)c_out * (int64_t)sizeof(T)) % 128 == 0;
  constexpr int ROW_BYTES = BN * (int)sizeof(T);
  constexpr int STRIDE = ROW_BYTES + 16;
  constexpr int CHUNKS = ROW_BYTES / 16;
  constexpr int PR = mfma_stage_rows(ROW_BYTES);
  static_assert((size_t)4 * PR * STRIDE <= dma_pool_bytes<T, BN, RB>(), "staging exceeds the pool");
  static_assert(WR % PR == 0, "whole passes");
  char* stage = pool + wave * PR * STRIDE;
  // this lane's columns' bias and batch norm in registers (see conv_mfma_kernel)
  float cbias[NB], cscale[NB], cshift[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int cl = nb * 32 + (lane & 31);
    cbias[nb] = s_bias[cl];
    cscale[nb] = s_scale[cl];
    cshift[nb] = s_shift[cl];
  }
#pragma unroll
  for (int pass = 0; pass < WR / PR; ++pass) {
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rblk = rb * 32 + (i >> 2) * 8;
        if (rblk / PR != pass) continue;
        const int row = rblk % PR + h * 4 + (i & 3);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int cl = nb * 32 + (lane & 31);
          *reinterpret_cast<T*>(stage + row * STRIDE + cl * (int)sizeof(T)) =
              from_f32<T>(finish(acc[rb][nb][i] + cbias[nb], cscale[nb], cshift[nb], affine,
                                 relu));
        }
      }
    __syncthreads();
    constexpr int NQ = PR * CHUNKS / 64;
    int32_t orows[NQ];
    uint4 vals[NQ];
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
      const int pc = qq * 64 + lane;
      const int row = pc / CHUNKS, ch = pc % CHUNKS;
      orows[qq] = s_orow[wave * WR + pass * PR + row];
      vals[qq] = *reinterpret_cast<const uint4*>(stage + row * STRIDE + ch * 16);
    }
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
      const int ch = (qq * 64 + lane) % CHUNKS;
      if (orows[qq] >= 0)
        store_out(out + (int64_t)orows[qq] * c_out + nbt * BN + ch * (16 / (int)sizeof(T)), vals[qq],
                  whole_lines);
    }
  }
}

// ------------------------------------------------- small-layer split --
// Layers too small to give half the CUs a 256-row tile (a LiDAR encoder's
// deepest layers, ~10k rows).  There the 256-row kernel is bound by one
// tile's chain of 27 stages per CU.  This kernel takes 64-row tiles and splits
// the slots over the tile's four waves: wave w takes the slots k with
// k % 4 == w that some row of the tile uses, and loads its weight operands
// straight from global memory into registers (no shared slab, no barrier per
// stage).  The waves' partial sums meet in LDS and are added in wave order,
// ((p0 + p1) + p2) + p3.  Each row's p_w is its own slots of residue w in
// ascending order (a slot the row does not use adds exact zeros), so every
// output is still a fixed sequence of fp32 operations, independent of which
// rows share its tile.
template <typename T, int BN, int CK>
__global__ void __launch_bounds__(256, 2) conv_split_kernel(
    const T* __restrict__ feat, int c_in, const T* __restrict__ W, Epilogue ep,
    const int32_t* __restrict__ nbr, const int32_t* __restrict__ order, int nbr_ordered,
    int64_t n_out, int K, int c_out, T* __restrict__ out) {
  using Op = MfmaOp<T>;
  using V = typename Op::V;
  constexpr bool F32 = std::is_same<T, float>::value;
  constexpr int VPL = 16 / (int)sizeof(T);  // values per 16-byte vector
  constexpr int UB = (CK / 2) / VPL;        // vectors per lane per row and stage
  static_assert(UB * VPL * 2 == CK && UB >= 1, "chunk must split into 16-byte runs");
  constexpr int NB = BN / 32;               // 32-wide column blocks
  constexpr int SR = kSplitRows;
  constexpr int PART = 2 * NB * 16 * 64;    // floats of one wave's partial sums

  __shared__ int32_t s_orow[SR];
  __shared__ float s_bias[BN], s_scale[BN], s_shift[BN];
  __shared__ uint64_t s_mask[4];
  extern __shared__ int32_t s_dyn[];  // [K][SR] map entries, then 3 waves' partial sums
  int32_t* s_nbr = s_dyn;
  float* s_part = reinterpret_cast<float*>(s_dyn + K * SR);

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int h = lane >> 5;
  const uint32_t ncol = static_cast<uint32_t>(c_out / BN);
  const uint32_t item = dealt_item(blockIdx.x, gridDim.x, ncol);
  const int64_t tile0 = static_cast<int64_t>(item / ncol) * SR;
  const int nbt = static_cast<int>(item % ncol);
  const int nch = (c_in + CK - 1) / CK;

  // ---- set-up: wave w reads the map entries of its own slots for the 64
  // rows, sixteen slots at a time, all in flight before any is used; a map
  // permuted into the execution order lets the first batch go out before the
  // order lookup
  {
    const int64_t tr = tile0 + lane;
    const bool in = tr < n_out;
    uint64_t m = 0;
    int32_t jv[16];
    auto issue = [&](int i0, int64_t src_row, int32_t self) {
      if (nbr) {
        const int32_t* col = nbr + src_row;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int k = wave + 4 * (i0 + i);
          jv[i] = col[(int64_t)(k < K ? k : K - 1) * n_out];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) jv[i] = self;
      }
    };
    auto consume = [&](int i0, int32_t orow) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int k = wave + 4 * (i0 + i);
        const int32_t j = orow >= 0 ? jv[i] : -1;
        if (k < K) {
          s_nbr[k * SR + lane] = j;
          m |= (j >= 0 ? uint64_t(1) : uint64_t(0)) << k;
        }
      }
    };
    int32_t orow;
    if (nbr && nbr_ordered) {
      issue(0, in ? tr : 0, 0);
      orow = in ? (order ? order[tr] : static_cast<int32_t>(tr)) : -1;
    } else {
      orow = in ? (order ? order[tr] : static_cast<int32_t>(tr)) : -1;
      issue(0, orow >= 0 ? orow : 0, orow >= 0 ? orow : 0);
    }
    if (wave == 0) s_orow[lane] = orow;
    if (t < BN) {
      const int64_t col = (int64_t)nbt * BN + t;
      s_bias[t] = ep.bias ? load_param(ep.bias, ep.bias_dt, col) : 0.f;
      channel_affine(ep, col, s_scale[t], s_shift[t]);
    }
    consume(0, orow);
    for (int i0 = 16; wave + 4 * i0 < K; i0 += 16) {
      issue(i0, nbr_ordered ? (in ? tr : 0) : (orow >= 0 ? orow : 0), orow >= 0 ? orow : 0);
      consume(i0, orow);
    }
    uint32_t lo = static_cast<uint32_t>(m), hi = static_cast<uint32_t>(m >> 32);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      lo |= __shfl_xor(lo, off, kWave);
      hi |= __shfl_xor(hi, off, kWave);
    }
    if (lane == 0) s_mask[wave] = (static_cast<uint64_t>(hi) << 32) | lo;
  }
  __syncthreads();
  // this wave's slots (wave-uniform, scalar registers)
  const uint64_t mine_v = s_mask[wave];
  const uint64_t mine =
      (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(mine_v >> 32))) << 32) |
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(mine_v));
  const int r0 = lane & 31;  // tile rows of this lane's A operands
  const int r1 = r0 + 32;

  auto advance = [&](int& k, int& c) {
    const bool done = k >= K;
    const bool more_c = c + 1 < nch;
    const uint64_t above = k + 1 < 64 ? mine >> (k + 1) : 0;
    const int nk = above ? k + 1 + __builtin_ctzll(above) : K;
    const int k2 = done ? K : (more_c ? k : nk);
    c = done ? c : (more_c ? c + 1 : 0);
    k = k2;
  };

  const uint4* Wv = reinterpret_cast<const uint4*>(W);
  const int nbt_all = c_out / 32;
  uint64_t zero_addr = reinterpret_cast<uint64_t>(g_zero_row);
  asm volatile("" : "+s"(zero_addr));
  const uint64_t feat_addr = reinterpret_cast<uint64_t>(feat);
  const uint32_t row_bytes = static_cast<uint32_t>(c_in) * static_cast<uint32_t>(sizeof(T));

  f32x16 acc[2][NB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][nb][i] = 0.f;

  uint4 ring[2][2][UB];   // gathered operands: this stage and the next
  uint4 bring[2][NB][UB];  // weight operands: this stage and the next

  // Loads are issued whether or not the stage exists (past the last stage they
  // re-read stage 0 or the zero row), keeping the loop body straight-line.
  auto load_b = [&](auto slot, int k, int c) {
    constexpr int S = decltype(slot)::value;
    if (k >= K) k = c = 0;
    const uint4* src = Wv + (((int64_t)k * nch + c) * nbt_all + (int64_t)nbt * NB) * UB * 64 + lane;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int u = 0; u < UB; ++u) bring[S][nb][u] = src[(nb * UB + u) * 64];
  };
  auto load_a = [&](auto slot, int k, int c) {
    constexpr int S = decltype(slot)::value;
    const bool live = k < K;
    const int kk = live ? k : K - 1;
    const int32_t e0 = s_nbr[kk * SR + r0];
    const int32_t e1 = s_nbr[kk * SR + r1];
    const int32_t j0 = live ? e0 : -1;
    const int32_t j1 = live ? e1 : -1;
    const int coff = c * CK + h * (CK / 2);
    const bool pad = coff >= c_in;  // the upper half of a half-filled last chunk
    // one 64-bit multiply-add per row, the zero row by a lane-mask select
    const uint64_t base = feat_addr + static_cast<uint64_t>(coff) * sizeof(T);
    const uint64_t a0 = static_cast<uint64_t>(static_cast<uint32_t>(j0)) * static_cast<uint64_t>(row_bytes) + base;
    const uint64_t a1 = static_cast<uint64_t>(static_cast<uint32_t>(j1)) * static_cast<uint64_t>(row_bytes) + base;
    const uint4* p0 = global_ptr<uint4>(select_lanes64(__ballot(j0 >= 0 && !pad), a0, zero_addr));
    const uint4* p1 = global_ptr<uint4>(select_lanes64(__ballot(j1 >= 0 && !pad), a1, zero_addr));
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      ring[S][0][u] = p0[u];
      ring[S][1][u] = p1[u];
    }
  };
  auto compute = [&](auto slot, int k) {
    constexpr int S = decltype(slot)::value;
    if (k >= K) return;
#pragma unroll
    for (int u = 0; u < UB; ++u) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint4 bv = bring[S][nb][u];
        if constexpr (F32) {
          const float4 a0 = __builtin_bit_cast(float4, ring[S][0][u]);
          const float4 a1 = __builtin_bit_cast(float4, ring[S][1][u]);
          const float4 b4 = __builtin_bit_cast(float4, bv);
          acc[0][nb] = Op::run(a0.x, b4.x, acc[0][nb]);
          acc[1][nb] = Op::run(a1.x, b4.x, acc[1][nb]);
          acc[0][nb] = Op::run(a0.y, b4.y, acc[0][nb]);
          acc[1][nb] = Op::run(a1.y, b4.y, acc[1][nb]);
          acc[0][nb] = Op::run(a0.z, b4.z, acc[0][nb]);
          acc[1][nb] = Op::run(a1.z, b4.z, acc[1][nb]);
          acc[0][nb] = Op::run(a0.w, b4.w, acc[0][nb]);
          acc[1][nb] = Op::run(a1.w, b4.w, acc[1][nb]);
        } else {
          const V b = __builtin_bit_cast(V, bv);
          acc[0][nb] = Op::run(__builtin_bit_cast(V, ring[S][0][u]), b, acc[0][nb]);
          acc[1][nb] = Op::run(__builtin_bit_cast(V, ring[S][1][u]), b, acc[1][nb]);
        }
      }
    }
  };

  int kc = -1, cc = nch - 1;
  advance(kc, cc);  // this wave's first slot
  int kn = kc, cn = cc;
  advance(kn, cn);
  load_b(Slot<0>{}, kc, cc);
  load_a(Slot<0>{}, kc, cc);
  auto body = [&](auto slot) {
    constexpr int S = decltype(slot)::value;
    load_b(Slot<(S + 1) % 2>{}, kn, cn);  // next stage's weights
    load_a(Slot<(S + 1) % 2>{}, kn, cn);  // and operands
    __builtin_amdgcn_sched_barrier(0);
    compute(Slot<S>{}, kc);
    kc = kn;
    cc = cn;
    advance(kn, cn);
  };
  while (kc < K) {
    body(Slot<0>{});
    body(Slot<1>{});
  }

  // ---- waves 1-3 hand their partial sums to wave 0, which adds them in wave
  // order and stores.  32x32 accumulator layout: register i of lane l holds
  // row (i/4)*8 + (l/32)*4 + i%4 and column l%32 of the block.
  if (wave > 0) {
    float* dst = s_part + (wave - 1) * PART;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i) dst[((rb * NB + nb) * 16 + i) * 64 + lane] = acc[rb][nb][i];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          acc[rb][nb][i] += s_part[w * PART + ((rb * NB + nb) * 16 + i) * 64 + lane];
  const bool affine = ep.mean != nullptr;
  const bool relu = ep.relu != 0;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = rb * 32 + (i >> 2) * 8 + h * 4 + (i & 3);
      const int32_t orow = s_orow[row];
      if (orow < 0) continue;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int cl = nb * 32 + (lane & 31);
        out[(int64_t)orow * c_out + nbt * BN + cl] =
            from_f32<T>(finish(acc[rb][nb][i] + s_bias[cl], s_scale[cl], s_shift[cl], affine, relu));
      }
    }
}

// --------------------------------------------------------- narrow MFMA --
// Layers with C_in % 4 == 0 and C_out % 16 == 0 that the 32x32 tile does not
// take.  The reduction runs over r = k * C_in + c (slot k, channel c) in steps
// of 4*LV values, LV = 16 / sizeof(T): one v_mfma_f32_16x16x32 for f16/bf16,
// four v_mfma_f32_16x16x4_f32 for f32.  A wave owns 16 output rows and NT
// 16-column tiles.  Lane l supplies row l%16's values r = 4*LV*i + LV*(l/16)
// .. +LV-1 of step i, gathered straight from the input rows the map names: one
// 16-byte piece, or for f16/bf16 with C_in % 8 == 4 two 8-byte pieces of four
// channels each (the zero row for absent neighbours and the padding past
// K * C_in).
// A group of steps loads all its map entries, then all its gathers and
// weight operands, then runs its MFMAs, so a 3x3x3 layer with C_in = 4 (four
// steps) costs two dependent memory round trips.  Each output is the same
// sequence of MFMAs whatever the row order, so results are bitwise
// reproducible and independent of the execution order.
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One step on 16-byte operands per lane: a 16x16x32 MFMA for f16/bf16, four
// 16x16x4 MFMAs for f32 (MFMA e takes element e of every lane's vectors).
template <typename T> struct Mfma16;
template <> struct Mfma16<__half> {
  static __device__ __forceinline__ f32x4 step(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16<__hip_bfloat16> {
  static __device__ __forceinline__ f32x4 step(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16<float> {
  static __device__ __forceinline__ f32x4 step(uint4 a, uint4 b, f32x4 c) {
    const float4 fa = __builtin_bit_cast(float4, a);
    const float4 fb = __builtin_bit_cast(float4, b);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.x, fb.x, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.y, fb.y, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(fa.z, fb.z, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x4f32(fa.w, fb.w, c, 0, 0, 0);
  }
};

constexpr int kNarrowRows = 16;  // output rows per wave (the MFMA's M)

__device__ __forceinline__ uint4 join_pieces(const uint4& a, const uint4&) { return a; }
__device__ __forceinline__ uint4 join_pieces(const uint2& a, const uint2& b) {
  return make_uint4(a.x, a.y, b.x, b.y);
}

// Entry i of a per-channel parameter, or dflt where the pointer is null.  The
// load is issued either way (from the zero row), so a run of these issues
// back to back instead of one branch and wait at a time.
__device__ __forceinline__ float param_or(const void* p, int dt, int64_t i, float dflt) {
  const float v = load_param(p ? p : static_cast<const void*>(g_zero_row), dt, p ? i : 0);
  return p ? v : dflt;
}

// PIECE: bytes per gather (16 or 8); NT: 16-column tiles per wave.  A group
// is SG steps: 8 / NT gathers and 32 / NP weight registers per lane.
// B32: layers whose features and map stay below 2^31 bytes (NarrowB32::fits).
// The gathers and map loads then go through buffer loads with 32-bit
// offsets: an offset past the buffer's end reads zeros, which gives absent
// neighbours their zero row and the identity map (a buffer of no bytes) its
// zero entries, and the slot of a reduction index is one multiply-high by
// C_in's rounded-up reciprocal.  The 64-bit addresses and the division cost
// each step about three times the vector instructions (a wave of the 20k-row
// 16->16 fp32 layer executed 1,623 of them for 108 MFMAs).  Both forms sum
// the same products in the same order.
struct NarrowB32 {
  uint32_t feat_bytes;  // n_in * C_in * sizeof(T)
  uint32_t map_bytes;   // K * n_out * 4, 0 for the identity map
  uint32_t row_bytes;   // C_in * sizeof(T)
  uint32_t cin_mag;     // ceil(2^32 / C_in)
  static bool fits(int64_t n_in, int c_in, int elem, int64_t n_out, int K, int64_t nsteps,
                   int lv) {
    const int64_t r_end = 4 * lv * nsteps;  // reduction indices stay below this
    return n_in * c_in * elem < (int64_t(1) << 31) && (int64_t)K * n_out * 4 < (int64_t(1) << 31) &&
           n_in < (int64_t(1) << 24) && (int64_t)c_in * elem < (int64_t(1) << 24) &&
           r_end * c_in < (int64_t(1) << 32);
  }
};
constexpr int kBufferWord3 = 0x00020000;  // raw buffer, 32-bit data (gfx9 family)

template <typename T, int PIECE, int NT, bool B32>
__global__ void __launch_bounds__(256) conv_narrow_kernel(
    const T* __restrict__ feat, int c_in, const T* __restrict__ W, Epilogue ep,
    const int32_t* __restrict__ nbr, const int32_t* __restrict__ order, int nbr_ordered,
    int64_t n_out, int K, int c_out, int nsteps, NarrowB32 nb32, T* __restrict__ out) {
  using Op = Mfma16<T>;
  using Piece = typename VecOf<PIECE>::type;
  constexpr int LV = 16 / (int)sizeof(T);      // reduction values per lane and step
  constexpr int VPP = PIECE / (int)sizeof(T);  // values per piece
  constexpr int NP = 16 / PIECE;               // pieces per lane and step
  constexpr int SG = 8 / (NP * NT) > 0 ? 8 / (NP * NT) : 1;
  static_assert(PIECE == 16 || (PIECE == 8 && sizeof(T) == 2), "8- or 16-byte pieces");
  const int lane = threadIdx.x & 63;
  const uint32_t q = lane >> 4;  // which 8 values of a step this lane supplies
  const int rl = lane & 15;      // A row, B and D column of this lane
  const int64_t p0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * kNarrowRows;
  const int64_t pa = p0 + rl;  // processing position of this lane's A row
  const bool va = pa < n_out;
  const int32_t oa = va ? (order ? order[pa] : static_cast<int32_t>(pa)) : 0;
  // its column of the map; lanes past the last row read column 0 (their
  // loads are issued too, and then discarded)
  const int64_t col = va ? (nbr_ordered ? pa : oa) : 0;
  const int nt_all = c_out / 16;
  const int nt0 = blockIdx.y * NT;
  uint64_t zero_addr = reinterpret_cast<uint64_t>(g_zero_row);
  asm volatile("" : "+s"(zero_addr));
  // global (not flat) loads for both the gathered rows and the zero row
  const Piece* zero_piece =
      (const Piece*)reinterpret_cast<const __attribute__((address_space(1))) Piece*>(zero_addr);
  const uint4* Wv = reinterpret_cast<const uint4*>(W);

  // the epilogue's per-column parameters: loaded before the main loop (their
  // latency overlaps the map loads), combined after it
  float bias[NT], mean[NT], var[NT], gamma[NT], beta[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int co = (nt0 + n) * 16 + rl;
    bias[n] = param_or(ep.bias, ep.bias_dt, co, 0.f);
    mean[n] = param_or(ep.mean, ep.bn_dt, co, 0.f);
    var[n] = param_or(ep.var, ep.bn_dt, co, 1.f);
    gamma[n] = param_or(ep.gamma, ep.bn_dt, co, 1.f);
    beta[n] = param_or(ep.beta, ep.bn_dt, co, 0.f);
  }
  // The identity map (1x1x1 layers): its map loads read 0 from the zero row
  // and its row is added on, so the loop has no branch on which map it reads.
  const int32_t* map = nbr ? nbr : reinterpret_cast<const int32_t*>(g_zero_row);
  const int64_t map_mask = nbr ? ~int64_t(0) : 0;
  const int32_t ident_row = nbr ? 0 : oa;

  f32x4 acc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  // B32: buffers over the features and the map (no bytes for the identity map)
  const __amdgpu_buffer_rsrc_t feat_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(feat), 0, static_cast<int>(nb32.feat_bytes), kBufferWord3);
  const __amdgpu_buffer_rsrc_t map_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(nbr), 0, static_cast<int>(nb32.map_bytes), kBufferWord3);
  const uint32_t col4 = static_cast<uint32_t>(col) * 4u;
  const uint32_t n_out4 = static_cast<uint32_t>(n_out) * 4u;

  for (int i0 = 0; i0 < nsteps; i0 += SG) {
    int32_t j[SG * NP];
    uint32_t ch[SG * NP];
#pragma unroll
    for (int u = 0; u < SG * NP; ++u) {
      const int i = i0 + u / NP;
      const uint32_t r = 4u * LV * static_cast<uint32_t>(i) + LV * q + VPP * static_cast<uint32_t>(u % NP);
      const uint32_t k = B32 ? __umulhi(r, nb32.cin_mag) : r / static_cast<uint32_t>(c_in);
      ch[u] = r - k * static_cast<uint32_t>(c_in);
      const bool live = va && i < nsteps && k < static_cast<uint32_t>(K);
      // every lane loads (dead ones from slot K-1 of their column), so the
      // group's map loads issue back to back; dead lanes then use -1
      int32_t e;
      if constexpr (B32) {
        const uint32_t kk = live ? k : static_cast<uint32_t>(K - 1);
        e = __builtin_amdgcn_raw_buffer_load_b32(map_rs, kk * n_out4 + col4, 0, 0);
      } else {
        const int64_t kk = live ? k : K - 1;
        e = map[(kk * n_out + col) & map_mask];
      }
      // an OR rather than a select: the load's value is then always used, and
      // the compiler keeps it unconditional instead of branching around it
      j[u] = (e + ident_row) | (live ? 0 : -1);
    }
    Piece v[SG * NP];
#pragma unroll
    for (int u = 0; u < SG * NP; ++u) {
      if constexpr (B32) {
        // absent rows read past the buffer's end: zeros
        const uint32_t off = j[u] >= 0 ? __umul24(static_cast<uint32_t>(j[u]), nb32.row_bytes) +
                                             ch[u] * static_cast<uint32_t>(sizeof(T))
                                       : 0x80000000u;
        if constexpr (PIECE == 16)
          v[u] = __builtin_bit_cast(Piece, __builtin_amdgcn_raw_buffer_load_b128(feat_rs, off, 0, 0));
        else
          v[u] = __builtin_bit_cast(Piece, __builtin_amdgcn_raw_buffer_load_b64(feat_rs, off, 0, 0));
      } else {
        const Piece* src = j[u] >= 0
                               ? reinterpret_cast<const Piece*>(feat + (int64_t)j[u] * c_in + ch[u])
                               : zero_piece;
        v[u] = *src;
      }
    }
    uint4 b[SG][NT];
#pragma unroll
    for (int u = 0; u < SG; ++u)
#pragma unroll
      for (int n = 0; n < NT; ++n)
        b[u][n] = i0 + u < nsteps ? Wv[((int64_t)(i0 + u) * nt_all + nt0 + n) * 64 + lane]
                                  : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int u = 0; u < SG; ++u) {
      if (i0 + u >= nsteps) break;
      const uint4 a = join_pieces(v[u * NP], v[u * NP + NP - 1]);
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[n] = Op::step(a, b[u][n], acc[n]);
    }
  }

  // D: lane l holds rows 4(l/16) + 0..3 of the wave's 16, column l%16; the
  // output row of wave row r is lane r's oa
  int32_t orow[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = 4 * static_cast<int>(q) + e;
    const int32_t o = __shfl(oa, r, kWave);
    orow[e] = p0 + r < n_out ? o : -1;
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int co = (nt0 + n) * 16 + rl;
    // the batch norm as v * sc + sh, in the order channel_affine computes it
    const float sc = gamma[n] * (1.f / sqrtf(var[n] + ep.eps));
    const float sh = beta[n] - mean[n] * sc;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (orow[e] >= 0)
        out[(int64_t)orow[e] * c_out + co] = from_f32<T>(
            finish(acc[n][e] + bias[n], sc, sh, ep.mean != nullptr, ep.relu != 0));
  }
}

template <typename T, int BN, int CK>
int launch_mfma(const void* feat, int c_in, const void* W, const Epilogue& ep,
                const int32_t* nbr, const int32_t* order, int nbr_ordered, int64_t n_out, int K,
                int c_out, void* out, hipStream_t s) {
  const int64_t items = ceil_div(n_out, kTileRows) * (c_out / BN);
  TSC_REQUIRE(items < (int64_t(1) << 31), "conv: %lld workgroups exceed the grid limit",
              static_cast<long long>(items));
  dim3 grid(static_cast<unsigned>(items));
  // dynamic LDS: the tile's slot lists, later reused to stage the output
  const size_t lds_nbr = (size_t)K * kTileRows * sizeof(int32_t);
  const int row_bytes = BN * (int)sizeof(T);
  const size_t lds_out = (size_t)4 * mfma_stage_rows(row_bytes) * (row_bytes + 16);  // 4 waves
  const size_t lds = lds_nbr > lds_out ? lds_nbr : lds_out;
  conv_mfma_kernel<T, BN, CK><<<grid, 256, lds, s>>>(
      static_cast<const T*>(feat), c_in, static_cast<const T*>(W), ep, nbr, order,
      nbr_ordered, n_out, K, c_out, static_cast<T*>(out));
  TSC_LAUNCH_CHECK("conv_mfma");
  return 0;
}

template <typename T, int BN, int RB>
int launch_dma(const void* feat, int c_in, const void* W, const Epilogue& ep,
               const int32_t* nbr, const int32_t* order, int nbr_ordered, int64_t n_out, int K,
               int c_out, void* out, hipStream_t s) {
  const int64_t items = ceil_div(n_out, 128 * RB) * (c_out / BN);
  TSC_REQUIRE(items < (int64_t(1) << 31), "conv: %lld workgroups exceed the grid limit",
              static_cast<long long>(items));
  constexpr int CK = 128 / (int)sizeof(T);
  TSC_REQUIRE(nbr != nullptr && c_in % CK == 0, "conv: the DMA kernel needs a map and C_in %% %d == 0",
              CK);
  constexpr size_t pool = dma_pool_bytes<T, BN, RB>();
  // more than 64 KB of dynamic LDS for the larger tiles
  if (int rc = allow_dynamic_lds(reinterpret_cast<const void*>(&conv_dma_kernel<T, BN, RB>),
                                 static_cast<int>(pool)))
    return rc;
  conv_dma_kernel<T, BN, RB><<<dim3(static_cast<unsigned>(items)), 256, pool, s>>>(
      static_cast<const T*>(feat), c_in, static_cast<const T*>(W), ep, nbr, order, nbr_ordered,
      n_out, K, c_out, static_cast<T*>(out));
  TSC_LAUNCH_CHECK("conv_dma");
  return 0;
}

template <typename T, int BN, int CK>
int launch_split(const void* feat, int c_in, const void* W, const Epilogue& ep,
                 const int32_t* nbr, const int32_t* order, int nbr_ordered, int64_t n_out, int K,
                 int c_out, void* out, hipStream_t s) {
  const int64_t items = ceil_div(n_out, kSplitRows) * (c_out / BN);
  TSC_REQUIRE(items < (int64_t(1) << 31), "conv: %lld workgroups exceed the grid limit",
              static_cast<long long>(items));
  // dynamic LDS: the tile's map entries, then three waves' partial sums
  const size_t lds = (size_t)K * kSplitRows * sizeof(int32_t) +
                     (size_t)3 * 2 * (BN / 32) * 16 * 64 * sizeof(float);
  conv_split_kernel<T, BN, CK><<<dim3(static_cast<unsigned>(items)), 256, lds, s>>>(
      static_cast<const T*>(feat), c_in, static_cast<const T*>(W), ep, nbr, order,
      nbr_ordered, n_out, K, c_out, static_cast<T*>(out));
  TSC_LAUNCH_CHECK("conv_split");
  return 0;
}

// Which 32x32-tile kernel runs a layer, and with which column tile width.
struct MfmaChoice {
  int bn;      // column tile width
  int ck;      // input-channel chunk of one stage
  bool split;  // the 64-row slot-split kernel instead of the 256-row one
  bool dma;    // the 256-row kernel's direct-to-LDS variant
  int rb;      // its 32-row blocks per wave (tiles of 128 * rb rows)
};

// Layers with fewer 256-row tiles than this run the direct-to-LDS kernel on
// 128-row tiles (32 rows per wave).  On such layers the kernel lasts as long
// as its heaviest tiles' chain of stages (27 slots x the channel chunks, each
// stage's MFMAs shared by the waves on a SIMD); halving a wave's rows halves
// the MFMAs of each stage and, with the smaller LDS pool, lets up to four
// workgroups share a CU.  Measured: the 166k-row 64->64 fp32 strided layer
// (651 tiles) 182 -> 140-152 us, the 32k-row 64->64 fp16 layers 31.4 -> 30.1
// us; the 500k-row 128->128 fp16 layer (1954 tiles) is slower that way, 327
// -> 339 us, where two 64-row waves share each weight slab read from LDS.
constexpr int64_t kShortTiles = 1024;

// Narrower column tiles for small layers: below two workgroups per CU, halve
// BN (each halving doubles the workgroups; gathers repeat per column tile,
// which a small layer can afford).  Layers that would leave more than half
// the CUs without a 256-row workgroup run on 64-row tiles with the slots
// split over the waves (the narrowing has then always reached 32 columns).
// Measured on 64->64 fp16 SubM layers: 9.7k rows (76 workgroups) 28.8 ->
// 20.0 us, but 32k rows (252 workgroups) 30.7 -> 38 us, where the four waves'
// separate weight loads cost more than the shorter slot chain saves.  Short
// slot lists (K < 8) gain nothing from splitting.  column_tile != 0 forces
// the 256-row kernel with that width (every width sums each output in the
// same order, so all give the same bits), always on the register-gather
// kernel.  The 256-row kernel's direct-to-LDS variant serves layers whose
// stages are 128 bytes of each row (f16/bf16 with C_in % 64 == 0, f32 with
// C_in % 32 == 0) and that have a map (K > 1); it sums in the same order too.
MfmaChoice choose_mfma(int dtype, int c_in, int c_out, int K, int64_t n_out, int column_tile) {
  MfmaChoice c{pick_bn(c_out), pick_ck(dtype, c_in), false, false, 2};
  if (column_tile) {
    c.bn = column_tile;
    return c;
  }
  while (c.bn > 32 && ceil_div(n_out, kTileRows) * (c_out / c.bn) < 512) c.bn /= 2;
  c.split = c.bn == 32 && K >= 8 && ceil_div(n_out, kTileRows) * (c_out / c.bn) < 128;
  c.dma = !c.split && K > 1 && c.ck * dtype_bytes(dtype) == 128 && c_in % c.ck == 0;
  if (c.dma && ceil_div(n_out, kTileRows) * (c_out / c.bn) < kShortTiles) c.rb = 1;
  return c;
}

template <typename T>
int dispatch_mfma(const void* feat, int c_in, const void* W, const Epilogue& ep,
                  const int32_t* nbr, const int32_t* order, int nbr_ordered, int64_t n_out, int K,
                  int c_out, int column_tile, void* out, hipStream_t s) {
  constexpr int dt = std::is_same<T, float>::value ? TSC_F32
                     : std::is_same<T, __half>::value ? TSC_F16 : TSC_BF16;
  const MfmaChoice ch = choose_mfma(dt, c_in, c_out, K, n_out, column_tile);
#define TSC_MFMA_CASE(BN_, CK_)                                                              \
  if (ch.bn == BN_ && ch.ck == CK_) {                                                        \
    if constexpr (BN_ == 32)                                                                 \
      if (ch.split)                                                                          \
        return launch_split<T, BN_, CK_>(feat, c_in, W, ep, nbr, order, nbr_ordered, n_out,  \
                                         K, c_out, out, s);                                  \
    if constexpr (CK_ * sizeof(T) == 128)                                                    \
      if (ch.dma)                                                                            \
        return ch.rb == 1 ? launch_dma<T, BN_, 1>(feat, c_in, W, ep, nbr, order, nbr_ordered,  \
                                                  n_out, K, c_out, out, s)                   \
                          : launch_dma<T, BN_, 2>(feat, c_in, W, ep, nbr, order, nbr_ordered,  \
                                                  n_out, K, c_out, out, s);                  \
    return launch_mfma<T, BN_, CK_>(feat, c_in, W, ep, nbr, order, nbr_ordered,          \
                                    n_out, K, c_out, out, s);                                \
  }
  if constexpr (!std::is_same<T, float>::value) {
    TSC_MFMA_CASE(128, 64)
    TSC_MFMA_CASE(64, 64)
    TSC_MFMA_CASE(32, 64)
  }
  TSC_MFMA_CASE(128, 32)
  TSC_MFMA_CASE(64, 32)
  TSC_MFMA_CASE(32, 32)
#undef TSC_MFMA_CASE
  return set_error(TSC_EUNSUPPORTED, "conv: no MFMA tile for c_in=%d c_out=%d", c_in, c_out);
}

template <typename T, int PIECE, int NT>
int launch_narrow(const void* feat, int64_t n_in, int c_in, const void* W, const Epilogue& ep,
                  const int32_t* nbr, const int32_t* order, int nbr_ordered, int64_t n_out, int K,
                  int c_out, void* out, hipStream_t s) {
  constexpr int dt = std::is_same<T, float>::value ? TSC_F32
                     : std::is_same<T, __half>::value ? TSC_F16 : TSC_BF16;
  const int64_t nsteps = narrow_steps(dt, K, c_in);
  TSC_REQUIRE(nsteps < (int64_t(1) << 26), "conv: K * C_in too large");
  dim3 grid(static_cast<unsigned>(ceil_div(n_out, 4 * kNarrowRows)),
            static_cast<unsigned>(c_out / 16 / NT));
  constexpr int elem = static_cast<int>(sizeof(T));
  if (NarrowB32::fits(n_in, c_in, elem, n_out, K, nsteps, 16 / elem)) {
    const NarrowB32 nb32{static_cast<uint32_t>(n_in * c_in * elem),
                         nbr ? static_cast<uint32_t>((int64_t)K * n_out * 4) : 0u,
                         static_cast<uint32_t>(c_in * elem),
                         static_cast<uint32_t>(((uint64_t(1) << 32) + c_in - 1) / c_in)};
    conv_narrow_kernel<T, PIECE, NT, true><<<grid, 256, 0, s>>>(
        static_cast<const T*>(feat), c_in, static_cast<const T*>(W), ep, nbr, order, nbr_ordered,
        n_out, K, c_out, static_cast<int>(nsteps), nb32, static_cast<T*>(out));
  } else {
    conv_narrow_kernel<T, PIECE, NT, false><<<grid, 256, 0, s>>>(
        static_cast<const T*>(feat), c_in, static_cast<const T*>(W), ep, nbr, order, nbr_ordered,
        n_out, K, c_out, static_cast<int>(nsteps), NarrowB32{}, static_cast<T*>(out));
  }
  TSC_LAUNCH_CHECK("conv_narrow");
  return 0;
}

template <typename T>
int dispatch_narrow(const void* feat, int64_t n_in, int c_in, const void* W, const Epilogue& ep,
                    const int32_t* nbr, const int32_t* order, int nbr_ordered, int64_t n_out,
                    int K, int c_out, void* out, hipStream_t s) {
  // Column tiles per wave: up to 4, fewer while that leaves under 2048
  // workgroups (each extra column group re-gathers its rows, from cache).
  const int nt_all = c_out / 16;
  const int64_t blocks = ceil_div(n_out, 4 * kNarrowRows);
  int nt = nt_all % 4 == 0 ? 4 : (nt_all % 2 == 0 ? 2 : 1);
  while (nt > 1 && blocks * (nt_all / nt) < 2048) nt /= 2;
  const int piece = (c_in % 8 == 0 || std::is_same<T, float>::value) ? 16 : 8;
  TSC_REQUIRE((reinterpret_cast<uintptr_t>(feat) & (piece - 1)) == 0 &&
                  (reinterpret_cast<uintptr_t>(W) & 15) == 0,
              "conv: features must be %d-byte and weights 16-byte aligned", piece);
#define TSC_NARROW_CASE(P_, NT_)                                                             \
  if (piece == P_ && nt == NT_)                                                              \
    return launch_narrow<T, P_, NT_>(feat, n_in, c_in, W, ep, nbr, order, nbr_ordered, n_out, K, \
                                     c_out, out, s);
  TSC_NARROW_CASE(16, 1)
  TSC_NARROW_CASE(16, 2)
  TSC_NARROW_CASE(16, 4)
  if constexpr (sizeof(T) == 2) {
    TSC_NARROW_CASE(8, 1)
    TSC_NARROW_CASE(8, 2)
    TSC_NARROW_CASE(8, 4)
  }
#undef TSC_NARROW_CASE
  return set_error(TSC_EUNSUPPORTED, "conv: no narrow tile for c_in=%d c_out=%d", c_in, c_out);
}

template <typename T, int CO>
int launch_valu(const void* feat, int c_in, const void* W, const Epilogue& ep,
                const int32_t* nbr, const int32_t* order, int nbr_ordered, int64_t n_out, int K,
                int c_out, void* out, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(ceil_div(n_out, 256)), static_cast<unsigned>(c_out / CO));
  const int row_bytes = c_in * (int)sizeof(T);
  const uintptr_t a = reinterpret_cast<uintptr_t>(feat);
#define TSC_VALU_LAUNCH(VB_)                                                                  \
  conv_valu_kernel<T, CO, VB_><<<grid, 256, 0, s>>>(static_cast<const T*>(feat), c_in,       \
                                                    static_cast<const float*>(W), ep, nbr,    \
                                                    order, nbr_ordered, n_out, K, c_out,      \
                                                    static_cast<T*>(out))
  if (row_bytes % 16 == 0 && a % 16 == 0)
    TSC_VALU_LAUNCH(16);
  else if (row_bytes % 8 == 0 && a % 8 == 0)
    TSC_VALU_LAUNCH(8);
  else
    TSC_VALU_LAUNCH(sizeof(T));
#undef TSC_VALU_LAUNCH
  TSC_LAUNCH_CHECK("conv_valu");
  return 0;
}

template <typename T>
int dispatch_valu(const void* feat, int c_in, const void* W, const Epilogue& ep,
                  const int32_t* nbr, const int32_t* order, int nbr_ordered, int64_t n_out, int K,
                  int c_out, void* out, hipStream_t s) {
  // Columns per thread: the widest that divides c_out, narrowed for small
  // layers until there are at least 64k threads (a small layer's time is one
  // thread's chain of slots; narrower threads shorten it, and the repeated
  // row loads of the column groups hit in cache).
  int co_max = 32;
  while (co_max > 4 && n_out * (c_out / co_max) < 65536) co_max /= 2;
#define TSC_VALU_CASE(CO_)                                                                   \
  if (CO_ <= co_max && c_out % CO_ == 0)                                                     \
    return launch_valu<T, CO_>(feat, c_in, W, ep, nbr, order, nbr_ordered, n_out, K,        \
                               c_out, out, s);
  TSC_VALU_CASE(32)
  TSC_VALU_CASE(16)
  TSC_VALU_CASE(8)
  TSC_VALU_CASE(4)
  TSC_VALU_CASE(2)
  TSC_VALU_CASE(1)
#undef TSC_VALU_CASE
  return set_error(TSC_EUNSUPPORTED, "conv: unsupported c_out=%d", c_out);
}

}  // namespace
}  // namespace tsc

using namespace tsc;

extern "C" int64_t tsc_packed_weight_bytes(int32_t k_vol, int32_t c_in, int32_t c_out,
                                           int32_t dtype) {
  if (pick_path(dtype, c_in, c_out, k_vol) == kMfma) {
    const int ck = pick_ck(dtype, c_in);
    return (int64_t)k_vol * mfma_chunks(c_in, ck) * ck * c_out * dtype_bytes(dtype);
  }
  if (pick_path(dtype, c_in, c_out, k_vol) == kNarrow)
    return narrow_steps(dtype, k_vol, c_in) * (c_out / 16) * 64 * 16;
  return (int64_t)k_vol * c_in * c_out * 4;
}

extern "C" int tsc_pack_weight(const void* w, int32_t w_dtype, int32_t layout, int32_t k_vol,
                               int32_t c_in, int32_t c_out, int32_t dtype, void* packed,
                               tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(dtype_ok(dtype) && dtype_ok(w_dtype), "pack: unsupported dtype");
  TSC_REQUIRE(layout == 0 || layout == 1, "pack: layout must be 0 (KRSC) or 1 (flat)");
  TSC_REQUIRE(k_vol > 0 && c_in > 0 && c_out > 0, "pack: sizes must be positive");
  TSC_REQUIRE(w && packed, "pack: null pointer");
  const int64_t total = (int64_t)k_vol * (c_in + 32) * c_out;  // covers a padded chunk or step
  const int grid = static_cast<int>(ceil_div(total, 256) < 2048 ? ceil_div(total, 256) : 2048);
  const Path path = pick_path(dtype, c_in, c_out, k_vol);
  if (path == kNarrow) {
    const int64_t nsteps = narrow_steps(dtype, k_vol, c_in);
    if (dtype == TSC_F32)
      pack_narrow_kernel<float><<<grid, 256, 0, s>>>(w, w_dtype, layout, k_vol, c_in, c_out,
                                                     nsteps, static_cast<float*>(packed));
    else if (dtype == TSC_F16)
      pack_narrow_kernel<__half><<<grid, 256, 0, s>>>(w, w_dtype, layout, k_vol, c_in, c_out,
                                                      nsteps, static_cast<__half*>(packed));
    else
      pack_narrow_kernel<__hip_bfloat16><<<grid, 256, 0, s>>>(
          w, w_dtype, layout, k_vol, c_in, c_out, nsteps, static_cast<__hip_bfloat16*>(packed));
  } else if (path == kMfma) {
    const int ck = pick_ck(dtype, c_in);
    if (dtype == TSC_F32)
      pack_mfma_kernel<float><<<grid, 256, 0, s>>>(w, w_dtype, layout, k_vol, c_in, c_out, ck,
                                                   static_cast<float*>(packed));
    else if (dtype == TSC_F16)
      pack_mfma_kernel<__half><<<grid, 256, 0, s>>>(w, w_dtype, layout, k_vol, c_in, c_out, ck,
                                                    static_cast<__half*>(packed));
    else
      pack_mfma_kernel<__hip_bfloat16><<<grid, 256, 0, s>>>(
          w, w_dtype, layout, k_vol, c_in, c_out, ck, static_cast<__hip_bfloat16*>(packed));
  } else {
    pack_valu_kernel<<<grid, 256, 0, s>>>(w, w_dtype, layout, k_vol, c_in, c_out,
                                          static_cast<float*>(packed));
  }
  TSC_LAUNCH_CHECK("pack_weight");
  return 0;
}

static int conv_forward(const void* feat, int32_t dtype, int64_t n_in, int32_t c_in,
                        const void* packed_w, const Epilogue& ep, const int32_t* nbr,
                        const int32_t* order, int32_t nbr_ordered, int64_t n_out, int32_t k_vol,
                        int32_t c_out, int32_t column_tile, void* out, hipStream_t s) {
  TSC_REQUIRE(dtype_ok(dtype), "conv: unsupported dtype %d", dtype);
  TSC_REQUIRE(!ep.bias || dtype_ok(ep.bias_dt), "conv: unsupported bias dtype %d", ep.bias_dt);
  TSC_REQUIRE((ep.mean == nullptr) == (ep.var == nullptr),
              "conv: batch-norm mean and variance come together");
  TSC_REQUIRE(ep.mean || (!ep.gamma && !ep.beta),
              "conv: batch-norm weight or bias without running statistics");
  TSC_REQUIRE(!ep.mean || dtype_ok(ep.bn_dt), "conv: unsupported batch-norm dtype %d", ep.bn_dt);
  TSC_REQUIRE(!ep.mean || ep.eps >= 0.f, "conv: batch-norm eps must be non-negative");
  TSC_REQUIRE(c_in > 0 && c_out > 0 && k_vol > 0, "conv: sizes must be positive");
  TSC_REQUIRE(n_out >= 0 && n_out < (int64_t(1) << 31) && n_in >= 0 && n_in < (int64_t(1) << 31),
              "conv: row counts out of range");
  TSC_REQUIRE(nbr || k_vol == 1, "conv: identity map needs k_vol == 1");
  TSC_REQUIRE(nbr || n_in >= n_out, "conv: identity map needs n_in >= n_out");
  TSC_REQUIRE(!nbr_ordered || (order && nbr), "conv: an ordered map needs its order");
  TSC_REQUIRE(nbr_ordered >= 0 && nbr_ordered <= 2, "conv: nbr_ordered must be 0, 1 or 2");
  TSC_REQUIRE(nbr_ordered != 2 || k_vol <= 32,
              "conv: a map with its slot-mask row (nbr_ordered = 2) needs k_vol <= 32");
  const Path path = pick_path(dtype, c_in, c_out, k_vol);
  TSC_REQUIRE(column_tile == 0 || (path == kMfma && (column_tile == 32 || column_tile == 64 ||
                                                     column_tile == 128) &&
                                   c_out % column_tile == 0),
              "conv: %d is not a column tile width of this layer (32, 64 or 128 dividing "
              "c_out=%d, on a 32x32-tile layer)", column_tile, c_out);
  if (n_out == 0) return 0;
  TSC_REQUIRE(packed_w && out && (feat || n_in == 0), "conv: null pointer");
  if (n_in == 0) {
    // no inputs: every output is the epilogue of zero
    TSC_REQUIRE(nbr != nullptr, "conv: empty input");
  }
  if (path == kMfma) {
    TSC_REQUIRE((reinterpret_cast<uintptr_t>(feat) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(packed_w) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & 15) == 0,
                "conv: feature, weight and output buffers must be 16-byte aligned");
    if (dtype == TSC_F32)
      return dispatch_mfma<float>(feat, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out, k_vol,
                                  c_out, column_tile, out, s);
    if (dtype == TSC_F16)
      return dispatch_mfma<__half>(feat, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out, k_vol,
                                   c_out, column_tile, out, s);
    return dispatch_mfma<__hip_bfloat16>(feat, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out,
                                         k_vol, c_out, column_tile, out, s);
  }
  if (path == kNarrow) {
    if (dtype == TSC_F32)
      return dispatch_narrow<float>(feat, n_in, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out,
                                    k_vol, c_out, out, s);
    if (dtype == TSC_F16)
      return dispatch_narrow<__half>(feat, n_in, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out,
                                     k_vol, c_out, out, s);
    return dispatch_narrow<__hip_bfloat16>(feat, n_in, c_in, packed_w, ep, nbr, order, nbr_ordered,
                                           n_out, k_vol, c_out, out, s);
  }
  if (dtype == TSC_F32)
    return dispatch_valu<float>(feat, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out, k_vol,
                                c_out, out, s);
  if (dtype == TSC_F16)
    return dispatch_valu<__half>(feat, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out, k_vol,
                                 c_out, out, s);
  return dispatch_valu<__hip_bfloat16>(feat, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out,
                                       k_vol, c_out, out, s);
}

extern "C" int tsc_conv_forward(const void* feat, int32_t dtype, int64_t n_in, int32_t c_in,
                                const void* packed_w, const void* bias, int32_t bias_dtype,
                                const int32_t* nbr, const int32_t* order, int32_t nbr_ordered,
                                int64_t n_out, int32_t k_vol, int32_t c_out, void* out,
                                tsc_stream_t stream) {
  const Epilogue ep{bias, bias_dtype, nullptr, nullptr, nullptr, nullptr, 0, 0.f, 0};
  return conv_forward(feat, dtype, n_in, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out, k_vol,
                      c_out, 0, out, static_cast<hipStream_t>(stream));
}

extern "C" int tsc_conv_forward_ep(const void* feat, int32_t dtype, int64_t n_in, int32_t c_in,
                                   const void* packed_w, const void* bias, int32_t bias_dtype,
                                   const void* bn_mean, const void* bn_var,
                                   const void* bn_weight, const void* bn_bias, int32_t bn_dtype,
                                   float bn_eps, int32_t relu, const int32_t* nbr,
                                   const int32_t* order, int32_t nbr_ordered, int64_t n_out,
                                   int32_t k_vol, int32_t c_out, void* out, tsc_stream_t stream) {
  const Epilogue ep{bias,      bias_dtype, bn_mean, bn_var, bn_weight,
                    bn_bias,   bn_dtype,   bn_eps,  relu != 0 ? 1 : 0};
  return conv_forward(feat, dtype, n_in, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out, k_vol,
                      c_out, 0, out, static_cast<hipStream_t>(stream));
}

extern "C" int tsc_conv_forward_tile(const void* feat, int32_t dtype, int64_t n_in, int32_t c_in,
                                     const void* packed_w, const void* bias, int32_t bias_dtype,
                                     const int32_t* nbr, const int32_t* order,
                                     int32_t nbr_ordered, int64_t n_out, int32_t k_vol,
                                     int32_t c_out, int32_t column_tile, void* out,
                                     tsc_stream_t stream) {
  const Epilogue ep{bias, bias_dtype, nullptr, nullptr, nullptr, nullptr, 0, 0.f, 0};
  return conv_forward(feat, dtype, n_in, c_in, packed_w, ep, nbr, order, nbr_ordered, n_out, k_vol,
                      c_out, column_tile, out, static_cast<hipStream_t>(stream));
}

extern "C" const char* tsc_conv_kernel_name(int32_t dtype, int32_t c_in, int32_t c_out,
                                            int32_t k_vol, int64_t n_out) {
  if (!dtype_ok(dtype) || c_in <= 0 || c_out <= 0 || k_vol <= 0 || n_out < 0) return "";
  switch (pick_path(dtype, c_in, c_out, k_vol)) {
    case kMfma: {
      const MfmaChoice ch = choose_mfma(dtype, c_in, c_out, k_vol, n_out, 0);
      return ch.split ? "conv_split_kernel" : ch.dma ? "conv_dma_kernel" : "conv_mfma_kernel";
    }
    case kNarrow:
      return "conv_narrow_kernel";
    default:
      return "conv_valu_kernel";
  }
}
