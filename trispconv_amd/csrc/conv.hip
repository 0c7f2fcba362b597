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
// Two code shapes share that structure:
//   * mfma: f16/bf16 with C_in, C_out multiples of 32 and K <= 64 —
//     v_mfma_f32_32x32x16_{f16,bf16}, 4 waves x (64 rows x BN cols) per tile.
//   * valu: everything else (narrow or ragged channels, fp32) — one output row
//     per lane and CO columns per thread, weights read with wave-uniform
//     addresses, slots skipped when no lane of the wave needs them.
#include "common.hpp"

namespace tsc {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum Path { kValu = 0, kMfma16 = 1 };

// 64-channel chunks keep accumulators plus double-buffered operands within
// 256 registers, so two workgroups (8 waves) share a CU.
int pick_ck(int c_in) { return c_in % 64 == 0 ? 64 : 32; }
int pick_bn(int c_out) { return c_out % 128 == 0 ? 128 : (c_out % 64 == 0 ? 64 : 32); }

Path pick_path(int dtype, int c_in, int c_out, int K) {
  if ((dtype == TSC_F16 || dtype == TSC_BF16) && c_in % 32 == 0 && c_out % 32 == 0 && K <= 64)
    return kMfma16;
  return kValu;
}

// ----------------------------------------------------------- weight pack --
__device__ __forceinline__ float load_any(const void* p, int dt, int64_t i) {
  if (dt == TSC_F32) return static_cast<const float*>(p)[i];
  if (dt == TSC_F16) return __half2float(static_cast<const __half*>(p)[i]);
  return __bfloat162float(static_cast<const __hip_bfloat16*>(p)[i]);
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

// MFMA layout: [k][chunk][c_out/32][step][lane][8].  At step s of a CK-wide
// input-channel chunk, lane l supplies B[kk][n] for n = l % 32 and
// kk = (l / 32) * CK/2 + s*8 + 0..7 — the same channel split the A operand
// uses, so that each lane's A data is a contiguous CK/2-channel run of a row.
template <typename T>
__global__ void pack_mfma_kernel(const void* w, int w_dt, int layout, int K, int c_in, int c_out,
                                 int ck, T* packed) {
  const int steps = ck / 16;
  const int nbt = c_out / 32;
  const int nch = c_in / ck;
  const int64_t total = (int64_t)K * c_in * c_out;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int i = e & 7;
    const int lane = (e >> 3) & 63;
    int64_t r = e >> 9;
    const int s = r % steps;
    r /= steps;
    const int nb = r % nbt;
    r /= nbt;
    const int c = r % nch;
    const int k = r / nch;
    const int ci = c * ck + (lane >> 5) * (ck / 2) + s * 8 + i;
    const int co = nb * 32 + (lane & 31);
    packed[e] = from_f32<T>(src_weight(w, w_dt, layout, K, c_in, c_out, k, ci, co));
  }
}

// ---------------------------------------------------------------- VALU --
template <typename T, int CO>
__global__ void __launch_bounds__(256) conv_valu_kernel(
    const T* __restrict__ feat, int c_in, const float* __restrict__ W, const void* bias, int bias_dt,
    const int32_t* __restrict__ nbr, const int32_t* __restrict__ order, int64_t n_out, int K,
    int c_out, T* __restrict__ out) {
  const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  const int co0 = blockIdx.y * CO;
  const bool valid = t < n_out;
  const int64_t o = valid ? (order ? order[t] : t) : 0;
  float acc[CO];
#pragma unroll
  for (int c = 0; c < CO; ++c) acc[c] = 0.f;
  for (int k = 0; k < K; ++k) {
    const int32_t j = valid ? (nbr ? nbr[(int64_t)k * n_out + o] : static_cast<int32_t>(o)) : -1;
    if (__ballot(j >= 0) == 0ull) continue;  // no lane of the wave uses slot k
    const T* x = feat + (int64_t)(j >= 0 ? j : 0) * c_in;
    const float* wk = W + (int64_t)k * c_in * c_out + co0;
    for (int ci = 0; ci < c_in; ++ci) {
      const float xv = j >= 0 ? to_f32<T>(x[ci]) : 0.f;
      const float* wr = wk + (int64_t)ci * c_out;
#pragma unroll
      for (int c = 0; c < CO; ++c) acc[c] = fmaf(xv, wr[c], acc[c]);
    }
  }
  if (!valid) return;
  T* dst = out + o * c_out + co0;
#pragma unroll
  for (int c = 0; c < CO; ++c) {
    const float b = bias ? load_any(bias, bias_dt, co0 + c) : 0.f;
    dst[c] = from_f32<T>(acc[c] + b);
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

constexpr int kTileRows = 256;  // 4 waves x 64 rows

// 16 bytes per lane, global memory -> LDS without passing through registers
// (global_load_lds_dwordx4): lane l of the wave writes lds_base + 16*l.  The
// builtin exists only for the device; the host pass sees an empty body.
__device__ __forceinline__ void copy16_to_lds(const uint4* src, uint4* lds_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, lds_base, 16, 0, 0);
#else
  (void)src;
  (void)lds_base;
#endif
}

// Operand source for absent neighbours: lanes whose output row has no input
// through the current slot read zeros from here instead of branching around
// their loads (64 bytes per lane are read at most).
__device__ __attribute__((aligned(256))) uint4 g_zero_row[16];
// s_waitcnt immediate for "vmcnt(0)", leaving expcnt / lgkmcnt unconstrained
constexpr int kWaitVmcnt0 = (0x7 << 4) | (0xf << 8);

template <typename T, int BN, int CK>
__global__ void __launch_bounds__(256, 2) conv_mfma_kernel(
    const T* __restrict__ feat, int c_in, const T* __restrict__ W, const void* bias, int bias_dt,
    const int32_t* __restrict__ nbr, const int32_t* __restrict__ order, int64_t n_out, int K,
    int c_out, T* __restrict__ out) {
  using Op = MfmaOp<T>;
  using V = typename Op::V;
  constexpr int STEPS = CK / 16;                 // 16-deep MFMA steps per chunk
  constexpr int NB = BN / 32;                    // 32-wide column blocks
  constexpr int SLAB_VECS = BN * CK / 8;         // 16-byte vectors of one weight stage
  constexpr int WV = SLAB_VECS >= 256 ? SLAB_VECS / 256 : 1;
  constexpr bool FULL = SLAB_VECS % 256 == 0;
  static_assert(!FULL || SLAB_VECS / 256 == WV, "slab split");

  __shared__ __attribute__((aligned(16))) uint4 s_w[2][SLAB_VECS];
  __shared__ __attribute__((aligned(16))) int32_t s_orow[kTileRows];
  __shared__ uint32_t s_mask[8];      // per 32-row block
  extern __shared__ int32_t s_nbr[];  // [K][kTileRows]

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int h = lane >> 5;
  // XCD-aware placement: workgroups are dispatched round-robin over the 8
  // XCDs, so give XCD x a contiguous run of (tile, column tile) items; all
  // column tiles of a row tile, and neighbouring row tiles of the execution
  // order, then share that XCD's L2.
  const int ncol = c_out / BN;
  int64_t item;
  {
    const int64_t nwg = gridDim.x, lin = blockIdx.x;
    const int64_t per = nwg / 8, rem = nwg % 8, x = lin % 8;
    item = x * per + (x < rem ? x : rem) + lin / 8;
  }
  const int64_t tile0 = (item / ncol) * kTileRows;
  const int nbt = static_cast<int>(item % ncol);
  const int nch = c_in / CK;

  // ---- tile set-up: output rows, their slot lists and slot masks
  {
    const int64_t tr = tile0 + t;
    const int32_t orow = tr < n_out ? (order ? order[tr] : static_cast<int32_t>(tr)) : -1;
    s_orow[t] = orow;
    uint32_t m = 0;
    for (int k = 0; k < K; ++k) {
      int32_t j = -1;
      if (orow >= 0) j = nbr ? nbr[(int64_t)k * n_out + orow] : orow;
      s_nbr[k * kTileRows + t] = j;
      m |= (j >= 0 ? 1u : 0u) << (k & 31);
    }
    // OR over each 32-row half-wave: the rows one MFMA row block covers
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) m |= __shfl_xor(m, off, kWave);
    if ((lane & 31) == 0) s_mask[wave * 2 + h] = m;
  }
  __syncthreads();
  uint32_t umask = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) umask |= s_mask[i];
  const uint32_t bmask0 = s_mask[wave * 2], bmask1 = s_mask[wave * 2 + 1];
  const int r0 = wave * 64 + (lane & 31);  // tile rows of this lane's A operands
  const int r1 = r0 + 32;

  auto next_k = [&](int k) {
    for (++k; k < K; ++k)
      if (umask & (1u << (k & 31))) return k;
    return K;
  };

  const uint4* Wv = reinterpret_cast<const uint4*>(W);
  const int nbt_all = c_out / 32;

  f32x16 acc[2][NB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[rb][nb][i] = 0.f;

  uint4 a_cur[2][STEPS], a_nxt[2][STEPS];

// Weight slab of stage (KK, CC) -> s_w[BUF], straight from global memory
// into LDS (global_load_lds_dwordx4: lane l of a wave lands at base + 16*l).
#define TSC_LOAD_W(KK, CC, BUF)                                                               \
  {                                                                                           \
    const uint4* src_ =                                                                       \
        Wv + (((int64_t)(KK) * nch + (CC)) * nbt_all + (int64_t)nbt * NB) * STEPS * 64;        \
    _Pragma("unroll") for (int v = 0; v < WV; ++v) {                                          \
      if (FULL || v * 256 + t < SLAB_VECS)                                                    \
        copy16_to_lds(src_ + v * 256 + t, &s_w[BUF][v * 256 + wave * 64]);                    \
    }                                                                                         \
  }
#define TSC_LOAD_A(DST, KK, CC)                                                               \
  {                                                                                           \
    const int32_t j0_ = s_nbr[(KK) * kTileRows + r0];                                         \
    const int32_t j1_ = s_nbr[(KK) * kTileRows + r1];                                         \
    const int coff_ = (CC) * CK + h * (CK / 2);                                               \
    const uint4* p0_ = j0_ >= 0 ? reinterpret_cast<const uint4*>(feat + (int64_t)j0_ * c_in + coff_) \
                                : g_zero_row;                                                  \
    const uint4* p1_ = j1_ >= 0 ? reinterpret_cast<const uint4*>(feat + (int64_t)j1_ * c_in + coff_) \
                                : g_zero_row;                                                  \
    _Pragma("unroll") for (int s_ = 0; s_ < STEPS; ++s_) {                                    \
      DST[0][s_] = p0_[s_];                                                                   \
      DST[1][s_] = p1_[s_];                                                                   \
    }                                                                                         \
  }

  int k = (umask & 1u) ? 0 : next_k(0);
  int c = 0;
  int buf = 0;
  if (k < K) {
    TSC_LOAD_W(k, c, 0);
    TSC_LOAD_A(a_cur, k, c);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  while (k < K) {
    int kn = k, cn = c + 1;
    if (cn == nch) {
      cn = 0;
      kn = next_k(k);
    }
    const bool more = kn < K;
    // gathers for the next stage go out before this stage's MFMAs; the weight
    // slab copy (global -> LDS) is issued after them so that no LDS write is
    // in flight while the MFMA operands are read from LDS
    if (more) TSC_LOAD_A(a_nxt, kn, cn);
    // a 32-row block with no input through slot k skips its MFMAs (its
    // operands are zero and would add exact zeros)
    const uint32_t kbit = 1u << (k & 31);
    const bool use0 = (bmask0 & kbit) != 0, use1 = (bmask1 & kbit) != 0;
    if (use0 || use1) {
      const uint4* sw = s_w[buf];
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        const V a0 = __builtin_bit_cast(V, a_cur[0][s]);
        const V a1 = __builtin_bit_cast(V, a_cur[1][s]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const V b = __builtin_bit_cast(V, sw[(nb * STEPS + s) * 64 + lane]);
          if (use0) acc[0][nb] = Op::run(a0, b, acc[0][nb]);
          if (use1) acc[1][nb] = Op::run(a1, b, acc[1][nb]);
        }
      }
    }
    if (more) TSC_LOAD_W(kn, cn, buf ^ 1);
    // the next stage's weight slab (and operands) must have landed before any
    // wave reads it
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int s = 0; s < STEPS; ++s) a_cur[rb][s] = a_nxt[rb][s];
    buf ^= 1;
    k = kn;
    c = cn;
  }
#undef TSC_LOAD_W
#undef TSC_LOAD_A

  // ---- epilogue: + bias, round once, store each output element once.
  // 32x32 accumulator layout: register i of lane l holds row
  // (i/4)*8 + (l/32)*4 + i%4 and column l%32 of the block.
  int4 orows[2][4];  // rows (rb, g): 4 consecutive rows starting at wave*64 + rb*32 + g*8 + h*4
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      orows[rb][g] = *reinterpret_cast<const int4*>(&s_orow[wave * 64 + rb * 32 + g * 8 + h * 4]);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = nbt * BN + nb * 32 + (lane & 31);
    const float bv = bias ? load_any(bias, bias_dt, col) : 0.f;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int4 q = orows[rb][i >> 2];
        const int32_t orow = (i & 3) == 0 ? q.x : (i & 3) == 1 ? q.y : (i & 3) == 2 ? q.z : q.w;
        if (orow >= 0) out[(int64_t)orow * c_out + col] = from_f32<T>(acc[rb][nb][i] + bv);
      }
    }
  }
}

template <typename T, int BN, int CK>
int launch_mfma(const void* feat, int c_in, const void* W, const void* bias, int bias_dt,
                const int32_t* nbr, const int32_t* order, int64_t n_out, int K, int c_out,
                void* out, hipStream_t s) {
  const int64_t items = ceil_div(n_out, kTileRows) * (c_out / BN);
  dim3 grid(static_cast<unsigned>(items));
  const size_t lds = (size_t)K * kTileRows * sizeof(int32_t);
  conv_mfma_kernel<T, BN, CK><<<grid, 256, lds, s>>>(
      static_cast<const T*>(feat), c_in, static_cast<const T*>(W), bias, bias_dt, nbr, order, n_out,
      K, c_out, static_cast<T*>(out));
  TSC_LAUNCH_CHECK("conv_mfma");
  return 0;
}

template <typename T>
int dispatch_mfma(const void* feat, int c_in, const void* W, const void* bias, int bias_dt,
                  const int32_t* nbr, const int32_t* order, int64_t n_out, int K, int c_out,
                  void* out, hipStream_t s) {
  const int bn = pick_bn(c_out), ck = pick_ck(c_in);
#define TSC_MFMA_CASE(BN_, CK_)                                                              \
  if (bn == BN_ && ck == CK_)                                                                \
    return launch_mfma<T, BN_, CK_>(feat, c_in, W, bias, bias_dt, nbr, order, n_out, K, c_out, \
                                    out, s);
  TSC_MFMA_CASE(128, 64)
  TSC_MFMA_CASE(128, 32)
  TSC_MFMA_CASE(64, 64)
  TSC_MFMA_CASE(64, 32)
  TSC_MFMA_CASE(32, 64)
  TSC_MFMA_CASE(32, 32)
#undef TSC_MFMA_CASE
  return set_error(TSC_EUNSUPPORTED, "conv: no MFMA tile for c_in=%d c_out=%d", c_in, c_out);
}

template <typename T, int CO>
int launch_valu(const void* feat, int c_in, const void* W, const void* bias, int bias_dt,
                const int32_t* nbr, const int32_t* order, int64_t n_out, int K, int c_out,
                void* out, hipStream_t s) {
  dim3 grid(static_cast<unsigned>(ceil_div(n_out, 256)), static_cast<unsigned>(c_out / CO));
  conv_valu_kernel<T, CO><<<grid, 256, 0, s>>>(static_cast<const T*>(feat), c_in,
                                               static_cast<const float*>(W), bias, bias_dt, nbr,
                                               order, n_out, K, c_out, static_cast<T*>(out));
  TSC_LAUNCH_CHECK("conv_valu");
  return 0;
}

template <typename T>
int dispatch_valu(const void* feat, int c_in, const void* W, const void* bias, int bias_dt,
                  const int32_t* nbr, const int32_t* order, int64_t n_out, int K, int c_out,
                  void* out, hipStream_t s) {
#define TSC_VALU_CASE(CO_)                                                                   \
  if (c_out % CO_ == 0)                                                                      \
    return launch_valu<T, CO_>(feat, c_in, W, bias, bias_dt, nbr, order, n_out, K, c_out, out, \
                               s);
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
  const int64_t elems = (int64_t)k_vol * c_in * c_out;
  return pick_path(dtype, c_in, c_out, k_vol) == kMfma16 ? elems * 2 : elems * 4;
}

extern "C" int tsc_pack_weight(const void* w, int32_t w_dtype, int32_t layout, int32_t k_vol,
                               int32_t c_in, int32_t c_out, int32_t dtype, void* packed,
                               tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(dtype_ok(dtype) && dtype_ok(w_dtype), "pack: unsupported dtype");
  TSC_REQUIRE(layout == 0 || layout == 1, "pack: layout must be 0 (KRSC) or 1 (flat)");
  TSC_REQUIRE(k_vol > 0 && c_in > 0 && c_out > 0, "pack: sizes must be positive");
  TSC_REQUIRE(w && packed, "pack: null pointer");
  const int64_t total = (int64_t)k_vol * c_in * c_out;
  const int grid = static_cast<int>(ceil_div(total, 256) < 2048 ? ceil_div(total, 256) : 2048);
  if (pick_path(dtype, c_in, c_out, k_vol) == kMfma16) {
    const int ck = pick_ck(c_in);
    if (dtype == TSC_F16)
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

extern "C" int tsc_conv_forward(const void* feat, int32_t dtype, int64_t n_in, int32_t c_in,
                                const void* packed_w, const void* bias, int32_t bias_dtype,
                                const int32_t* nbr, const int32_t* order, int64_t n_out,
                                int32_t k_vol, int32_t c_out, void* out, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(dtype_ok(dtype), "conv: unsupported dtype %d", dtype);
  TSC_REQUIRE(!bias || dtype_ok(bias_dtype), "conv: unsupported bias dtype %d", bias_dtype);
  TSC_REQUIRE(c_in > 0 && c_out > 0 && k_vol > 0, "conv: sizes must be positive");
  TSC_REQUIRE(n_out >= 0 && n_out < (int64_t(1) << 31) && n_in >= 0 && n_in < (int64_t(1) << 31),
              "conv: row counts out of range");
  TSC_REQUIRE(nbr || k_vol == 1, "conv: identity map needs k_vol == 1");
  TSC_REQUIRE(nbr || n_in >= n_out, "conv: identity map needs n_in >= n_out");
  if (n_out == 0) return 0;
  TSC_REQUIRE(packed_w && out && (feat || n_in == 0), "conv: null pointer");
  if (n_in == 0) {
    // no inputs: every output is the bias alone
    TSC_REQUIRE(nbr != nullptr, "conv: empty input");
  }
  const Path path = pick_path(dtype, c_in, c_out, k_vol);
  if (path == kMfma16) {
    TSC_REQUIRE((reinterpret_cast<uintptr_t>(feat) & 15) == 0 &&
                    (reinterpret_cast<uintptr_t>(packed_w) & 15) == 0,
                "conv: feature and weight buffers must be 16-byte aligned");
    if (dtype == TSC_F16)
      return dispatch_mfma<__half>(feat, c_in, packed_w, bias, bias_dtype, nbr, order, n_out,
                                   k_vol, c_out, out, s);
    return dispatch_mfma<__hip_bfloat16>(feat, c_in, packed_w, bias, bias_dtype, nbr, order,
                                         n_out, k_vol, c_out, out, s);
  }
  if (dtype == TSC_F32)
    return dispatch_valu<float>(feat, c_in, packed_w, bias, bias_dtype, nbr, order, n_out, k_vol,
                                c_out, out, s);
  if (dtype == TSC_F16)
    return dispatch_valu<__half>(feat, c_in, packed_w, bias, bias_dtype, nbr, order, n_out, k_vol,
                                 c_out, out, s);
  return dispatch_valu<__hip_bfloat16>(feat, c_in, packed_w, bias, bias_dtype, nbr, order, n_out,
                                       k_vol, c_out, out, s);
}
