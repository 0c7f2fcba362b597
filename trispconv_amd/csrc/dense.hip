// Sparse -> dense scatter (SparseConvTensor.dense()).
//
// Reference: trispconv/pytorch/tensor.py:72-99 builds a zero (B, D, H, W, C)
// tensor, asserts every coordinate is in range, assigns dense[b, z, y, x] =
// features, and for channels_first returns permute(0, 4, 1, 2, 3).contiguous()
// — three passes over the dense volume (zero, scatter, transposing copy).
//
// MI355X design: the output is written once in its final layout.  A fill
// kernel clears it with 16-byte stores; the scatter then writes each row's C
// values: contiguously for (B, D, H, W, C), at stride D*H*W for (B, C, D, H,
// W), with consecutive lanes on consecutive channels of one row so a wave's
// stores for channels-last are one contiguous run.  Rows with a coordinate
// outside [0,B) x [0,D) x [0,H) x [0,W) are not written and set a status flag
// (the host raises, as the reference's asserts do).  Repeated coordinates:
// each element holds one of the rows' values, as with the reference's
// index_put on the GPU, where the winner is unspecified.
#include "common.hpp"

#include <algorithm>

namespace tsc {
namespace {

__global__ void __launch_bounds__(256) zero_kernel(uint4* __restrict__ p, int64_t n16,
                                                   uint8_t* __restrict__ tail, int tail_bytes) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16; i += stride)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
  if (blockIdx.x == 0 && threadIdx.x < tail_bytes) tail[threadIdx.x] = 0;
}

// One thread per (row, channel), channel fastest; E is a raw element of the
// features' size (1, 2, 4 or 8 bytes: every dtype the features may have).
template <typename E>
__global__ void __launch_bounds__(256) scatter_kernel(const E* __restrict__ feat,
                                                      const int4* __restrict__ coords, int64_t n,
                                                      int C, int B, int D, int H, int W,
                                                      int channels_first, E* __restrict__ out,
                                                      int32_t* __restrict__ status) {
  const int64_t total = n * C;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t vol = (int64_t)D * H * W;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += stride) {
    const int64_t r = e / C;
    const int c = static_cast<int>(e - r * C);
    const int4 q = coords[r];  // (b, z, y, x)
    if (q.x < 0 || q.x >= B || q.y < 0 || q.y >= D || q.z < 0 || q.z >= H || q.w < 0 ||
        q.w >= W) {
      if (c == 0) atomicOr(status, 1);
      continue;
    }
    const int64_t cell = ((int64_t)q.y * H + q.z) * W + q.w;  // inside one sample
    const int64_t dst = channels_first ? ((int64_t)q.x * C + c) * vol + cell
                                       : ((int64_t)q.x * vol + cell) * C + c;
    out[dst] = feat[e];
  }
}

}  // namespace
}  // namespace tsc

using namespace tsc;

extern "C" int tsc_dense_scatter(const void* feat, int32_t elem_bytes, int64_t n, int32_t c,
                                 const int32_t* coords, int32_t batch_size,
                                 const int32_t spatial[3], int32_t channels_first, void* out,
                                 int32_t* status, tsc_stream_t stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  TSC_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
              "dense: element size must be 1, 2, 4 or 8 bytes");
  TSC_REQUIRE(n >= 0 && c > 0 && batch_size > 0 && spatial, "dense: invalid sizes");
  TSC_REQUIRE(spatial[0] > 0 && spatial[1] > 0 && spatial[2] > 0, "dense: spatial shape must be positive");
  TSC_REQUIRE(out && status, "dense: null pointer");
  const int64_t elems = (int64_t)batch_size * spatial[0] * spatial[1] * spatial[2] * c;
  const int64_t bytes = elems * elem_bytes;
  TSC_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15) == 0, "dense: output must be 16-byte aligned");
  int rc = fill_u32(reinterpret_cast<uint32_t*>(status), 1, 0u, s);
  if (rc) return rc;
  const int64_t n16 = bytes / 16;
  const int tail = static_cast<int>(bytes - n16 * 16);
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(n16, 256), 8192));
  zero_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(
      static_cast<uint4*>(out), n16, static_cast<uint8_t*>(out) + n16 * 16, tail);
  TSC_LAUNCH_CHECK("dense_zero");
  if (n == 0) return 0;
  TSC_REQUIRE(feat && coords, "dense: null pointer");
  const int64_t work = n * c;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(work, 256), 65536));
  const int4* c4 = reinterpret_cast<const int4*>(coords);
  // the values are moved as raw elements of their size: any dtype of that size
  auto launch = [&](auto tag) {
    using E = decltype(tag);
    scatter_kernel<E><<<grid, 256, 0, s>>>(static_cast<const E*>(feat), c4, n, c, batch_size,
                                           spatial[0], spatial[1], spatial[2], channels_first,
                                           static_cast<E*>(out), status);
  };
  switch (elem_bytes) {
    case 1: launch(uint8_t{}); break;
    case 2: launch(uint16_t{}); break;
    case 4: launch(uint32_t{}); break;
    default: launch(uint64_t{}); break;
  }
  TSC_LAUNCH_CHECK("dense_scatter");
  return 0;
}
