// HBM read ceiling of one launch (a measurement kernel for the roofline, not
// part of the decode path): reads a set of equally long rows once, as 16-byte
// loads, and folds them into one word per workgroup so that no load is dead.
//
// Row r starts at base + (r % inner) * inner_stride + (r / inner) * outer_stride
// (bytes).  One KV head's rows of a layer [P, 2, page, Hkv, D] are inner =
// P * 2 * page rows of D * 2 bytes at a stride of Hkv * D * 2 bytes, the heads
// outer_stride = D * 2 apart: the access pattern of the decode kernels, which
// read one KV head's 256-byte rows per tile.  inner = rows gives a plain
// contiguous read when row_bytes = inner_stride.
//
// A workgroup takes groups of kProbeThreads * kProbeUnroll chunks (whole rows:
// the chunks per row are a power of two no larger than that), issues all of a
// thread's kProbeUnroll loads before it consumes any, and locates a group's
// first row with one division; the rows after it advance the (outer, inner)
// pair by carries.

#include "common.h"

namespace be {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;
constexpr int kProbeGroupChunks = kProbeThreads * kProbeUnroll;

__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const char* base, int64_t rows, int64_t inner,
                                                                   int64_t inner_stride, int64_t outer_stride,
                                                                   int chunks_log2, uint32_t* sink) {
  const int64_t group_rows = kProbeGroupChunks >> chunks_log2;
  const int64_t groups = (rows + group_rows - 1) / group_rows;
  const int cmask = (1 << chunks_log2) - 1;
  uint32_t acc = 0;
  for (int64_t g = blockIdx.x; g < groups; g += gridDim.x) {
    const int64_t r0 = g * group_rows;
    const int64_t outer0 = r0 / inner, rem0 = r0 - outer0 * inner;
    uint4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) {
      const int idx = u * kProbeThreads + (int)threadIdx.x;
      const int64_t lr = idx >> chunks_log2;
      int64_t rem = rem0 + lr, outer = outer0;
      while (rem >= inner) {
        rem -= inner;
        ++outer;
      }
      v[u] = uint4{0, 0, 0, 0};
      if (r0 + lr < rows)
        v[u] = *reinterpret_cast<const uint4*>(base + rem * inner_stride + outer * outer_stride +
                                               (int64_t)(idx & cmask) * 16);
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
  __shared__ uint32_t part[kProbeThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t x = 0;
    for (int i = 0; i < kProbeThreads / 64; ++i) x ^= part[i];
    sink[blockIdx.x] = x;
  }
}

}  // namespace be

extern "C" int be_read_probe(const void* base, int64_t rows, int64_t inner, int64_t inner_stride,
                             int64_t outer_stride, int row_bytes, uint32_t* sink, int grid, void* stream) {
  BE_REQUIRE(base && sink, "null base or sink");
  BE_REQUIRE(rows >= 0 && inner > 0 && grid > 0, "rows >= 0, inner > 0 and grid > 0 required");
  const int chunks = row_bytes / 16;
  BE_REQUIRE(row_bytes > 0 && row_bytes % 16 == 0 && (chunks & (chunks - 1)) == 0 && chunks <= be::kProbeGroupChunks,
             "row_bytes must be 16 bytes times a power of two, at most 16 * 2048");
  BE_REQUIRE((reinterpret_cast<uintptr_t>(base) & 15) == 0 && inner_stride % 16 == 0 && outer_stride % 16 == 0,
             "base and strides must be 16-byte aligned");
  if (rows == 0) return BE_OK;
  int log2 = 0;
  while ((1 << log2) < chunks) ++log2;
  be::read_probe_kernel<<<grid, be::kProbeThreads, 0, reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const char*>(base), rows, inner, inner_stride, outer_stride, log2, sink);
  BE_HIP_CHECK(hipGetLastError());
  return BE_OK;
}
