// Read-only HBM stream for gfx950: the bandwidth ceiling the decode kernels'
// roofline fractions are read against (a device copy also writes, so it
// understates what a read-dominated kernel can reach).  Each thread reads
// 16-byte units grid-stride, four in flight, and folds them into one word;
// each block stores one word.
#include "rfsn_common.h"
#include "rfsn_internal.h"

namespace rfsn {
namespace {

__global__ void __launch_bounds__(256) read_stream_kernel(const uint4* __restrict__ src, int64_t n,
                                                          uint32_t* __restrict__ out) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int k = 0; k < 256; ++k) r ^= red[k];
    out[blockIdx.x] = r;
  }
}

}  // namespace
}  // namespace rfsn

using namespace rfsn;

extern "C" int rfsn_read_stream(const void* src, int64_t bytes, uint32_t* out, int32_t blocks, void* stream) {
  RFSN_REQUIRE(src && out, "read_stream: null pointer");
  RFSN_REQUIRE(bytes > 0 && bytes % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0,
               "read_stream: bytes must be a positive multiple of 16 on a 16-byte aligned buffer");
  RFSN_REQUIRE(blocks > 0 && blocks <= (1 << 20), "read_stream: blocks must be in [1, 2^20]");
  hipLaunchKernelGGL(read_stream_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)src, bytes / 16, out);
  return check_launch("read_stream");
}
