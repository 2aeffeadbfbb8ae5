// Streaming probes of the device's memory ceilings, for measurement only (bench.py --ceilings): read-only,
// write-only and copy over a buffer of 16-byte units, grid-stride, every unit touched once.  The rule's kernels are
// judged against these rates beside the vendor peak.
#include <hip/hip_runtime.h>

#include "gdr_abi.h"

namespace {

__global__ void __launch_bounds__(256) probe_read_kernel(const uint4* __restrict__ src, int64_t n, uint4* sink) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const uint4 x = src[i];
    acc ^= x.x ^ x.y ^ x.z ^ x.w;
  }
  // a store the compiler cannot prove dead, taken by (almost) no lane: keeps every load
  if (acc == 0x9e3779b9u) sink[0] = uint4{acc, acc, acc, acc};
}

__global__ void __launch_bounds__(256) probe_write_kernel(uint4* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const uint32_t v = (uint32_t)i;
    dst[i] = uint4{v, v + 1, v + 2, v + 3};
  }
}

__global__ void __launch_bounds__(256) probe_copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                         int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

}  // namespace

extern "C" int macai_gdr_probe_stream(int32_t mode, const void* src, void* dst, int64_t bytes, int32_t blocks,
                                      void* stream) {
  const char* what = "macai_gdr_probe_stream";
  if (mode < 0 || mode > 2) return fail(MACAI_GDR_EINVAL, "%s: mode must be 0 (read), 1 (write) or 2 (copy)", what);
  if (bytes < 16 || bytes % 16 != 0) return fail(MACAI_GDR_EINVAL, "%s: bytes must be a positive multiple of 16", what);
  if (blocks < 1 || blocks > (1 << 20)) return fail(MACAI_GDR_EINVAL, "%s: blocks must be in [1, 2^20]", what);
  if ((mode != 1 && !src) || !dst) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  if (!aligned16(src) || !aligned16(dst)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  const int64_t n = bytes / 16;
  hipStream_t st = (hipStream_t)stream;
  if (mode == 0)
    hipLaunchKernelGGL(probe_read_kernel, dim3(blocks), dim3(256), 0, st, (const uint4*)src, n, (uint4*)dst);
  else if (mode == 1)
    hipLaunchKernelGGL(probe_write_kernel, dim3(blocks), dim3(256), 0, st, (uint4*)dst, n);
  else
    hipLaunchKernelGGL(probe_copy_kernel, dim3(blocks), dim3(256), 0, st, (const uint4*)src, (uint4*)dst, n);
  return launched(what);
}
