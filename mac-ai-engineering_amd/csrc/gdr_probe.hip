// Probes of the device's ceilings, for measurement only (bench.py --ceilings): the memory streams (read-only,
// write-only and copy over a buffer of 16-byte units, grid-stride, every unit touched once) and the matrix cores (back
// to back MFMAs of the shapes the kernels use).  The rule's kernels are judged against these rates beside the vendor
// peaks.
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

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// MFMA throughput: every wave runs `iters` rounds of NCH independent accumulator chains of one instruction (round r of
// a chain depends on round r - 1, so NCH chains in flight cover the instruction's latency), on operands formed once in
// registers; the accumulators are stored at the end, so no product is dead.  MODE 0: v_mfma_f32_16x16x32_bf16 (the
// bf16 kernels' shape, 16,384 FLOP), 1: v_mfma_f32_16x16x4_f32 (the float32 kernels', 2,048), 2:
// v_mfma_f32_32x32x16_bf16 (gfx950's larger bf16 shape, 32,768).
constexpr int NCH = 8;
template <int MODE>
__global__ void __launch_bounds__(256) probe_mfma_kernel(int iters, float* out) {
  const int l = threadIdx.x & 63;
  const float x = 1.0f + 1e-3f * (float)l;
  if constexpr (MODE == 2) {
    f16v acc[NCH];
    bf16x8 a, b;
    for (int e = 0; e < 8; ++e) {
      a[e] = (__bf16)(x + e);
      b[e] = (__bf16)(x - e);
    }
    for (int c = 0; c < NCH; ++c)
      for (int e = 0; e < 16; ++e) acc[c][e] = 0.f;
    for (int i = 0; i < iters; ++i)
#pragma unroll
      for (int c = 0; c < NCH; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    float s = 0.f;
    for (int c = 0; c < NCH; ++c)
      for (int e = 0; e < 16; ++e) s += acc[c][e];
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
  } else {
    f4 acc[NCH];
    for (int c = 0; c < NCH; ++c) acc[c] = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (MODE == 0) {
      bf16x8 a, b;
      for (int e = 0; e < 8; ++e) {
        a[e] = (__bf16)(x + e);
        b[e] = (__bf16)(x - e);
      }
      for (int i = 0; i < iters; ++i)
#pragma unroll
        for (int c = 0; c < NCH; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[c], 0, 0, 0);
    } else {
      const float a = x, b = 2.f - x;
      for (int i = 0; i < iters; ++i)
#pragma unroll
        for (int c = 0; c < NCH; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[c], 0, 0, 0);
    }
    float s = 0.f;
    for (int c = 0; c < NCH; ++c) s += (acc[c][0] + acc[c][1]) + (acc[c][2] + acc[c][3]);
    out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
  }
}

}  // namespace

extern "C" int64_t macai_gdr_probe_mfma_flops(int32_t mode, int32_t iters, int32_t blocks) {
  static const int64_t per_instr[3] = {16384, 2048, 32768};
  if (mode < 0 || mode > 2 || iters < 1 || blocks < 1) return -1;
  return per_instr[mode] * NCH * (int64_t)iters * (int64_t)blocks * 4;   // 4 waves a workgroup
}

extern "C" int macai_gdr_probe_mfma(int32_t mode, int32_t iters, void* out, int32_t blocks, void* stream) {
  const char* what = "macai_gdr_probe_mfma";
  if (mode < 0 || mode > 2) return fail(MACAI_GDR_EINVAL, "%s: mode must be 0, 1 or 2", what);
  if (iters < 1 || iters > (1 << 24)) return fail(MACAI_GDR_EINVAL, "%s: iters must be in [1, 2^24]", what);
  if (blocks < 1 || blocks > (1 << 20)) return fail(MACAI_GDR_EINVAL, "%s: blocks must be in [1, 2^20]", what);
  if (!out || !aligned16(out))
    return fail(MACAI_GDR_EINVAL, "%s: out (blocks x 256 floats) must be 16-byte aligned", what);
  hipStream_t st = (hipStream_t)stream;
  if (mode == 0) hipLaunchKernelGGL(probe_mfma_kernel<0>, dim3(blocks), dim3(256), 0, st, iters, (float*)out);
  else if (mode == 1) hipLaunchKernelGGL(probe_mfma_kernel<1>, dim3(blocks), dim3(256), 0, st, iters, (float*)out);
  else hipLaunchKernelGGL(probe_mfma_kernel<2>, dim3(blocks), dim3(256), 0, st, iters, (float*)out);
  return launched(what);
}

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
