// chunk_bwd8's launches in a translation unit of their own: it takes gdr_kernels.hip's device code (its C ABI section
// is left out), instantiates only the chunk_bwd8 kernels, and is compiled with LLVM's max-memory-clause machine
// scheduling strategy (-mllvm -amdgpu-sched-strategy=max-memory-clause, see build.py), which keeps the kernel's
// vector-memory instructions in clauses: chunk_bwd8 2.5% faster at config 1 with its inputs out of the caches, the
// same bits.  Called from macai_gdr_chunk_bwd (gdr_kernels.hip) for bf16 inputs.
#define GDR_CB8_ONLY 1
#include "gdr_kernels.hip"

namespace gdr {

void cb8_launch(const ChunkBwdArgs& a, int DK, int DV, bool xn, int wgs, int units, dim3 grid, hipStream_t st) {
#define CB8_DISPATCH_DK(...)                                   \
  switch (DK) {                                                \
    case 32: { constexpr int DKC = 32; __VA_ARGS__; } break;   \
    case 64: { constexpr int DKC = 64; __VA_ARGS__; } break;   \
    default: { constexpr int DKC = 128; __VA_ARGS__; } break;  \
  }
  if (xn) {
    CB8_DISPATCH_DK(hipLaunchKernelGGL((chunk_bwd8xn_kernel<DKC>), dim3((unsigned)wgs), dim3(512), 0, st, a, units));
  } else {
    CB8_DISPATCH_DK(switch (DV) {
      case 32: hipLaunchKernelGGL((chunk_bwd8_kernel<DKC, 32>), grid, dim3(512), 0, st, a); break;
      case 64: hipLaunchKernelGGL((chunk_bwd8_kernel<DKC, 64>), grid, dim3(512), 0, st, a); break;
      case 96: hipLaunchKernelGGL((chunk_bwd8_kernel<DKC, 96>), grid, dim3(512), 0, st, a); break;
      default: hipLaunchKernelGGL((chunk_bwd8_kernel<DKC, 128>), grid, dim3(512), 0, st, a); break;
    })
  }
#undef CB8_DISPATCH_DK
}

}  // namespace gdr
