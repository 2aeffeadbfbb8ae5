// The rule's inference forward in one call: prep, then the state pass with the output (and the final state), the two
// launches the drop-in's forward makes without gradients, with the per-chunk operands in a workspace the caller
// passes.  It goes through macai_gdr_prep and macai_gdr_state_fwd, so it runs the same kernels with the same arguments
// as the separate calls: the same bits.
#include <hip/hip_runtime.h>

#include "gdr_abi.h"

namespace {

constexpr int64_t CH = 64;   // chunk length of the kernels

int64_t align256(int64_t n) { return (n + 255) & ~(int64_t)255; }

// Byte offsets of W, U, Ke, GL, Qg, M in a workspace for B batch rows (or packed sequences over NT chunks), each part
// on a 256-byte boundary; returns the total.
int64_t layout(int64_t B, int64_t T, int64_t H, int64_t DK, int64_t DV, int32_t dtype, int64_t NT_packed,
               int64_t off[6]) {
  const int64_t es = dtype == MACAI_GDR_F32 ? 4 : 2;
  const int64_t n = (NT_packed > 0 ? NT_packed : B * ((T + CH - 1) / CH)) * H;   // chunk-heads
  const int64_t sizes[6] = {n * CH * DK * es, n * CH * DV * 4, n * CH * DK * es, n * 4, n * CH * DK * es,
                            n * CH * CH * es};
  int64_t total = 0;
  for (int i = 0; i < 6; ++i) {
    off[i] = total;
    total += align256(sizes[i]);
  }
  return total;
}

// The value split for `rows` head-rows when the caller passes 0: the smallest split that gives every CU a workgroup
// (rows x split >= 256) with at most four column waves a workgroup, else the largest such split (the rule of the
// Python host's op.split_for: eight waves plus the loader leave too few registers a wave).
int32_t auto_split(int64_t rows, int64_t DV) {
  const int ncb = (int)(DV / 16);
  int32_t last = 0;
  for (int s = 1; s <= ncb; ++s) {
    if (ncb % s) continue;
    const int nw = ncb / s;
    if (nw != 1 && nw != 2 && nw != 4) continue;
    last = s;
    if (rows * s >= 256) return s;
  }
  return last;   // 0 when DV / 16 has no such split: the entry point's own choice
}

int forward_in(const char* what, const void* q, const void* k, const void* v, const float* g, const float* beta,
               const float* s0, void* o, float* sT, char* ws, int64_t ws_bytes, int64_t B, int64_t T, int64_t H,
               int64_t Hk, int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm, float q_scale, int32_t split,
               const int32_t* pack, int64_t NT_packed, void* stream) {
  if (B < 1 || T < 1 || H < 1 || DK < 1 || DV < 1)
    return fail(MACAI_GDR_EINVAL, "%s: B, T, H, DK, DV must be >= 1", what);
  if (pack && NT_packed < 1) return fail(MACAI_GDR_EINVAL, "%s: packed rows need their chunk count", what);
  int64_t off[6];
  const int64_t need = layout(B, T, H, DK, DV, dtype, pack ? NT_packed : 0, off);
  if (!ws) return fail(MACAI_GDR_EINVAL, "%s: null workspace", what);
  if (((uintptr_t)ws & 255u) != 0) return fail(MACAI_GDR_EINVAL, "%s: the workspace must be 256-byte aligned", what);
  if (ws_bytes < need)
    return fail(MACAI_GDR_EINVAL, "%s: the workspace holds %lld bytes, this shape needs %lld", what,
                (long long)ws_bytes, (long long)need);
  void* W = ws + off[0];
  float* U = (float*)(ws + off[1]);
  void* Ke = ws + off[2];
  float* GL = (float*)(ws + off[3]);
  void* Qg = ws + off[4];
  void* M = ws + off[5];
  if (int rc = macai_gdr_prep(q, k, v, g, beta, W, U, Ke, GL, Qg, M, nullptr, B, T, H, Hk, DK, DV, dtype, use_l2norm,
                              q_scale, pack, NT_packed, stream))
    return rc;
  if (split == 0) split = auto_split(B * H, DV);
  return macai_gdr_state_fwd(W, U, Ke, GL, Qg, M, s0, o, sT, nullptr, nullptr, B, T, H, DK, DV, dtype, 0, split, pack,
                             NT_packed, stream);
}

}  // namespace

extern "C" {

int64_t macai_gdr_forward_workspace(int64_t B, int64_t T, int64_t H, int64_t DK, int64_t DV, int32_t dtype,
                                    int64_t NT_packed) {
  int64_t off[6];
  return layout(B, T, H, DK, DV, dtype, NT_packed, off);
}

int macai_gdr_forward(const void* q, const void* k, const void* v, const float* g, const float* beta,
                      const float* s0, void* o, float* sT, void* workspace, int64_t workspace_bytes, int64_t B,
                      int64_t T, int64_t H, int64_t Hk, int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm,
                      float q_scale, int32_t split, const int32_t* pack, int64_t NT_packed, void* stream) {
  return forward_in("macai_gdr_forward", q, k, v, g, beta, s0, o, sT, (char*)workspace, workspace_bytes, B, T, H, Hk,
                    DK, DV, dtype, use_l2norm, q_scale, split, pack, NT_packed, stream);
}

}  // extern "C"
