// The rule's inference forward in one call: prep, then the state pass with the output (and the final state), the two
// launches the drop-in's forward makes without gradients.  macai_gdr_forward takes the per-chunk operands' workspace
// from the caller; macai_gdr_forward_noalloc takes it from a fixed device array of this file instead, for callers that
// cannot allocate (HIP graph capture, serving loops).  Both go through macai_gdr_prep and macai_gdr_state_fwd, so they
// run the same kernels with the same arguments as the separate calls: the same bits.
#include <hip/hip_runtime.h>

#include <mutex>

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

// The value split for `rows` head-rows when the caller passes 0: the largest split with at most four column waves a
// workgroup whose workgroups all fit the 256 CUs at once (rows x split <= 256), else the smallest such split (the rule
// of the Python host's op.split_for: eight waves plus the loader leave too few registers a wave, and a second round
// of workgroups would double a sequential pass's time).
int32_t auto_split(int64_t rows, int64_t DV) {
  const int ncb = (int)(DV / 16);
  int32_t first = 0, best = 0;
  for (int s = 1; s <= ncb; ++s) {
    if (ncb % s) continue;
    const int nw = ncb / s;
    if (nw != 1 && nw != 2 && nw != 4) continue;
    if (!first) first = s;
    if (rows * s <= 256) best = s;
  }
  return best ? best : first;   // 0 when DV / 16 has no such split: the entry point's own choice
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

// The workspace of macai_gdr_forward_noalloc: one copy per device, held for the process's lifetime.  Host code reaches
// it only through the address hipGetSymbolAddress returns on the current device (device_scratch), never by its name:
// in host code the name stands for a host-side shadow, not device memory.  Every call on a device shares its copy,
// and prep rewrites every byte the state pass then reads, so nothing in it needs clearing between calls.  This file
// defines no kernel, so its code object holds the array alone and is loaded (the array reserved) by the first
// hipGetSymbolAddress on a device, not when the library loads.
constexpr int64_t SCRATCH_BYTES = MACAI_GDR_NOALLOC_SCRATCH_BYTES;
constexpr int MAX_DEVICES = 64;
__device__ __align__(256) char scratch[SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch[MAX_DEVICES] = {};

// The scratch array's address on the current device, looked up on the first call there.
int device_scratch(const char* what, char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MACAI_GDR_ELAUNCH, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= MAX_DEVICES) return fail(MACAI_GDR_EUNSUP, "%s: device %d out of range", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MACAI_GDR_ELAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                  hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = (char*)g_scratch[dev];
  return MACAI_GDR_OK;
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

int macai_gdr_forward_noalloc(const void* q, const void* k, const void* v, const float* g, const float* beta,
                              const float* s0, void* o, float* sT, int64_t B, int64_t T, int64_t H, int64_t Hk,
                              int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm, float q_scale, int32_t split,
                              const int32_t* pack, int64_t NT_packed, void* stream) {
  const char* what = "macai_gdr_forward_noalloc";
  if (B >= 1 && T >= 1 && H >= 1 && DK >= 1 && DV >= 1 && (!pack || NT_packed >= 1)) {
    int64_t off[6];
    const int64_t need = layout(B, T, H, DK, DV, dtype, pack ? NT_packed : 0, off);
    if (need > SCRATCH_BYTES)
      return fail(MACAI_GDR_EINVAL,
                  "%s: this shape needs %lld bytes of per-chunk operands, over the fixed %lld-byte scratch; use "
                  "macai_gdr_forward with a workspace",
                  what, (long long)need, (long long)SCRATCH_BYTES);
  }
  char* ws = nullptr;
  if (int rc = device_scratch(what, &ws)) return rc;
  return forward_in(what, q, k, v, g, beta, s0, o, sT, ws, SCRATCH_BYTES, B, T, H, Hk, DK, DV, dtype, use_l2norm,
                    q_scale, split, pack, NT_packed, stream);
}

}  // extern "C"
