// attn_noalloc.hip -- flashAttentionBackwardNoAlloc: the stored-dS backward
// (flashAttentionBackwardWorkspace) for callers that cannot allocate device memory (code under
// HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The dS tiles go into a
// file-scope device array of METALLLM_ATTN_NOALLOC_SCRATCH_BYTES instead of a caller workspace;
// shapes whose tiles do not fit are rejected. At D = 64 the workspace entry point stores no dS
// tiles (the fused short-sequence kernel, or the recomputing kernels), so every D = 64 shape
// fits. Every GPU the library runs on holds its own copy of the array until the process ends, and
// every call on one GPU shares it: calls that overlap on one GPU (different streams, or different
// host threads) race. The kernels write every dS tile they read within one call, so the array
// needs no clearing between calls.
#include <mutex>

#include "../../include/metalllm_attn.h"
#include "attn_launch.hpp"

namespace {

constexpr size_t kScratchBytes = METALLLM_ATTN_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

// The array's address on each device (hipGetSymbolAddress, taken once per device with that
// device current). In host code the name `scratch` is a host-side stand-in: only these
// addresses may be handed to kernels.
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};

int scratch_on_current_device(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return METALLLM_ATTN_E_LIBRARY;
  std::lock_guard<std::mutex> g(g_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return METALLLM_ATTN_E_LIBRARY;
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return METALLLM_ATTN_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace

extern "C" int flashAttentionBackwardNoAlloc(const uint16_t* dZ, const float* d, const float* l, const uint16_t* q,
                                             const uint16_t* k, const uint16_t* v, float* dQ, uint16_t* dK,
                                             uint16_t* dV, const AttentionParams* p, metalllm_stream_t stream) {
  // every argument is checked on the host before the device is touched
  uint64_t need = 0;
  const int rc = metalllmAttnBackwardWorkspaceSize(p, &need);  // validates the shape
  if (rc) return rc;
  // At D = 64 the workspace entry point never reads the workspace (M <= 256: the fused
  // short-sequence backward keeps dS in LDS; longer: the recomputing kernels): any shape fits
  // there, and the nominal size is passed on so that the entry point's own size check accepts it
  const int M = (int)p->M, D = (int)p->D;
  const bool no_tiles = mla::backward_is_short(M, D) || mla::workspace_recomputes(M, D);
  if (!no_tiles && need > kScratchBytes) return METALLLM_ATTN_E_SIZE;
  if (!dZ || !d || !l || !q || !k || !v || !dQ || !dK || !dV) return METALLLM_ATTN_E_NULL;
  if (!aligned16(dZ) || !aligned16(d) || !aligned16(l) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      !aligned16(dQ) || !aligned16(dK) || !aligned16(dV))
    return METALLLM_ATTN_E_ALIGN;
  void* ws = nullptr;
  const int src = scratch_on_current_device(&ws);
  if (src) return src;
  return flashAttentionBackwardWorkspace(dZ, d, l, q, k, v, dQ, dK, dV, ws, no_tiles ? need : kScratchBytes, p,
                                         stream);
}
