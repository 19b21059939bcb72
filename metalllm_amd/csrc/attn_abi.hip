// attn_abi.hip -- extern "C" entry points of libmetalllm_attn.so (declared in
// include/metalllm_attn.h). Validation happens on the host before any HIP call, so argument
// errors are reported without touching the device.
#include <cmath>

#include "../../include/metalllm_attn.h"
#include "attn_launch.hpp"

namespace {

int validate(const AttentionParams* p) {
  if (!p) return METALLLM_ATTN_E_NULL;
  if (p->M == 0 || p->M % 64) return METALLLM_ATTN_E_SEQLEN;
  if (p->D != 64 && p->D != 128) return METALLLM_ATTN_E_HEADDIM;
  if (p->NH == 0 || p->B == 0 || (uint64_t)p->N != (uint64_t)p->NH * p->D) return METALLLM_ATTN_E_LAYOUT;
  if ((uint64_t)p->B * p->M * p->N >= (1ull << 31)) return METALLLM_ATTN_E_SIZE;
  return METALLLM_ATTN_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

float head_scale(uint32_t D) { return 1.0f / std::sqrt((float)D); }  // attention.metal:109,268

}  // namespace

extern "C" {

int flashAttentionForward(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out, float* l,
                          const AttentionParams* p, metalllm_stream_t stream) {
  const int rc = validate(p);
  if (rc) return rc;
  if (!q || !k || !v || !out || !l) return METALLLM_ATTN_E_NULL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out) || !aligned16(l))
    return METALLLM_ATTN_E_ALIGN;
  mla::FwdArgs a{q, k, v, out, l, (int)p->M, (int)p->NH, (int)p->B, head_scale(p->D)};
  return mla::launch_forward(a, (int)p->D, (hipStream_t)stream) == hipSuccess ? METALLLM_ATTN_OK
                                                                               : METALLLM_ATTN_E_LAUNCH;
}

int computeD(const uint16_t* dO, const uint16_t* O, float* D, const AttentionParams* p, metalllm_stream_t stream) {
  const int rc = validate(p);
  if (rc) return rc;
  if (!dO || !O || !D) return METALLLM_ATTN_E_NULL;
  if (!aligned16(dO) || !aligned16(O) || !aligned16(D)) return METALLLM_ATTN_E_ALIGN;
  mla::ComputeDArgs a{dO, O, D, (int)p->M, (int)p->NH, (int)p->B};
  return mla::launch_compute_d(a, (int)p->D, (hipStream_t)stream) == hipSuccess ? METALLLM_ATTN_OK
                                                                                : METALLLM_ATTN_E_LAUNCH;
}

int metalllmAttnBackwardWorkspaceSize(const AttentionParams* p, uint64_t* bytes) {
  const int rc = validate(p);
  if (rc) return rc;
  if (!bytes) return METALLLM_ATTN_E_NULL;
  *bytes = (uint64_t)mla::ds_scratch_bytes((int)p->B, (int)p->NH, (int)p->M);
  return METALLLM_ATTN_OK;
}

int metalllmAttnBackwardPart(int part, const uint16_t* dZ, const float* d, const float* l, const uint16_t* q,
                             const uint16_t* k, const uint16_t* v, float* dQ, uint16_t* dK, uint16_t* dV,
                             void* workspace, uint64_t workspace_bytes, const AttentionParams* p,
                             metalllm_stream_t stream) {
  const int rc = validate(p);
  if (rc) return rc;
  if (part < 0 || part > 3) return METALLLM_ATTN_E_LAYOUT;
  if (!dZ || !d || !l || !q || !k || !v || !dQ || !dK || !dV) return METALLLM_ATTN_E_NULL;
  if (!aligned16(dZ) || !aligned16(d) || !aligned16(l) || !aligned16(q) || !aligned16(k) || !aligned16(v) ||
      !aligned16(dQ) || !aligned16(dK) || !aligned16(dV))
    return METALLLM_ATTN_E_ALIGN;
  mla::BwdArgs a{dZ, d, l, q, k, v, dQ, dK, dV, (int)p->M, (int)p->NH, (int)p->B, head_scale(p->D)};
  if (part >= 2) {
    if (!workspace) return METALLLM_ATTN_E_NULL;
    if (!aligned16(workspace)) return METALLLM_ATTN_E_ALIGN;
    if (workspace_bytes < (uint64_t)mla::ds_scratch_bytes(a.B, a.H, a.T)) return METALLLM_ATTN_E_SIZE;
    a.dS = (uint16_t*)workspace;
  }
  if (mla::backward_is_short(a.T, (int)p->D)) {
    // one fused kernel computes dK, dV and dQ (part 0 adds dQ, part 2 writes it); parts 1 and 3
    // have nothing left to do
    if (part == 1 || part == 3) return METALLLM_ATTN_OK;
    return mla::launch_backward_short(a, part == 0, (hipStream_t)stream) == hipSuccess ? METALLLM_ATTN_OK
                                                                                         : METALLLM_ATTN_E_LAUNCH;
  }
  hipError_t e;
  if (part >= 2 && mla::workspace_recomputes(a.T, (int)p->D)) {
    // the recomputing kernels, dQ written: faster than the dS round trip at this head size (the
    // workspace is validated but not used)
    a.dS = nullptr;
    e = part == 2 ? mla::launch_backward(a, (int)p->D, (hipStream_t)stream)
                  : mla::launch_backward_dq(a, (int)p->D, false, (hipStream_t)stream);
  } else {
    e = part == 0 || part == 2 ? mla::launch_backward(a, (int)p->D, (hipStream_t)stream)
        : part == 1           ? mla::launch_backward_dq(a, (int)p->D, true, (hipStream_t)stream)
                              : mla::launch_backward_dqs(a, (int)p->D, (hipStream_t)stream);
  }
  return e == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

int flashAttentionBackward(const uint16_t* dZ, const float* d, const float* l, const uint16_t* q,
                           const uint16_t* k, const uint16_t* v, float* dQ, uint16_t* dK, uint16_t* dV,
                           const AttentionParams* p, metalllm_stream_t stream) {
  // dK/dV by the key-block owners, then dQ by the query-block owners (both on `stream`, in order)
  const int rc = metalllmAttnBackwardPart(0, dZ, d, l, q, k, v, dQ, dK, dV, nullptr, 0, p, stream);
  if (rc) return rc;
  return metalllmAttnBackwardPart(1, dZ, d, l, q, k, v, dQ, dK, dV, nullptr, 0, p, stream);
}

int flashAttentionBackwardWorkspace(const uint16_t* dZ, const float* d, const float* l, const uint16_t* q,
                                    const uint16_t* k, const uint16_t* v, float* dQ, uint16_t* dK, uint16_t* dV,
                                    void* workspace, uint64_t workspace_bytes, const AttentionParams* p,
                                    metalllm_stream_t stream) {
  // dK/dV by the key-block owners, storing dS into the workspace; then dQ = dS.K
  const int rc = metalllmAttnBackwardPart(2, dZ, d, l, q, k, v, dQ, dK, dV, workspace, workspace_bytes, p, stream);
  if (rc) return rc;
  return metalllmAttnBackwardPart(3, dZ, d, l, q, k, v, dQ, dK, dV, workspace, workspace_bytes, p, stream);
}

const char* metalllmAttnErrorString(int code) {
  switch (code) {
    case METALLLM_ATTN_OK: return "ok";
    case METALLLM_ATTN_E_NULL: return "a required pointer is NULL";
    case METALLLM_ATTN_E_SEQLEN: return "sequence length M must be a positive multiple of 64";
    case METALLLM_ATTN_E_HEADDIM: return "head size D must be 64 or 128";
    case METALLLM_ATTN_E_LAYOUT: return "N must equal NH*D with NH >= 1 and B >= 1";
    case METALLLM_ATTN_E_SIZE: return "a tensor exceeds 2^31 elements";
    case METALLLM_ATTN_E_ALIGN: return "tensor pointers must be 16-byte aligned";
    case METALLLM_ATTN_E_LAUNCH: return "kernel launch failed";
    case METALLLM_ATTN_E_LIBRARY: return "platform library call (rocBLAS, device allocation) failed";
    case METALLLM_ATTN_E_CAPTURE: return "scratch would grow during stream capture (call metalllmSublayerReserve first)";
    default: return "unknown error";
  }
}

int metalllmAttnWorkMap(int kind, const AttentionParams* p, int32_t* out, int32_t count) {
  const int rc = validate(p);
  if (rc) return rc;
  if (!out && count > 0) return METALLLM_ATTN_E_NULL;
  if (kind < 0 || kind > 2) return METALLLM_ATTN_E_LAYOUT;
  const int npairs = (int)(p->B * p->NH);
  const int blk = kind == 0 ? mla::kFwdBlockM : kind == 1 ? mla::kBwdBlockN : mla::kDqBlockM;
  const int nblk = ((int)p->M + blk - 1) / blk;
  const int grid = npairs * nblk;
  for (int i = 0; i < count && i < grid; ++i) {
    int pair, b;
    const int round = kind == 0 ? mla::kFwdDispatchRound : mla::bwd_dispatch_round((int)p->D);
    mla::decode_workgroup(i, npairs, nblk, kind != 1, round, pair, b);
    out[2 * i] = pair;
    out[2 * i + 1] = b;
  }
  return grid;
}

int metalllmAttnForwardItems(const AttentionParams* p, int32_t grid, int32_t* out, int32_t count) {
  const int rc = validate(p);
  if (rc) return rc;
  if (grid <= 0) return METALLLM_ATTN_E_LAYOUT;
  if (!out && count > 0) return METALLLM_ATTN_E_NULL;
  const int npairs = (int)(p->B * p->NH);
  const int nblk = ((int)p->M + mla::kFwdBlockM - 1) / mla::kFwdBlockM;
  int n = 0;
  for (int w = 0; w < grid; ++w) {
    int pair, blk;
    for (int k = 0; mla::fwd_item_of(w, grid, k, npairs, nblk, pair, blk); ++k, ++n) {
      if (n < count) {
        out[3 * n] = w;
        out[3 * n + 1] = pair;
        out[3 * n + 2] = blk;
      }
    }
  }
  return n;
}

}  // extern "C"
