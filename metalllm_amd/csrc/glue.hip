// glue.hip -- the elementwise glue kernels of metalLLM's training step that sit next to the
// attention sublayer (declared in include/metalllm_attn.h):
//   castFloatToBfloat  elementwise.metal:19-28  out[i] = bf16(in[i])  (model.h:692: the fp32 dX of
//                      computeGradDx handed to the layernorm backward as bf16)
// HBM-bound streaming kernels: 16-byte loads, grid-stride loops sized to a few waves per CU.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/metalllm_attn.h"

namespace {

// float -> bf16, round to nearest even (Metal's float -> bfloat conversion); NaN stays a quiet
// NaN of the same sign, infinities and overflow to infinity as in IEEE rounding.
__device__ __forceinline__ uint32_t to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__global__ void __launch_bounds__(256) cast_kernel(const float* __restrict__ in, uint16_t* __restrict__ out,
                                                   uint32_t count) {
  const size_t n4 = count / 4;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = ((const float4*)in)[i];
    ((uint2*)out)[i] = uint2{to_bf16(v.x) | (to_bf16(v.y) << 16), to_bf16(v.z) | (to_bf16(v.w) << 16)};
  }
  // the count % 4 tail
  const size_t t = 4 * n4 + blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (t < count) out[t] = (uint16_t)to_bf16(in[t]);
}

unsigned grid_for(size_t items) { return (unsigned)std::max<size_t>(1, std::min<size_t>((items + 255) / 256, 8192)); }

}  // namespace

extern "C" {

int castFloatToBfloat(const float* in, uint16_t* out, uint32_t count, metalllm_stream_t stream) {
  if (count == 0) return METALLLM_ATTN_OK;
  if (!in || !out) return METALLLM_ATTN_E_NULL;
  if (((uintptr_t)in & 15u) || ((uintptr_t)out & 15u)) return METALLLM_ATTN_E_ALIGN;
  hipLaunchKernelGGL(cast_kernel, dim3(grid_for(count / 4 + 1)), dim3(256), 0, (hipStream_t)stream, in, out, count);
  return hipGetLastError() == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

}  // extern "C"
