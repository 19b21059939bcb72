// attn_computed.hip -- computeD on gfx950.
//
// Reference: /root/reference/attention.metal:166-195. D[t,h] = sum_d dO[t,h,d]*O[t,h,d] with
// each product rounded to bf16 (MSL bfloat*bfloat) and summed in fp32; the reference stores the
// result as bf16, which this build keeps (rounded to bf16, written into the fp32 D buffer).
//
// HBM-bound: reads 4*B*T*H*D bytes, writes 4*B*H*T. One lane owns 8 consecutive d of one
// (b,t,h) row (a 16-byte load from each tensor); the D/8 lanes of a row sum their 8 products
// in order and combine with an xor butterfly (pairs 0+1, 2+3, ..., then pairs of pairs).
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

template <int D>
__global__ void __launch_bounds__(256) compute_d_kernel(ComputeDArgs a, uint64_t nseg) {
  constexpr int CPS = D / 8;  // lanes per (b,t,h) row
  const uint64_t gid = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  const uint64_t seg = gid / CPS;
  float acc = 0.0f;
  if (seg < nseg) {
    const u32x4 x = *(const u32x4*)(a.dO + gid * 8);
    const u32x4 y = *(const u32x4*)(a.O + gid * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t p = pack_bf16(bf_lo(x[i]) * bf_lo(y[i]), bf_hi(x[i]) * bf_hi(y[i]));
      acc = acc + bf_lo(p);
      acc = acc + bf_hi(p);
    }
  }
#pragma unroll
  for (int w = 1; w < CPS; w <<= 1) acc = acc + __shfl_xor(acc, w, 64);
  if (seg < nseg && (gid % CPS) == 0) {
    const uint64_t h = seg % (uint64_t)a.H, bt = seg / (uint64_t)a.H;
    const uint64_t t = bt % (uint64_t)a.T, b = bt / (uint64_t)a.T;
    const uint32_t r = pack_bf16(acc, acc);
    a.Dv[(b * a.H + h) * a.T + t] = bf_lo(r);
  }
}

hipError_t launch_compute_d(const ComputeDArgs& a, int D, hipStream_t s) {
  const uint64_t nseg = (uint64_t)a.B * a.T * a.H;
  const uint64_t lanes = nseg * (uint64_t)(D / 8);
  const dim3 grid((unsigned)((lanes + 255) / 256));
  if (D == 64)
    hipLaunchKernelGGL(compute_d_kernel<64>, grid, dim3(256), 0, s, a, nseg);
  else
    hipLaunchKernelGGL(compute_d_kernel<128>, grid, dim3(256), 0, s, a, nseg);
  return hipGetLastError();
}

}  // namespace mla
