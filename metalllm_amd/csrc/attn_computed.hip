// attn_computed.hip -- computeD on gfx950.
//
// Reference: /root/reference/attention.metal:166-195. One 32-lane simdgroup per (t, h) row:
// lane l sums bf16(dO*O) over the columns l, l+32, ... in fp32 starting from 0 (:188-191; MSL
// bfloat*bfloat rounds the product to bfloat), simd_sum adds the 32 lane sums (:192), and D is
// stored as bf16 (:193). This build keeps the bf16 value, written into the fp32 D buffer
// ([B,H,T]). simd_sum's order is not published; it is taken as the xor butterfly (partners at
// distance 16, 8, 4, 2, 1), the same order the CPU oracle uses, so the two agree bit for bit.
//
// HBM-bound: reads 4*B*T*H*D bytes, writes 4*B*H*T. Four lanes (a DPP quad) own one row: lane
// j of the quad holds the reference lanes 8j .. 8j+7, i.e. columns 32m + 8j .. +7 for every
// 32-column block m (16-byte loads of dO and O). Each lane forms its eight reference-lane sums in
// column order; the butterfly's distances 16 and 8 are quad partners j^2 and j^1 (DPP quad
// permutes), distances 4, 2, 1 are in-lane.
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

// quad_perm controls of the DPP move: the partner lane j^1 and j^2 within each quad
constexpr int kQuadXor1 = 1 | (0 << 2) | (3 << 4) | (2 << 6);
constexpr int kQuadXor2 = 2 | (3 << 2) | (0 << 4) | (1 << 6);

template <int CTRL>
__device__ __forceinline__ float quad_partner(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

template <int D>
__global__ void __launch_bounds__(256) compute_d_kernel(ComputeDArgs a, uint64_t nrows) {
  constexpr int NB = D / 32;  // 32-column blocks of a row
  const uint64_t gid = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  const uint64_t row = gid >> 2;  // (b*T + t)*H + h: rows of [B,T,H,D] are contiguous
  const int j = (int)(gid & 3);
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  if (row < nrows) {
    u32x4 x[NB], y[NB];
#pragma unroll
    for (int m = 0; m < NB; ++m) {
      x[m] = *(const u32x4*)(a.dO + row * D + 32 * m + 8 * j);
      y[m] = *(const u32x4*)(a.O + row * D + 32 * m + 8 * j);
    }
#pragma unroll
    for (int m = 0; m < NB; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t p = pack_bf16(bf_lo(x[m][i]) * bf_lo(y[m][i]), bf_hi(x[m][i]) * bf_hi(y[m][i]));
        acc[2 * i] = acc[2 * i] + bf_lo(p);
        acc[2 * i + 1] = acc[2 * i + 1] + bf_hi(p);
      }
  }
  // butterfly over the 32 reference lanes 8j + e
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = acc[e] + quad_partner<kQuadXor2>(acc[e]);  // distance 16
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = acc[e] + quad_partner<kQuadXor1>(acc[e]);  // distance 8
#pragma unroll
  for (int e = 0; e < 4; ++e) acc[e] = acc[e] + acc[e ^ 4];  // distance 4
#pragma unroll
  for (int e = 0; e < 2; ++e) acc[e] = acc[e] + acc[e ^ 2];  // distance 2
  const float total = acc[0] + acc[1];                         // distance 1
  if (row < nrows && j == 0) {
    const uint64_t h = row % (uint64_t)a.H, bt = row / (uint64_t)a.H;
    const uint64_t t = bt % (uint64_t)a.T, b = bt / (uint64_t)a.T;
    a.Dv[(b * a.H + h) * a.T + t] = bf_lo(pack_bf16(total, total));
  }
}

hipError_t launch_compute_d(const ComputeDArgs& a, int D, hipStream_t s) {
  const uint64_t nrows = (uint64_t)a.B * a.T * a.H;
  const dim3 grid((unsigned)((nrows * 4 + 255) / 256));
  if (D == 64)
    hipLaunchKernelGGL(compute_d_kernel<64>, grid, dim3(256), 0, s, a, nrows);
  else
    hipLaunchKernelGGL(compute_d_kernel<128>, grid, dim3(256), 0, s, a, nrows);
  return hipGetLastError();
}

}  // namespace mla
