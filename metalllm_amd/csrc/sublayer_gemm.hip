// sublayer_gemm.hip -- hand-written matrix-core kernel for computeGradDx
// (/root/reference/attention.metal:301-341):
//   dX += dQ.Wq^T + dK.Wk^T + dV.Wv^T
// with dQ fp32, dK and dV bf16 [R, C], weights bf16 [C, C] indexed [input feature][output
// feature] and dX fp32 [R, C] (read once, written once).
//
// The reference reads the fp32 dQ directly (its matmul2d mixes the float dQ with bfloat weights
// into a float destination). Here the kernel loads dQ as fp32 and splits every element in
// registers into two bf16 terms, hi = bf16(x) and lo = bf16(x - hi) (|x - hi - lo| <= 2^-17 |x|),
// and runs the product on both: the fp32 gradient reaches the matrix cores without a bf16 round
// trip and without a separate split pass through HBM. All three products accumulate into one set
// of fp32 accumulators, so dX is read and written once instead of once per product.
//
// Tiling: a workgroup of 4 waves computes a 128 (rows r) x 128 (features i) tile of dX as
// dX^T = W . G^T (m = i, n = r, k = j): the A operand is a weight row W[i][j..j+7] and the B
// operand a gradient row G[r][j..j+7], both 16-byte reads from row-major LDS tiles (pitch 72
// elements: conflict-free 16-byte row reads), and each lane ends with four consecutive i of one
// row r, stored as 16-byte words. Wave w owns the 64 x 64 quarter (i block w%2, r block w/2) as
// 2 x 2 tiles of v_mfma_f32_32x32x16_bf16. The k loop runs over 64-wide steps of j: C/64 steps
// of dQ (hi and lo products share the weight operand), then of dK, then of dV. Each step's tiles
// are loaded into registers during the previous step's products and written to LDS (dQ split on
// the way) between two barriers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attn_common.hpp"

namespace mla {

namespace {

constexpr int kGxTile = 128;        // rows and features per workgroup
constexpr int kGxK = 64;            // j per step
constexpr int kGxP = kGxK + 8;      // LDS row pitch (elements)
constexpr int kGxTileBytes = kGxTile * kGxP * 2;

__device__ __forceinline__ u32x4 lds_ld16(uint32_t a) { return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)a; }
__device__ __forceinline__ void lds_st16(uint32_t a, u32x4 v) { *(__attribute__((address_space(3))) u32x4*)(uintptr_t)a = v; }
__device__ __forceinline__ void lds_st8(uint32_t a, u32x2 v) { *(__attribute__((address_space(3))) u32x2*)(uintptr_t)a = v; }

__global__ void __launch_bounds__(256, 2) grad_dx_kernel(float* __restrict__ dX, const float* __restrict__ dQ,
                                                        const uint16_t* __restrict__ dK, const uint16_t* __restrict__ dV,
                                                        const uint16_t* __restrict__ Wq, const uint16_t* __restrict__ Wk,
                                                        const uint16_t* __restrict__ Wv, int C) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[3 * kGxTileBytes];  // W, G hi, G lo
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const int r0 = blockIdx.x * kGxTile, i0 = blockIdx.y * kGxTile;
  const int wi = wave & 1, wr = wave >> 1;
  const uint32_t sW = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)smem;
  const uint32_t sH = sW + kGxTileBytes, sL = sW + 2 * kGxTileBytes;
  const int nb = C / kGxK;  // steps per segment

  // Copy roles. bf16 tiles (128 rows x 64 j): thread t moves 16-byte chunks c = t + 256q, q < 4
  // (row c/8, chunk c%8). The fp32 dQ tile: chunks c = t + 256q, q < 8, of 4 floats (row c/16,
  // floats 4(c%16)..+3), split and written as 8-byte hi and lo words.
  u32x4 wreg[4], greg[4];
  f32x4 qreg[8];
  auto load_w = [&](const uint16_t* W, int j0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q, row = c >> 3, ch = c & 7;
      wreg[q] = *(const u32x4*)(W + (size_t)(i0 + row) * C + j0 + 8 * ch);
    }
  };
  auto load_g = [&](const uint16_t* G, int j0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q, row = c >> 3, ch = c & 7;
      greg[q] = *(const u32x4*)(G + (size_t)(r0 + row) * C + j0 + 8 * ch);
    }
  };
  auto load_q = [&](int j0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = tid + 256 * q, row = c >> 4, ch = c & 15;
      qreg[q] = *(const f32x4*)(dQ + (size_t)(r0 + row) * C + j0 + 4 * ch);
    }
  };
  auto store_w = [&]() {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q, row = c >> 3, ch = c & 7;
      lds_st16(sW + 2 * (row * kGxP + 8 * ch), wreg[q]);
    }
  };
  auto store_g = [&]() {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q, row = c >> 3, ch = c & 7;
      lds_st16(sH + 2 * (row * kGxP + 8 * ch), greg[q]);
    }
  };
  auto store_q = [&]() {  // hi = bf16(x), lo = bf16(x - hi)
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = tid + 256 * q, row = c >> 4, ch = c & 15;
      const f32x4 x = qreg[q];
      const uint32_t h01 = pack_bf16(x[0], x[1]), h23 = pack_bf16(x[2], x[3]);
      const uint32_t l01 = pack_bf16(x[0] - bf_lo(h01), x[1] - bf_hi(h01));
      const uint32_t l23 = pack_bf16(x[2] - bf_lo(h23), x[3] - bf_hi(h23));
      const uint32_t off = 2 * (row * kGxP + 4 * ch);
      lds_st8(sH + off, u32x2{h01, h23});
      lds_st8(sL + off, u32x2{l01, l23});
    }
  };

  // operand addresses: A = W row i (m), B = G row r (n); lane row l32, j = 16ks + 8h
  const uint32_t aoff = 2 * ((64 * wi + l32) * kGxP + 8 * h);
  const uint32_t boff = 2 * ((64 * wr + l32) * kGxP + 8 * h);
  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = zero16();
  // one 64-wide step of products from the staged tiles; TWO: dQ steps (hi and lo share A)
  auto compute = [&](auto two_tag) {
    constexpr bool TWO = decltype(two_tag)::value;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 A[2], Bh[2], Bl[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        A[t] = lds_ld16(sW + aoff + 2 * (32 * t * kGxP + 16 * ks));
        Bh[t] = lds_ld16(sH + boff + 2 * (32 * t * kGxP + 16 * ks));
        if (TWO) Bl[t] = lds_ld16(sL + boff + 2 * (32 * t * kGxP + 16 * ks));
      }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          acc[mi][ni] = mfma(A[mi], Bh[ni], acc[mi][ni]);
          if (TWO) acc[mi][ni] = mfma(A[mi], Bl[ni], acc[mi][ni]);
        }
    }
  };

  // dQ segment (Wq), its next tiles loaded during each step's products
  load_w(Wq, 0);
  load_q(0);
  store_w();
  store_q();
  __syncthreads();
  for (int b = 0; b < nb; ++b) {
    const bool last = b + 1 == nb;
    load_w(last ? Wk : Wq, last ? 0 : (b + 1) * kGxK);
    if (last) load_g(dK, 0);
    else load_q((b + 1) * kGxK);
    compute(std::true_type{});
    __syncthreads();  // every wave is done with this step's tiles
    store_w();
    if (last) store_g();
    else store_q();
    __syncthreads();
  }
  // dK segment (Wk), then dV (Wv)
  for (int b = 0; b < 2 * nb; ++b) {
    const int nxt = b + 1;
    const bool more = nxt < 2 * nb;
    if (more) {
      const bool v = nxt >= nb;
      load_w(v ? Wv : Wk, (v ? nxt - nb : nxt) * kGxK);
      load_g(v ? dV : dK, (v ? nxt - nb : nxt) * kGxK);
    }
    compute(std::false_type{});
    if (more) {
      __syncthreads();
      store_w();
      store_g();
      __syncthreads();
    }
  }

  // dX^T tile (mi, ni): lane holds row r = r0 + 64wr + 32ni + l32, features i0 + 64wi + 32mi +
  // 8g + 4h + (0..3) in registers 4g..4g+3
#pragma unroll
  for (int ni = 0; ni < 2; ++ni) {
    float* row = dX + (size_t)(r0 + 64 * wr + 32 * ni + l32) * C + i0 + 64 * wi + 4 * h;
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4* p = (f32x4*)(row + 32 * mi + 8 * g);
        const f32x4 v = f32x4{acc[mi][ni][4 * g], acc[mi][ni][4 * g + 1], acc[mi][ni][4 * g + 2], acc[mi][ni][4 * g + 3]};
        *p = *p + v;
      }
  }
}

}  // namespace

bool grad_dx_fused_ok(int R, int C) { return R % kGxTile == 0 && C % kGxTile == 0; }

hipError_t launch_grad_dx(float* dX, const float* dQ, const uint16_t* dK, const uint16_t* dV, const uint16_t* Wq,
                          const uint16_t* Wk, const uint16_t* Wv, int R, int C, hipStream_t s) {
  const dim3 grid((unsigned)(R / kGxTile), (unsigned)(C / kGxTile));
  hipLaunchKernelGGL(grad_dx_kernel, grid, dim3(256), 0, s, dX, dQ, dK, dV, Wq, Wk, Wv, C);
  return hipGetLastError();
}

}  // namespace mla
