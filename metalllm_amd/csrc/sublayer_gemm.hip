// sublayer_gemm.hip -- hand-written matrix-core kernels for the two GEMMs of metalLLM's attention
// sublayer that read the fp32 dQ:
//   computeGradDx (/root/reference/attention.metal:301-341)  dX += dQ.Wq^T + dK.Wk^T + dV.Wv^T
//   computeGradDw (/root/reference/attention.metal:343-383)  dWq += X^T.dQ, dWk += X^T.dK, dWv += X^T.dV
// with dQ fp32, X, dK and dV bf16 [R, C], weights bf16 [C, C] indexed [input feature][output
// feature], dX and dWq fp32, dWk and dWv bf16; every destination is read once and written once.
//
// The reference reads the fp32 dQ directly (its matmul2d mixes the float dQ with bfloat weights
// into a float destination). Here both kernels load dQ as fp32 and split every element in
// registers into two bf16 terms, hi = bf16(x) and lo = bf16(x - hi) (|x - hi - lo| <= 2^-17 |x|),
// and run the product on both: the fp32 gradient reaches the matrix cores without a bf16 round
// trip and without a separate split pass through HBM.
//
// computeGradDx: all three products accumulate into one set of fp32 accumulators, so dX is read
// and written once instead of once per product. Tiling: a workgroup of 4 waves computes a 128
// (rows r) x FI (features i, FI = 128 or 192) tile of dX as
// dX^T = W . G^T (m = i, n = r, k = j): the A operand is a weight row W[i][j..j+7] and the B
// operand a gradient row G[r][j..j+7], both 16-byte reads from row-major LDS tiles (pitch 72
// elements: conflict-free 16-byte row reads), and each lane ends with four consecutive i of one
// row r, stored as 16-byte words. Wave w owns the FI/2 x 64 part (i block w%2, r block w/2) as
// FI/64 x 2 tiles of v_mfma_f32_32x32x16_bf16. The k loop runs over 64-wide steps of j: C/64 steps
// of dQ (hi and lo products share the weight operand), then of dK, then of dV. Each step's tiles
// are loaded into registers during the previous step's products and written to LDS (dQ split on
// the way) between two barriers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "attn_common.hpp"

namespace mla {

namespace {

constexpr int kGxTile = 128;        // rows per workgroup (and the smaller feature tile)
constexpr int kGxK = 64;            // j per step
constexpr int kGxP = kGxK + 8;      // LDS row pitch (elements)
constexpr int kGxTileBytes = kGxTile * kGxP * 2;

__device__ __forceinline__ u32x4 lds_ld16(uint32_t a) { return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)a; }
__device__ __forceinline__ void lds_st16(uint32_t a, u32x4 v) { *(__attribute__((address_space(3))) u32x4*)(uintptr_t)a = v; }
__device__ __forceinline__ void lds_st8(uint32_t a, u32x2 v) { *(__attribute__((address_space(3))) u32x2*)(uintptr_t)a = v; }

// ACC: dX += the products (the reference's contract); otherwise dX = 0 + the products, written
// without reading dX (the phase encoder, which would zero dX just before).
template <int FI>
constexpr int grad_dx_smem() { return FI * kGxP * 2 + 2 * kGxTileBytes; }  // W, G hi, G lo

// The kernel's body on the LDS at smem (grad_dx_smem<FI>() bytes), as workgroup bid of the grid.
template <bool ACC, int FI>
__device__ __forceinline__ void grad_dx_body(unsigned char* smem, int bid, float* __restrict__ dX,
                                             const float* __restrict__ dQ, const uint16_t* __restrict__ dK,
                                             const uint16_t* __restrict__ dV, const uint16_t* __restrict__ Wq,
                                             const uint16_t* __restrict__ Wk, const uint16_t* __restrict__ Wv, int C,
                                             int items) {
  static_assert(FI == 128 || FI == 192, "feature tile");
  constexpr int MI = FI / 64;                          // 32-wide i tiles per wave
  constexpr int WQ = FI / 32;                          // W tile chunks per thread
  constexpr int WBYTES = FI * kGxP * 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  // tile order: row block major, feature block minor. Workgroups are dealt to the 8 XCDs in turn
  // (blockIdx % 8); when 8 divides the tile count each XCD takes a contiguous range of tiles, so
  // the C/FI tiles that read the same gradient rows run together on one XCD and share its L2.
  const int nfb = C / FI;
  const int item = items % 8 == 0 ? (bid % 8) * (items / 8) + bid / 8 : bid;
  const int r0 = (item / nfb) * kGxTile, i0 = (item % nfb) * FI;
  const int wi = wave & 1, wr = wave >> 1;
  const uint32_t sW = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)smem;
  const uint32_t sH = sW + WBYTES, sL = sH + kGxTileBytes;
  const int nb = C / kGxK;  // steps per segment

  // Copy roles. bf16 tiles (128 or FI rows x 64 j): thread t moves 16-byte chunks c = t + 256q,
  // q < 4 (W: q < FI/32) (row c/8, chunk c%8). The fp32 dQ tile: chunks c = t + 256q, q < 8, of
  // 4 floats (row c/16, floats 4(c%16)..+3), split and written as 8-byte hi and lo words.
  u32x4 wreg[WQ], greg[4];
  f32x4 qreg[8];
  auto load_w = [&](const uint16_t* W, int j0) {
#pragma unroll
    for (int q = 0; q < WQ; ++q) {
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
    for (int q = 0; q < WQ; ++q) {
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
  const uint32_t aoff = 2 * ((FI / 2 * wi + l32) * kGxP + 8 * h);
  const uint32_t boff = 2 * ((64 * wr + l32) * kGxP + 8 * h);
  f32x16 acc[MI][2];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = zero16();
  // one 64-wide step of products from the staged tiles; TWO: dQ steps (hi and lo share A)
  auto compute = [&](auto two_tag) {
    constexpr bool TWO = decltype(two_tag)::value;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 A[MI], Bh[2], Bl[2];
#pragma unroll
      for (int t = 0; t < MI; ++t) A[t] = lds_ld16(sW + aoff + 2 * (32 * t * kGxP + 16 * ks));
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        Bh[t] = lds_ld16(sH + boff + 2 * (32 * t * kGxP + 16 * ks));
        if (TWO) Bl[t] = lds_ld16(sL + boff + 2 * (32 * t * kGxP + 16 * ks));
      }
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
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

  // dX^T tile (mi, ni): lane holds row r = r0 + 64wr + 32ni + l32, features i0 + (FI/2)wi + 32mi +
  // 8g + 4h + (0..3) in registers 4g..4g+3
#pragma unroll
  for (int ni = 0; ni < 2; ++ni) {
    float* row = dX + (size_t)(r0 + 64 * wr + 32 * ni + l32) * C + i0 + FI / 2 * wi + 4 * h;
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4* p = (f32x4*)(row + 32 * mi + 8 * g);
        const f32x4 v = f32x4{acc[mi][ni][4 * g], acc[mi][ni][4 * g + 1], acc[mi][ni][4 * g + 2], acc[mi][ni][4 * g + 3]};
        if (ACC)
          *p = *p + v;
        else
          *p = v + 0.0f;  // bit for bit 0 + v (-0 becomes +0)
      }
  }
}

template <bool ACC, int FI>
__global__ void __launch_bounds__(256, 2) grad_dx_kernel(float* __restrict__ dX, const float* __restrict__ dQ,
                                                        const uint16_t* __restrict__ dK, const uint16_t* __restrict__ dV,
                                                        const uint16_t* __restrict__ Wq, const uint16_t* __restrict__ Wk,
                                                        const uint16_t* __restrict__ Wv, int C, int items) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[grad_dx_smem<FI>()];
  grad_dx_body<ACC, FI>(smem, (int)blockIdx.x, dX, dQ, dK, dV, Wq, Wk, Wv, C, items);
}

// ---- computeGradDw (attention.metal:343-383): dWq += X^T.dQ (fp32), dKw += X^T.dK, dVw += X^T.dV
// (bf16), X bf16 [R, C], dQ fp32, dK and dV bf16 [R, C]; the sums run over all R rows into C x C
// outputs, too few tiles to fill the chip, so the rows are split into chunks. A work item is one
// tile (128 output features j x FI input features i) of one weight over one chunk of rows,
// written as an fp32 partial; dWq items run two products per row (hi and lo of dQ, split in
// registers as in grad_dx_kernel), and the chunk counts of dWq and of dKw/dVw are chosen so that
// the two kinds of item carry nearly the same matrix-core work (grad_dw_shape).
// grad_dw_reduce_kernel then adds the partials and the destination's previous value once and
// rounds once. projBackwarddW (attention.metal:407-430, dProjw += attn_out^T.dZ) runs the same
// kernel with one bf16 weight (grad_dw_one_shape), and the phase encoder adds it to
// computeGradDw's items as a fourth weight (Xp = attn_out, Gp = dZ; launch_grad_dxdw4).
//
// Operands: the tile is computed transposed, W^T = G^T . X (m = j, n = i, k = r), so each lane
// ends with four consecutive j of one i, stored as 16-byte words of the row-major partial. Both
// operands need 8 rows r of one column per lane: they come from row-major LDS tiles [r][128 or FI
// columns] by ds_read_b64_tr_b16 (pitch 160 or FI + 32 elements: the 4 rows x 64 bytes read by 32
// lanes of one transposing read fall in distinct banks).
constexpr int kGwTile = 128;                     // output features j per tile (and the narrower i width)
constexpr int kGwK = 64;                         // rows r per step
constexpr int kGwP = kGwTile + 32;               // LDS row pitch of a 128-column tile (elements)
constexpr int kGwTileBytes = kGwK * kGwP * 2;    // 20 KB

__device__ __forceinline__ u32x2 lds_tr8(uint32_t a) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(uintptr_t)a));
}

struct GwShape {
  int C, nti, ntj;  // features; tiles along i (FI wide) and along j (128 wide)
  int steps;        // R / kGwK
  int nq, nkv;      // row chunks of dWq, and of each bf16 weight (dKw, dVw, and dPw when fused)
  int items;        // tiles (nq + nb nkv), nb bf16 weights
  // XCD deal (0 in lx: workgroup order): XCD x takes items long0 + x lx + k for k < lx, then
  // short0 + x sx + (k - lx)
  int lx, sx, long0, short0;
};

// Work items in order (weight, chunk, i block, j block): dWq's, then dKw's, then dVw's, then (the
// phase encoder's fused form) dPw's, the projection weight's gradient Xp^T . Gp.
// Workgroups are dealt to the 8 XCDs in turn (blockIdx % 8, workgroup k of an XCD is blockIdx / 8).
// When 8 divides the item count of each kind, each XCD takes a contiguous range of the longer
// kind's items first (the kind with more products per item: dWq's or the bf16 weights'), then a
// contiguous range of the other kind's: the items that share a chunk's rows run on one XCD and
// share its L2, and an XCD's first workgroups, which start one on each CU, carry the long items,
// so that a CU's second workgroup is a short one.
template <int FI>
constexpr int grad_dw_smem() { return kGwK * (FI + 32) * 2 + 2 * kGwTileBytes; }  // X, G (dQ hi), dQ lo

template <int FI>
__device__ __forceinline__ void grad_dw_body(unsigned char* smem, int bid, const uint16_t* __restrict__ X,
                                             const float* __restrict__ dQ, const uint16_t* __restrict__ dK,
                                             const uint16_t* __restrict__ dV, const uint16_t* __restrict__ Xp,
                                             const uint16_t* __restrict__ Gp, float* __restrict__ part, const GwShape& sh) {
  static_assert(FI == 128 || FI == 192, "input-feature tile");
  constexpr int NI = FI / 64;                 // 32-wide i tiles per wave
  constexpr int XQ = FI / 32;                 // X tile chunks per thread
  constexpr int XCH = FI / 8;                 // 16-byte chunks per X row
  constexpr int XP = FI + 32;                 // X tile pitch (elements)
  constexpr int XBYTES = kGwK * XP * 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31, g16 = lane >> 4, s16 = lane & 15;
  const int C = sh.C, tiles = sh.nti * sh.ntj;
  int item = bid;
  if (sh.lx) {
    const int x = bid % 8, k = bid / 8;
    item = k < sh.lx ? sh.long0 + x * sh.lx + k : sh.short0 + x * sh.sx + (k - sh.lx);
  }
  int wsel = 0, nch = sh.nq, pbase = 0;
  if (item >= tiles * sh.nq) {
    item -= tiles * sh.nq;
    wsel = 1 + item / (tiles * sh.nkv);
    item -= (wsel - 1) * tiles * sh.nkv;
    nch = sh.nkv;
    pbase = sh.nq + (wsel - 1) * sh.nkv;
  }
  const int chunk = item / tiles, tile = item - chunk * tiles;
  const int i0 = (tile / sh.ntj) * FI, j0 = (tile % sh.ntj) * kGwTile;
  const int s0 = (int)((long)chunk * sh.steps / nch), s1 = (int)((long)(chunk + 1) * sh.steps / nch);
  const uint16_t* G = wsel == 1 ? dK : (wsel == 2 ? dV : Gp);
  const uint16_t* Xs = wsel == 3 ? Xp : X;
  const int wi = wave & 1, wj = wave >> 1;
  const uint32_t sX = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)smem;
  const uint32_t sH = sX + XBYTES, sL = sH + kGwTileBytes;

  // copies of a step's tiles (64 rows): bf16 G, c = t + 256q, q < 4: row c/16, 16-byte chunk c%16
  // (X: q < FI/32, row c/(FI/8), chunk c%(FI/8)); fp32 dQ, c = t + 256q, q < 8: row c/32, floats
  // 4(c%32)..+3
  u32x4 xreg[XQ], greg[4];
  f32x4 qreg[8];
  auto load_x = [&](int r) {
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int c = tid + 256 * q;
      xreg[q] = *(const u32x4*)(Xs + (size_t)(r + c / XCH) * C + i0 + 8 * (c % XCH));
    }
  };
  auto load_g = [&](int r) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q;
      greg[q] = *(const u32x4*)(G + (size_t)(r + (c >> 4)) * C + j0 + 8 * (c & 15));
    }
  };
  auto load_q = [&](int r) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = tid + 256 * q;
      qreg[q] = *(const f32x4*)(dQ + (size_t)(r + (c >> 5)) * C + j0 + 4 * (c & 31));
    }
  };
  auto store_x = [&]() {
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      const int c = tid + 256 * q;
      lds_st16(sX + 2 * ((c / XCH) * XP + 8 * (c % XCH)), xreg[q]);
    }
  };
  auto store_g = [&]() {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q;
      lds_st16(sH + 2 * ((c >> 4) * kGwP + 8 * (c & 15)), greg[q]);
    }
  };
  auto store_q = [&]() {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int c = tid + 256 * q;
      const f32x4 x = qreg[q];
      const uint32_t h01 = pack_bf16(x[0], x[1]), h23 = pack_bf16(x[2], x[3]);
      const uint32_t l01 = pack_bf16(x[0] - bf_lo(h01), x[1] - bf_hi(h01));
      const uint32_t l23 = pack_bf16(x[2] - bf_lo(h23), x[3] - bf_hi(h23));
      const uint32_t off = 2 * ((c >> 5) * kGwP + 4 * (c & 31));
      lds_st8(sH + off, u32x2{h01, h23});
      lds_st8(sL + off, u32x2{l01, l23});
    }
  };

  // transposing reads of a 32-column block: source lane s16 of group g16 addresses row
  // 4h + s16/4 (+8 for the second read, +16 per k step), column 16(g16%2) + 4(s16%4); the lane
  // receives column l32 of the block at rows {4h..4h+3, 8+4h..8+4h+3}, the same rows for both
  // operands. Both pitches (160 and FI + 32 elements) put the 4 rows x 64 bytes that 32 lanes
  // of one read touch in distinct banks.
  auto tr_op = [&](auto pitch_tag, uint32_t base, int col0, int ks) -> u32x4 {
    constexpr int PP = decltype(pitch_tag)::value;
    const uint32_t tr = 2 * ((4 * h + (s16 >> 2)) * PP + 16 * (g16 & 1) + 4 * (s16 & 3));
    const uint32_t a = base + tr + 2 * (16 * ks * PP + col0);
    const u32x2 lo = lds_tr8(a), hi = lds_tr8(a + 2 * 8 * PP);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  using PX = std::integral_constant<int, XP>;
  using PG = std::integral_constant<int, kGwP>;
  // acc[mj][ni]: W^T block (j = 64 wj + 32 mj, i = (FI/2) wi + 32 ni)
  f32x16 acc[2][NI];
#pragma unroll
  for (int mj = 0; mj < 2; ++mj)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mj][ni] = zero16();
  auto compute = [&](auto two_tag) {
    constexpr bool TWO = decltype(two_tag)::value;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 Bx[NI], Ah[2], Al[2];
#pragma unroll
      for (int t = 0; t < NI; ++t) Bx[t] = tr_op(PX{}, sX, FI / 2 * wi + 32 * t, ks);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        Ah[t] = tr_op(PG{}, sH, 64 * wj + 32 * t, ks);
        if (TWO) Al[t] = tr_op(PG{}, sL, 64 * wj + 32 * t, ks);
      }
#pragma unroll
      for (int mj = 0; mj < 2; ++mj)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
          acc[mj][ni] = mfma(Ah[mj], Bx[ni], acc[mj][ni]);
          if (TWO) acc[mj][ni] = mfma(Al[mj], Bx[ni], acc[mj][ni]);
        }
    }
  };
  auto run = [&](auto two_tag) {
    constexpr bool TWO = decltype(two_tag)::value;
    load_x(s0 * kGwK);
    if (TWO) load_q(s0 * kGwK);
    else load_g(s0 * kGwK);
    store_x();
    if (TWO) store_q();
    else store_g();
    __syncthreads();
    for (int s = s0; s < s1; ++s) {
      const bool more = s + 1 < s1;
      if (more) {
        load_x((s + 1) * kGwK);
        if (TWO) load_q((s + 1) * kGwK);
        else load_g((s + 1) * kGwK);
      }
      compute(two_tag);
      if (more) {
        __syncthreads();
        store_x();
        if (TWO) store_q();
        else store_g();
        __syncthreads();
      }
    }
  };
  if (wsel == 0) run(std::true_type{});
  else run(std::false_type{});

  // lane: i = i0 + (FI/2) wi + 32 ni + l32, j = j0 + 64 wj + 32 mj + 8g + 4h + (0..3)
  float* dst = part + (size_t)(pbase + chunk) * C * C;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    float* row = dst + (size_t)(i0 + FI / 2 * wi + 32 * ni + l32) * C + j0 + 64 * wj + 4 * h;
#pragma unroll
    for (int mj = 0; mj < 2; ++mj)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(f32x4*)(row + 32 * mj + 8 * g) =
            f32x4{acc[mj][ni][4 * g], acc[mj][ni][4 * g + 1], acc[mj][ni][4 * g + 2], acc[mj][ni][4 * g + 3]};
  }
}

template <int FI>
__global__ void __launch_bounds__(256, 2) grad_dw_kernel(const uint16_t* __restrict__ X, const float* __restrict__ dQ,
                                                        const uint16_t* __restrict__ dK, const uint16_t* __restrict__ dV,
                                                        const uint16_t* __restrict__ Xp, const uint16_t* __restrict__ Gp,
                                                        float* __restrict__ part, GwShape sh) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[grad_dw_smem<FI>()];
  grad_dw_body<FI>(smem, (int)blockIdx.x, X, dQ, dK, dV, Xp, Gp, part, sh);
}

// computeGradDx (written, not accumulated) and the four-weight computeGradDw in one launch (the
// phase encoder): workgroups [0, nx) take computeGradDx's items and the rest computeGradDw's, so
// that the weight-gradient items start on the CUs whose dX tiles are done while the other dX
// tiles' stores drain. Where 8 divides nx both parts keep their XCD deal (else only their L2
// sharing changes, not the results).
template <int FI>
__global__ void __launch_bounds__(256, 2) grad_dxdw_kernel(float* __restrict__ dX, const uint16_t* __restrict__ X,
                                                          const float* __restrict__ dQ, const uint16_t* __restrict__ dK,
                                                          const uint16_t* __restrict__ dV, const uint16_t* __restrict__ Wq,
                                                          const uint16_t* __restrict__ Wk, const uint16_t* __restrict__ Wv,
                                                          const uint16_t* __restrict__ Xp, const uint16_t* __restrict__ Gp,
                                                          float* __restrict__ part, int nx, GwShape sh) {
  constexpr int SM = grad_dx_smem<FI>() > grad_dw_smem<FI>() ? grad_dx_smem<FI>() : grad_dw_smem<FI>();
  __shared__ __attribute__((aligned(1024))) unsigned char smem[SM];
  const int bid = (int)blockIdx.x;
  if (bid < nx) grad_dx_body<false, FI>(smem, bid, dX, dQ, dK, dV, Wq, Wk, Wv, sh.C, nx);
  else grad_dw_body<FI>(smem, bid - nx, X, dQ, dK, dV, Xp, Gp, part, sh);
}

// dQw += the sum of its nq partials (fp32, in chunk order); dKw, dVw, dPw = bf16(previous + the
// sum of their nkv partials). Partials [nq + nb nkv][C][C]; four consecutive elements per thread.
// Only the weights w0 .. w0 + nw - 1 (0 dQw, 1 dKw, 2 dVw, 3 dPw) are reduced. Without acc the
// destinations are written as if they held zeros (bit for bit 0 + sum), and not read.
__global__ void __launch_bounds__(256) grad_dw_reduce_kernel(const float* __restrict__ part, float* __restrict__ dQw,
                                                               uint16_t* __restrict__ dKw, uint16_t* __restrict__ dVw,
                                                               uint16_t* __restrict__ dPw, int C, int nq, int nkv, int w0,
                                                               int nw, bool acc_dst) {
  const size_t cc = (size_t)C * C, n4 = cc / 4;
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < nw * n4; e += (size_t)gridDim.x * blockDim.x) {
    const int w = w0 + (int)(e / n4);
    const size_t o = 4 * (e - (size_t)(w - w0) * n4);
    const int p0 = w == 0 ? 0 : nq + (w - 1) * nkv, np = w == 0 ? nq : nkv;
    f32x4 acc = *(const f32x4*)(part + (size_t)p0 * cc + o);
    // unrolled so that several partials' loads are in flight; the adds stay in chunk order
#pragma unroll 4
    for (int p = 1; p < np; ++p) acc += *(const f32x4*)(part + (size_t)(p0 + p) * cc + o);
    if (w == 0) {
      f32x4* d = (f32x4*)(dQw + o);
      *d = (acc_dst ? *d : f32x4{0.0f, 0.0f, 0.0f, 0.0f}) + acc;
    } else {
      u32x2* d = (u32x2*)((w == 1 ? dKw : (w == 2 ? dVw : dPw)) + o);
      const u32x2 old = acc_dst ? *d : u32x2{0u, 0u};
      *d = u32x2{pack_bf16(bf_lo(old[0]) + acc[0], bf_hi(old[0]) + acc[1]),
                 pack_bf16(bf_lo(old[1]) + acc[2], bf_hi(old[1]) + acc[3])};
    }
  }
}

// The XCD deal of GwShape for nq_items dWq items (first in item order) and kv_items items of the
// bf16 weights; q_long: dWq's items carry more products than the others'.
void deal(GwShape& sh, int nq_items, int kv_items, bool q_long) {
  sh.lx = sh.sx = sh.long0 = sh.short0 = 0;
  if (nq_items % 8 || kv_items % 8) return;
  sh.lx = (q_long ? nq_items : kv_items) / 8;
  sh.sx = (q_long ? kv_items : nq_items) / 8;
  sh.long0 = q_long ? 0 : nq_items;
  sh.short0 = q_long ? nq_items : 0;
}

// Input-feature tile of computeGradDw: 192 where it divides C (36 -> 24 tiles at C = 768, with
// fewer operand reads per product), else 128. projBackwarddW's one-weight launch keeps 128: with
// 24 tiles its row chunks would be a third shorter, and it measured slower.
int gw_fi(int C) { return C % 192 == 0 ? 192 : 128; }

// nb bf16 weights beside dWq: 2 (computeGradDw) or 3 (with dPw, the phase encoder's fused form)
GwShape grad_dw_shape(int R, int C, int cus, int nb = 2) {
  GwShape sh;
  sh.C = C;
  sh.nti = C / gw_fi(C);
  sh.ntj = C / kGwTile;
  sh.steps = R / kGwK;
  const int tiles = sh.nti * sh.ntj;
  // as many items per tile as fill one round of two workgroups per CU (k), split so that a dWq
  // item (2 steps / nq products per row step) and a bf16-weight item (steps / nkv) are as close as
  // k allows (nq near 2 nkv): at C = 768 on 256 CUs, k = 21: nq 11, nkv 5 (504 items, 47 and 51
  // product-steps); with dPw nq 9, nkv 4 (504 items, 57 and 64)
  const int k = std::max(2 + nb, 2 * cus / tiles);
  sh.nkv = std::max(1, std::min((k + 2) / (2 + nb), sh.steps / 2));
  sh.nq = std::max(1, std::min(k - nb * sh.nkv, sh.steps));
  sh.items = tiles * (sh.nq + nb * sh.nkv);
  deal(sh, tiles * sh.nq, nb * tiles * sh.nkv, 2 * sh.nkv > sh.nq);
  return sh;
}

// One bf16 gradient (projBackwarddW): no dWq items, every item takes the dKw path with G = dZ; as
// many row chunks as fill one round of two workgroups per CU.
GwShape grad_dw_one_shape(int R, int C, int cus) {
  GwShape sh;
  sh.C = C;
  sh.nti = C / kGwTile;
  sh.ntj = C / kGwTile;
  sh.steps = R / kGwK;
  const int tiles = sh.nti * sh.ntj;
  sh.nq = 0;
  sh.nkv = std::max(1, std::min(2 * cus / tiles, sh.steps / 2));
  sh.items = tiles * sh.nkv;
  deal(sh, 0, sh.items, false);
  return sh;
}

int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return 256;
  return cus;
}

}  // namespace

bool grad_dx_fused_ok(int R, int C) { return R % kGxTile == 0 && C % kGxTile == 0; }

bool grad_dw_fused_ok(int R, int C) { return R % (2 * kGwK) == 0 && C % kGwTile == 0; }

// Partial floats launch_grad_dw needs for R x C on the current device (the chunk counts follow
// its compute-unit count).
size_t grad_dw_partial_floats(int R, int C) {
  const GwShape sh = grad_dw_shape(R, C, device_cus());
  return (size_t)(sh.nq + 2 * sh.nkv) * C * C;
}

hipError_t launch_grad_dw(const uint16_t* X, const float* dQ, const uint16_t* dK, const uint16_t* dV, float* dQw,
                          uint16_t* dKw, uint16_t* dVw, float* partial, int R, int C, bool accumulate, hipStream_t s) {
  const GwShape sh = grad_dw_shape(R, C, device_cus());
  hipLaunchKernelGGL(gw_fi(C) == 192 ? grad_dw_kernel<192> : grad_dw_kernel<128>, dim3((unsigned)sh.items), dim3(256), 0,
                     s, X, dQ, dK, dV, nullptr, nullptr, partial, sh);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t n4 = 3 * (size_t)C * C / 4;
  hipLaunchKernelGGL(grad_dw_reduce_kernel, dim3((unsigned)std::min<size_t>((n4 + 255) / 256, 4096)), dim3(256), 0, s,
                     partial, dQw, dKw, dVw, nullptr, C, sh.nq, sh.nkv, 0, 3, accumulate);
  return hipGetLastError();
}

// Partial floats of the phase encoder's four-weight form (computeGradDw with projBackwarddW's
// dPw = Xp^T . Gp, attn_out^T . dZ, as a fourth weight; launch_grad_dxdw4).
size_t grad_dw4_partial_floats(int R, int C) {
  const GwShape sh = grad_dw_shape(R, C, device_cus(), 3);
  return (size_t)(sh.nq + 3 * sh.nkv) * C * C;
}

// The phase encoder's computeGradDx (dX written) and four-weight computeGradDw in one launch,
// then the reduction of the four weights; computeGradDx's tiles as launch_grad_dx's and the
// weight-gradient items of grad_dw_shape with three bf16 weights (feature tiles of the same width:
// 192 where it divides C, else 128).
hipError_t launch_grad_dxdw4(float* dX, const uint16_t* X, const float* dQ, const uint16_t* dK, const uint16_t* dV,
                             const uint16_t* Wq, const uint16_t* Wk, const uint16_t* Wv, const uint16_t* Xp,
                             const uint16_t* Gp, float* dQw, uint16_t* dKw, uint16_t* dVw, uint16_t* dPw, float* partial,
                             int R, int C, hipStream_t s) {
  const GwShape sh = grad_dw_shape(R, C, device_cus(), 3);
  const bool wide = gw_fi(C) == 192;
  const int nx = (R / kGxTile) * (C / (wide ? 192 : 128));
  hipLaunchKernelGGL(wide ? grad_dxdw_kernel<192> : grad_dxdw_kernel<128>, dim3((unsigned)(nx + sh.items)), dim3(256), 0,
                     s, dX, X, dQ, dK, dV, Wq, Wk, Wv, Xp, Gp, partial, nx, sh);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t n4 = 4 * (size_t)C * C / 4;
  hipLaunchKernelGGL(grad_dw_reduce_kernel, dim3((unsigned)std::min<size_t>((n4 + 255) / 256, 4096)), dim3(256), 0, s,
                     partial, dQw, dKw, dVw, dPw, C, sh.nq, sh.nkv, 0, 4, false);
  return hipGetLastError();
}

size_t grad_dw_one_partial_floats(int R, int C) {
  const GwShape sh = grad_dw_one_shape(R, C, device_cus());
  return (size_t)sh.nkv * C * C;
}

hipError_t launch_grad_dw_one(const uint16_t* X, const uint16_t* G, uint16_t* dW, float* partial, int R, int C,
                              bool accumulate, hipStream_t s) {
  const GwShape sh = grad_dw_one_shape(R, C, device_cus());
  hipLaunchKernelGGL(grad_dw_kernel<128>, dim3((unsigned)sh.items), dim3(256), 0, s, X, nullptr, G, G, nullptr, nullptr,
                     partial, sh);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const size_t n4 = (size_t)C * C / 4;
  hipLaunchKernelGGL(grad_dw_reduce_kernel, dim3((unsigned)std::min<size_t>((n4 + 255) / 256, 4096)), dim3(256), 0, s,
                     partial, nullptr, dW, nullptr, nullptr, C, 0, sh.nkv, 1, 1, accumulate);
  return hipGetLastError();
}

// Feature tile: 192 where it divides C (config 4's C = 768: 512 tiles of 128 x 192 fill one round
// of two workgroups per CU, where 768 tiles of 128 x 128 took a round and a half), else 128.
hipError_t launch_grad_dx(float* dX, const float* dQ, const uint16_t* dK, const uint16_t* dV, const uint16_t* Wq,
                          const uint16_t* Wk, const uint16_t* Wv, int R, int C, bool accumulate, hipStream_t s) {
  const bool wide = C % 192 == 0;
  const int items = (R / kGxTile) * (C / (wide ? 192 : 128));
  auto kern = wide ? (accumulate ? grad_dx_kernel<true, 192> : grad_dx_kernel<false, 192>)
                   : (accumulate ? grad_dx_kernel<true, 128> : grad_dx_kernel<false, 128>);
  hipLaunchKernelGGL(kern, dim3((unsigned)items), dim3(256), 0, s, dX, dQ, dK, dV, Wq, Wk, Wv, C, items);
  return hipGetLastError();
}

}  // namespace mla
