// attn_fwd.hip -- flashAttentionForward on gfx950.
//
// Reference: /root/reference/attention.metal:56-164. Per (batch, head, query row):
//   S = bf16(Q.K^T)                      (:113, bf16 LDS tile)
//   s = bf16(S * scale + causal mask)    (:115-121; for D=64 scale is 0.125 and the second
//                                         rounding is exact, so it is skipped)
//   online softmax over 64-key tiles: m' = max(m, max s), a = exp(m - m'), e = exp(s - m'),
//   P = bf16(e), l' = l*a + sum e (unrounded), O = O*a + P.V   (:125-153)
//   out = bf16(O * (1/l)), lse = m + log(l)                    (:156-161)
//
// Work split: one workgroup of 4 waves owns 128 query rows of one (b,h); each wave owns 32
// rows and holds its Q rows as matrix-core B operands in registers for the whole kernel. Key/V
// tiles of 64 rows are double-buffered through LDS (swizzled, no padding); the next tile's
// global loads are issued before the current tile's math. Key tiles entirely above a wave's
// diagonal are skipped; only diagonal tiles apply the mask.
//
// Orientation: the wave computes S^T (keys x queries) so that lane = query column. Row
// statistics are then in-lane (16 values per 32-key subtile) plus one swap of the two lane
// halves; the S^T accumulator is directly the B operand (P^T) of O^T += V^T.P^T, whose A
// operand (V^T) comes from ds_read_b64_tr_b16 on the row-major V tile.
//
// Matrix-core passes, as the oracle models them: S sums d in passes of 8 consecutive values;
// P.V sums keys in passes {16c+0..3, 16c+8..11} then {16c+4..7, 16c+12..15}.
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

template <int D>
struct FwdCfg {
  static constexpr int BM = kFwdBlockM;        // query rows per workgroup
  static constexpr int BN = kTile;             // keys per tile
  static constexpr int THREADS = 256;
  static constexpr int TILE_ELEMS = BN * D;
  static constexpr int CH = D / 8;             // 16-byte chunks per row
  static constexpr int LOADS = BN * CH / THREADS;  // 16-byte loads per thread per tensor per tile
  static constexpr int KC = D / 16;            // 16-deep matrix-core steps over d
  static constexpr int DT = D / 32;            // 32-wide d tiles of the output
};

template <int D>
__global__ void __launch_bounds__(256) fwd_kernel(FwdArgs a) {
  using C = FwdCfg<D>;
  using Sw = SwzTile<D>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * 2 * C::TILE_ELEMS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int nqb = (a.T + C::BM - 1) / C::BM;
  int pair, qb;
  decode_workgroup(blockIdx.x, a.B * a.H, nqb, true, pair, qb);
  const int b = pair / a.H, hd = pair - b * a.H;
  const int rs = a.H * D;  // elements between consecutive tokens
  const size_t base = ((size_t)b * a.T * a.H + hd) * D;
  const uint16_t* Qg = a.q + base;
  const uint16_t* Kg = a.k + base;
  const uint16_t* Vg = a.v + base;

  const int q0 = qb * C::BM;
  const int qw = q0 + 32 * wave;  // this wave's first query row
  const bool wave_active = qw < a.T;
  const int q_end = min(q0 + C::BM, a.T);
  const int last_kt = (q_end - 1) / C::BN;
  const int q = qw + l32;  // this lane's query row

  // Q^T as B operands: lane holds Q[q][16c + 8h .. +7].
  u32x4 Qr[C::KC];
#pragma unroll
  for (int c = 0; c < C::KC; ++c) {
    if (wave_active)
      Qr[c] = *(const u32x4*)(Qg + (size_t)q * rs + 16 * c + 8 * h);
    else
      Qr[c] = u32x4{0, 0, 0, 0};
  }

  f32x16 O[C::DT];
#pragma unroll
  for (int i = 0; i < C::DT; ++i) O[i] = zero16();
  float m_run = -INFINITY, l_run = 0.0f;
  // Scores are carried in units u: s = x*su. For D=64, x = bf16(S) and su = 0.125 (exact);
  // for D=128, x = bf16(bf16(S)*scale) and su = 1.
  const float su = (D == 64) ? 0.125f : 1.0f;
  const float c1 = su * kLog2e;

  u32x4 kreg[C::LOADS], vreg[C::LOADS];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < C::LOADS; ++i) {
      const int idx = tid + i * C::THREADS, row = idx / C::CH, ch = idx % C::CH;
      const size_t g = (size_t)(kt * C::BN + row) * rs + ch * 8;
      kreg[i] = *(const u32x4*)(Kg + g);
      vreg[i] = *(const u32x4*)(Vg + g);
    }
  };
  auto lstore = [&](int stage) {
    uint16_t* Ks = smem + stage * 2 * C::TILE_ELEMS;
    uint16_t* Vs = Ks + C::TILE_ELEMS;
#pragma unroll
    for (int i = 0; i < C::LOADS; ++i) {
      const int idx = tid + i * C::THREADS, row = idx / C::CH, ch = idx % C::CH;
      *(u32x4*)(Ks + Sw::off(row, ch * 8)) = kreg[i];
      *(u32x4*)(Vs + Sw::off(row, ch * 8)) = vreg[i];
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();

  for (int kt = 0; kt <= last_kt; ++kt) {
    if (kt < last_kt) gload(kt + 1);
    const uint16_t* Ks = smem + (kt & 1) * 2 * C::TILE_ELEMS;
    const uint16_t* Vs = Ks + C::TILE_ELEMS;
    if (wave_active && kt * C::BN <= qw + 31) {
      // ---- S^T = K.Q^T for 64 keys (two 32-key subtiles) x 32 queries ----
      f32x16 S0 = zero16(), S1 = zero16();
#pragma unroll
      for (int c = 0; c < C::KC; ++c) {
        const u32x4 k0 = lds_read16(Ks + Sw::off(l32, 16 * c + 8 * h));
        const u32x4 k1 = lds_read16(Ks + Sw::off(32 + l32, 16 * c + 8 * h));
        S0 = mfma(k0, Qr[c], S0);
        S1 = mfma(k1, Qr[c], S1);
      }
      // ---- rounding points, mask, online softmax (lane = query q) ----
      float x[32];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        x[r] = S0[r];
        x[r + 1] = S0[r + 1];
        x[16 + r] = S1[r];
        x[16 + r + 1] = S1[r + 1];
      }
#pragma unroll
      for (int i = 0; i < 32; i += 2) {
        round_pair(x[i], x[i + 1]);
        if (D != 64) {
          x[i] *= a.scale;
          x[i + 1] *= a.scale;
          round_pair(x[i], x[i + 1]);
        }
      }
      if (kt * C::BN + C::BN - 1 > qw) {  // diagonal tile for this wave
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          const int r = i & 15;
          const int key = kt * C::BN + 32 * (i >> 4) + 8 * (r >> 2) + 4 * h + (r & 3);
          if (key > q) x[i] = -INFINITY;
        }
      }
      float mt = x[0];
#pragma unroll
      for (int i = 1; i < 32; ++i) mt = fmaxf(mt, x[i]);
      mt = max_halves(mt);
      const float m_new = fmaxf(m_run, mt);
      const float alpha = exp2_hw((m_run - m_new) * c1);
      const float mb = m_new * c1;
      l_run *= alpha;
      uint32_t P[16];
#pragma unroll
      for (int i = 0; i < 32; i += 2) {
        const float e0 = exp2_hw(fmaf(x[i], c1, -mb));
        const float e1 = exp2_hw(fmaf(x[i + 1], c1, -mb));
        l_run += e0;
        l_run += e1;
        P[i >> 1] = pack_bf16(e0, e1);
      }
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) O[dt][r] *= alpha;
      m_run = m_new;
      // ---- O^T += V^T . P^T ----
      const int cb = 16 * ((lane >> 4) & 1);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 Bp = {P[4 * c], P[4 * c + 1], P[4 * c + 2], P[4 * c + 3]};
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const u32x2 lo = lds_tr(tr_addr<D>(Vs, 16 * c + 4 * h, 32 * dt + cb, lane));
          const u32x2 hi = lds_tr(tr_addr<D>(Vs, 16 * c + 8 + 4 * h, 32 * dt + cb, lane));
          const u32x4 Av = {lo[0], lo[1], hi[0], hi[1]};
          O[dt] = mfma(Av, Bp, O[dt]);
        }
      }
    }
    if (kt < last_kt) lstore((kt + 1) & 1);
    __syncthreads();
  }

  if (!wave_active) return;
  // ---- epilogue: out = bf16(O * (1/l)), lse = m + log(l) ----
  const float lt = sum_halves(l_run);
  const float inv = 1.0f / lt;
  uint16_t* Og = a.out + base + (size_t)q * rs;
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * dt + 8 * g + 4 * h;
      u32x2 w;
      w[0] = pack_bf16(O[dt][4 * g] * inv, O[dt][4 * g + 1] * inv);
      w[1] = pack_bf16(O[dt][4 * g + 2] * inv, O[dt][4 * g + 3] * inv);
      *(u32x2*)(Og + d0) = w;
    }
  if (h == 0) a.lse[(size_t)pair * a.T + q] = m_run * su + logf(lt);
}

hipError_t launch_forward(const FwdArgs& a, int D, hipStream_t s) {
  const int nqb = (a.T + kFwdBlockM - 1) / kFwdBlockM;
  const dim3 grid((unsigned)(a.B * a.H * nqb));
  if (D == 64)
    hipLaunchKernelGGL(fwd_kernel<64>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(fwd_kernel<128>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace mla
