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
// rows and holds its Q rows as matrix-core B operands in registers. Key tiles of 64 rows are
// double-buffered through LDS: K row-major ([key][d], pitch D+8) and V transposed ([d][key],
// pitch 72), so every matrix-core operand read is one conflict-free 16-byte ds_read at a
// per-lane base plus a compile-time offset. The next tile's global loads are issued before the
// current tile's math; key tiles entirely above a wave's diagonal are skipped and only
// diagonal tiles apply the mask. The O rescale is skipped when no row's running max moved
// (the factor is then exactly 1).
//
// Orientation: the wave computes S^T (keys x queries) so that lane = query column. Row
// statistics are in-lane (16 values per 32-key subtile) plus one exchange between the two lane
// halves; the S^T accumulator is directly the B operand (P^T) of O^T += V^T.P^T. Lane half h of
// a 32-key subtile holds keys {8g + 4h + i}; the transposed V tile stores each 16-key chunk in
// the order {0-3, 8-11, 4-7, 12-15} so that those 8 keys are one contiguous 16-byte read.
//
// Matrix-core passes, as the oracle models them: S sums d in passes of 8 consecutive values;
// P.V sums keys in passes {16c+0..3, 16c+8..11} then {16c+4..7, 16c+12..15}.
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

template <int D>
struct FwdCfg {
  static constexpr int BM = kFwdBlockM;  // query rows per workgroup
  static constexpr int BN = kTile;       // keys per tile
  static constexpr int THREADS = 256;
  static constexpr int KP = D + 8;       // K tile pitch (elements): 16-row column reads hit distinct banks
  static constexpr int VP = BN + 8;      // transposed V tile pitch
  static constexpr int K_ELEMS = BN * KP;
  static constexpr int V_ELEMS = D * VP;
  static constexpr int STAGE = K_ELEMS + V_ELEMS;
  static constexpr int CH = D / 8;                 // 16-byte chunks per row
  static constexpr int KLOADS = BN * CH / THREADS;  // 16-byte K loads per thread per tile
  static constexpr int VKEYS = D / 32;             // keys per thread in the V transpose (4 or 2)
  static constexpr int VGROUPS = BN / VKEYS;       // key groups across threads (16 or 32)
  static constexpr int KC = D / 16;                // 16-deep matrix-core steps over d
  static constexpr int DT = D / 32;                // 32-wide d tiles of the output
};

// Position of key k (0..63) inside a transposed-tile row: chunk of 16 keys, stored in the
// order {0-3, 8-11, 4-7, 12-15}.
__device__ __forceinline__ int perm_pos(int k) {
  return (k & ~15) + 8 * ((k >> 2) & 1) + 4 * ((k >> 3) & 1) + (k & 3);
}

// {lo16(a), lo16(b)} and {hi16(a), hi16(b)}
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

template <int D>
__global__ void __launch_bounds__(256, 2) fwd_kernel(FwdArgs a) {
  using C = FwdCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * C::STAGE];

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

  // ---- tile loaders: K rows as 16-byte chunks; V as VKEYS keys x 8 d per thread ----
  const int vg = tid / C::VGROUPS;           // d group: d = 8vg .. 8vg+7
  const int vk = (tid % C::VGROUPS) * C::VKEYS;  // first key of this thread's group
  u32x4 kreg[C::KLOADS], vreg[C::VKEYS];
  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < C::KLOADS; ++i) {
      const int idx = tid + i * C::THREADS, row = idx / C::CH, ch = idx % C::CH;
      kreg[i] = *(const u32x4*)(Kg + (size_t)(kt * C::BN + row) * rs + ch * 8);
    }
#pragma unroll
    for (int i = 0; i < C::VKEYS; ++i) vreg[i] = *(const u32x4*)(Vg + (size_t)(kt * C::BN + vk + i) * rs + 8 * vg);
  };
  auto lstore = [&](int stage) {
    uint16_t* Ks = smem + stage * C::STAGE;
    uint16_t* Vt = Ks + C::K_ELEMS;
#pragma unroll
    for (int i = 0; i < C::KLOADS; ++i) {
      const int idx = tid + i * C::THREADS, row = idx / C::CH, ch = idx % C::CH;
      *(u32x4*)(Ks + row * C::KP + ch * 8) = kreg[i];
    }
    uint16_t* vrow = Vt + 8 * vg * C::VP + perm_pos(vk);
#pragma unroll
    for (int j = 0; j < 8; ++j) {  // d = 8vg + j
      const int w = j >> 1;
      if (C::VKEYS == 4) {
        u32x2 o;
        o[0] = (j & 1) ? pack_hi(vreg[0][w], vreg[1][w]) : pack_lo(vreg[0][w], vreg[1][w]);
        o[1] = (j & 1) ? pack_hi(vreg[2][w], vreg[3][w]) : pack_lo(vreg[2][w], vreg[3][w]);
        *(u32x2*)(vrow + j * C::VP) = o;
      } else {
        *(uint32_t*)(vrow + j * C::VP) = (j & 1) ? pack_hi(vreg[0][w], vreg[1][w]) : pack_lo(vreg[0][w], vreg[1][w]);
      }
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();

  for (int kt = 0; kt <= last_kt; ++kt) {
    if (kt < last_kt) gload(kt + 1);
    const uint16_t* Ks = smem + (kt & 1) * C::STAGE;
    const uint16_t* Vt = Ks + C::K_ELEMS;
    if (wave_active && kt * C::BN <= qw + 31) {
      // ---- S^T = K.Q^T for 64 keys (two 32-key subtiles) x 32 queries ----
      const uint16_t* kb = Ks + l32 * C::KP + 8 * h;
      f32x16 S0 = zero16(), S1 = zero16();
#pragma unroll
      for (int c = 0; c < C::KC; ++c) {
        S0 = mfma(lds_read16(kb + 16 * c), Qr[c], S0);
        S1 = mfma(lds_read16(kb + 32 * C::KP + 16 * c), Qr[c], S1);
      }
      // ---- rounding points, mask, online softmax (lane = query q) ----
      float x[32];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x[r] = S0[r];
        x[16 + r] = S1[r];
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
      uint32_t P[16];
      float ls = 0.0f;
#pragma unroll
      for (int i = 0; i < 32; i += 2) {
        const float e0 = exp2_hw(fmaf(x[i], c1, -mb));
        const float e1 = exp2_hw(fmaf(x[i + 1], c1, -mb));
        ls += e0;
        ls += e1;
        P[i >> 1] = pack_bf16(e0, e1);
      }
      l_run = l_run * alpha + ls;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) O[dt][r] *= alpha;
      }
      m_run = m_new;
      // ---- O^T += V^T . P^T ----
      const uint16_t* vb = Vt + l32 * C::VP + 8 * h;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 Bp = {P[4 * c], P[4 * c + 1], P[4 * c + 2], P[4 * c + 3]};
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) O[dt] = mfma(lds_read16(vb + 32 * dt * C::VP + 16 * c), Bp, O[dt]);
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
