// attn_bwd.hip -- flashAttentionBackward on gfx950.
//
// Reference: /root/reference/attention.metal:198-299. For each 64-key tile kt and each 64-row
// query tile qt >= kt:
//   dP = bf16(dO.V^T), S = bf16(Q.K^T)                           (:274-275)
//   p = exp(S*scale - lse[q]), p = 0 where key > q (diagonal), P = bf16(p)
//   dS = bf16(p * (dP - D[q]) * scale)                            (:277-286)
//   dQ[qt rows] += bf16(dS.K)        (fp32 atomic add, :288,292-296)
//   dK = bf16(dK + dS^T.Q), dV = bf16(dV + P^T.dO)   once per query tile (:289-290)
// The key-tile owner accumulates dK/dV race-free; only dQ is shared, through fp32 atomics.
//
// Work split: one workgroup of 4 waves owns 128 keys (two reference key tiles) of one (b,h);
// wave w owns keys 32w..32w+31 and keeps their K and V rows in registers as matrix-core B
// operands, plus fp32 dK^T/dV^T accumulators rounded to bf16 after every 64-row query block
// (the reference's rounding points). K is also staged once, transposed, for the dQ product.
// Per 64-row query block the workgroup stages Q and dO twice -- row-major [q][d] and transposed
// [d][q] -- plus lse and D, so that every matrix-core operand is one conflict-free 16-byte LDS
// read at a per-lane base plus a compile-time offset. Each wave computes S and dP for its keys
// one 32-row subtile at a time (lane = key), forms P and dS in registers, stores dS as [q][key],
// and updates dV^T/dK^T (A operands from the transposed tiles). After a barrier each wave
// computes its share of the dQ block [64 q][D] from dS and the transposed K, one bf16-rounded
// part per reference key tile, and adds it to dQ with fp32 atomics. Query blocks entirely above
// a wave's keys are skipped; the dQ product skips the same key halves.
//
// Matrix-core passes, as the oracle models them: S and dP sum d in passes of 8 consecutive
// values; dK/dV sum q in passes {16c+0..3, 16c+8..11} then {16c+4..7, 16c+12..15}; dQ sums keys
// in passes of 8 consecutive keys.
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

template <int D>
struct BwdCfg {
  static constexpr int BN = kBwdBlockN;  // keys per workgroup
  static constexpr int BM = kTile;       // query rows per step (the reference's query tile)
  static constexpr int THREADS = 256;
  static constexpr int KTP = BN + 8;     // transposed K pitch [D][BN]
  static constexpr int QP = D + 8;       // row-major Q / dO pitch [BM][D]
  static constexpr int QTP = BM + 8;     // transposed Q / dO pitch [D][BM]
  static constexpr int SP = BN + 8;      // dS pitch [BM][BN]
  static constexpr int KT_ELEMS = D * KTP;
  static constexpr int Q_ELEMS = BM * QP;
  static constexpr int QT_ELEMS = D * QTP;
  static constexpr int S_ELEMS = BM * SP;
  static constexpr int KC = D / 16;
  static constexpr int DT = D / 32;
  static constexpr int QROWS = D / 32;         // query rows per thread in the Q/dO loader
  static constexpr int QGROUPS = BM / QROWS;   // row groups across threads
  static constexpr int KROWS = BN * D / (8 * THREADS);  // keys per thread in the K loader (8 or 4)
  static constexpr int KGROUPS = BN / KROWS;
  static constexpr int DQ_TILES = (BM / 32) * DT / 4;   // 32x32 dQ tiles per wave
};

// Position of row k (0..63) inside a transposed-tile row: chunk of 16, stored in the order
// {0-3, 8-11, 4-7, 12-15} (the q order of a 32x32 accumulator's lane halves).
__device__ __forceinline__ int perm_pos_b(int k) {
  return (k & ~15) + 8 * ((k >> 2) & 1) + 4 * ((k >> 3) & 1) + (k & 3);
}
__device__ __forceinline__ uint32_t pk_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pk_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

template <int D>
__global__ void __launch_bounds__(256, 1) bwd_kernel(BwdArgs a) {
  using C = BwdCfg<D>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[C::KT_ELEMS + 2 * C::Q_ELEMS + 2 * C::QT_ELEMS + C::S_ELEMS];
  __shared__ __attribute__((aligned(16))) float lse_s[C::BM];
  __shared__ __attribute__((aligned(16))) float dd_s[C::BM];
  uint16_t* Kt = smem;
  uint16_t* Qs = Kt + C::KT_ELEMS;
  uint16_t* Gs = Qs + C::Q_ELEMS;
  uint16_t* Qt = Gs + C::Q_ELEMS;
  uint16_t* Gt = Qt + C::QT_ELEMS;
  uint16_t* dSs = Gt + C::QT_ELEMS;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int nkb = (a.T + C::BN - 1) / C::BN;
  int pair, kb;
  decode_workgroup(blockIdx.x, a.B * a.H, nkb, false, pair, kb);
  const int b = pair / a.H, hd = pair - b * a.H;
  const int rs = a.H * D;
  const size_t base = ((size_t)b * a.T * a.H + hd) * D;
  const uint16_t* Qg = a.q + base;
  const uint16_t* Kg = a.k + base;
  const uint16_t* Vg = a.v + base;
  const uint16_t* Gg = a.dO + base;
  const float* lse_g = a.lse + (size_t)pair * a.T;
  const float* dd_g = a.Dv + (size_t)pair * a.T;

  const int k0 = kb * C::BN;
  const int kw = k0 + 32 * wave;  // this wave's first key
  const bool wave_keys = kw < a.T;
  const int key = kw + l32;       // this lane's key (column of S / dP)

  // ---- K block, transposed -> LDS (keys past T zero-filled); own K/V rows -> registers ----
  {
    const int kg = tid % C::KGROUPS, g = tid / C::KGROUPS;  // keys KROWS*kg.., d 8g..8g+7
    u32x4 kr[C::KROWS];
#pragma unroll
    for (int i = 0; i < C::KROWS; ++i) {
      const int row = C::KROWS * kg + i;
      kr[i] = (k0 + row < a.T) ? *(const u32x4*)(Kg + (size_t)(k0 + row) * rs + 8 * g) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int w = j >> 1;
      uint16_t* dst = Kt + (8 * g + j) * C::KTP + C::KROWS * kg;
      if (C::KROWS == 8) {
        u32x4 o;
#pragma unroll
        for (int p = 0; p < 4; ++p) o[p] = (j & 1) ? pk_hi(kr[2 * p][w], kr[2 * p + 1][w]) : pk_lo(kr[2 * p][w], kr[2 * p + 1][w]);
        *(u32x4*)dst = o;
      } else {
        u32x2 o;
#pragma unroll
        for (int p = 0; p < 2; ++p) o[p] = (j & 1) ? pk_hi(kr[2 * p][w], kr[2 * p + 1][w]) : pk_lo(kr[2 * p][w], kr[2 * p + 1][w]);
        *(u32x2*)dst = o;
      }
    }
  }
  u32x4 Kr[C::KC], Vr[C::KC];
#pragma unroll
  for (int c = 0; c < C::KC; ++c) {
    if (wave_keys) {
      Kr[c] = *(const u32x4*)(Kg + (size_t)key * rs + 16 * c + 8 * h);
      Vr[c] = *(const u32x4*)(Vg + (size_t)key * rs + 16 * c + 8 * h);
    } else {
      Kr[c] = u32x4{0, 0, 0, 0};
      Vr[c] = u32x4{0, 0, 0, 0};
    }
  }
  f32x16 dKa[C::DT], dVa[C::DT];
#pragma unroll
  for (int i = 0; i < C::DT; ++i) {
    dKa[i] = zero16();
    dVa[i] = zero16();
  }

  // ---- per query block loader: QROWS rows x 8 d per thread, stored row-major and transposed ----
  const int nqb = a.T / C::BM;
  const int qb0 = k0 / C::BM;
  const int qg = tid % C::QGROUPS, dg = tid / C::QGROUPS;
  u32x4 qreg[C::QROWS], greg[C::QROWS];
  float sreg = 0.0f;
  auto gload = [&](int qb) {
#pragma unroll
    for (int i = 0; i < C::QROWS; ++i) {
      const size_t g = (size_t)(qb * C::BM + C::QROWS * qg + i) * rs + 8 * dg;
      qreg[i] = *(const u32x4*)(Qg + g);
      greg[i] = *(const u32x4*)(Gg + g);
    }
    if (tid < C::BM)
      sreg = lse_g[qb * C::BM + tid];
    else if (tid < 2 * C::BM)
      sreg = dd_g[qb * C::BM + tid - C::BM];
  };
  auto tstore = [&](uint16_t* dstT, const u32x4* r) {
    uint16_t* row0 = dstT + 8 * dg * C::QTP + perm_pos_b(C::QROWS * qg);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int w = j >> 1;
      if (C::QROWS == 4) {
        u32x2 o;
        o[0] = (j & 1) ? pk_hi(r[0][w], r[1][w]) : pk_lo(r[0][w], r[1][w]);
        o[1] = (j & 1) ? pk_hi(r[2][w], r[3][w]) : pk_lo(r[2][w], r[3][w]);
        *(u32x2*)(row0 + j * C::QTP) = o;
      } else {
        *(uint32_t*)(row0 + j * C::QTP) = (j & 1) ? pk_hi(r[0][w], r[1][w]) : pk_lo(r[0][w], r[1][w]);
      }
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < C::QROWS; ++i) {
      *(u32x4*)(Qs + (C::QROWS * qg + i) * C::QP + 8 * dg) = qreg[i];
      *(u32x4*)(Gs + (C::QROWS * qg + i) * C::QP + 8 * dg) = greg[i];
    }
    tstore(Qt, qreg);
    tstore(Gt, greg);
    if (tid < C::BM)
      lse_s[tid] = sreg * kLog2e;  // the exponent is evaluated in base 2
    else if (tid < 2 * C::BM)
      dd_s[tid - C::BM] = sreg;
  };

  gload(qb0);
  lstore();
  __syncthreads();

  const float sl = a.scale * kLog2e;
  for (int qb = qb0; qb < nqb; ++qb) {
    if (qb + 1 < nqb) gload(qb + 1);
    const int qbase = qb * C::BM;
    const bool active = wave_keys && kw <= qbase + C::BM - 1;
    if (active) {
      const bool diag = kw + 31 > qbase;
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) {
        // ---- S = Q.K^T and dP = dO.V^T for 32 q x this wave's 32 keys (lane = key) ----
        const uint16_t* qa = Qs + (32 * qs + l32) * C::QP + 8 * h;
        const uint16_t* ga = Gs + (32 * qs + l32) * C::QP + 8 * h;
        f32x16 S = zero16(), dP = zero16();
#pragma unroll
        for (int c = 0; c < C::KC; ++c) {
          S = mfma(lds_read16(qa + 16 * c), Kr[c], S);
          dP = mfma(lds_read16(ga + 16 * c), Vr[c], dP);
        }
        // ---- P and dS for rows q = 32qs + 8g + 4h + i ----
        uint32_t Pw[8], dSw[8];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ql = 32 * qs + 8 * g + 4 * h;
          const f32x4 lv = *(const f32x4*)(lse_s + ql);
          const f32x4 dv = *(const f32x4*)(dd_s + ql);
          float sv[4], dpv[4], pv[4], dsv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sv[i] = S[4 * g + i];
            dpv[i] = dP[4 * g + i];
          }
          round_pair(sv[0], sv[1]);
          round_pair(sv[2], sv[3]);
          round_pair(dpv[0], dpv[1]);
          round_pair(dpv[2], dpv[3]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float p = exp2_hw(fmaf(sv[i], sl, -lv[i]));
            if (diag && key > qbase + ql + i) p = 0.0f;
            pv[i] = p;
            dsv[i] = (p * (dpv[i] - dv[i])) * a.scale;
          }
          Pw[2 * g] = pack_bf16(pv[0], pv[1]);
          Pw[2 * g + 1] = pack_bf16(pv[2], pv[3]);
          dSw[2 * g] = pack_bf16(dsv[0], dsv[1]);
          dSw[2 * g + 1] = pack_bf16(dsv[2], dsv[3]);
          uint16_t* dcol = dSs + ql * C::SP + 32 * wave + l32;
          dcol[0] = (uint16_t)dSw[2 * g];
          dcol[C::SP] = (uint16_t)(dSw[2 * g] >> 16);
          dcol[2 * C::SP] = (uint16_t)dSw[2 * g + 1];
          dcol[3 * C::SP] = (uint16_t)(dSw[2 * g + 1] >> 16);
        }
        // ---- dV^T += dO^T.P and dK^T += Q^T.dS over these 32 q (m = d, n = key) ----
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int cq = 2 * qs + half, w0 = 4 * half;
          const u32x4 Bp = {Pw[w0], Pw[w0 + 1], Pw[w0 + 2], Pw[w0 + 3]};
          const u32x4 Bs = {dSw[w0], dSw[w0 + 1], dSw[w0 + 2], dSw[w0 + 3]};
          const uint16_t* gt = Gt + l32 * C::QTP + 16 * cq + 8 * h;
          const uint16_t* qt = Qt + l32 * C::QTP + 16 * cq + 8 * h;
#pragma unroll
          for (int dt = 0; dt < C::DT; ++dt) {
            dVa[dt] = mfma(lds_read16(gt + 32 * dt * C::QTP), Bp, dVa[dt]);
            dKa[dt] = mfma(lds_read16(qt + 32 * dt * C::QTP), Bs, dKa[dt]);
          }
        }
      }
      // the reference stores dK/dV as bf16 after every query tile
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          round_pair(dKa[dt], r);
          round_pair(dVa[dt], r);
        }
    }
    __syncthreads();  // dS complete; Q/dO tiles no longer read
    if (qb + 1 < nqb) lstore();

    // ---- dQ block: one bf16 part per reference key tile (64 keys), fp32 atomic add ----
#pragma unroll
    for (int t = 0; t < C::DQ_TILES; ++t) {
      const int tile = wave * C::DQ_TILES + t;
      const int qs = tile / C::DT, dt = tile % C::DT;
      const uint16_t* sa = dSs + (32 * qs + l32) * C::SP + 8 * h;
      const uint16_t* kb_ = Kt + (32 * dt + l32) * C::KTP + 8 * h;
      f32x16 sum = zero16();
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // keys of the reference key tile 2kb+half: present, and at or below this query tile
        if (k0 + 64 * half >= a.T || 2 * kb + half > qb) continue;
        f32x16 acc = zero16();
#pragma unroll
        for (int ck = 0; ck < 4; ++ck)
          acc = mfma(lds_read16(sa + 64 * half + 16 * ck), lds_read16(kb_ + 64 * half + 16 * ck), acc);
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          round_pair(acc, r);
          sum[r] += acc[r];
          sum[r + 1] += acc[r + 1];
        }
      }
      float* dQg = a.dQ + base + (size_t)qbase * rs;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int ql = 32 * qs + 8 * (r >> 2) + 4 * h + (r & 3);
        unsafeAtomicAdd(dQg + (size_t)ql * rs + 32 * dt + l32, sum[r]);
      }
    }
    __syncthreads();  // dS consumed; next Q/dO tiles visible
  }

  // ---- dK, dV (already bf16-valued): lane = key, rows d = 32dt + 8g + 4h + i ----
  if (!wave_keys) return;
  uint16_t* dKg = a.dK + base + (size_t)key * rs;
  uint16_t* dVg = a.dV + base + (size_t)key * rs;
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * dt + 8 * g + 4 * h;
      *(u32x2*)(dKg + d0) = u32x2{pack_bf16(dKa[dt][4 * g], dKa[dt][4 * g + 1]),
                                  pack_bf16(dKa[dt][4 * g + 2], dKa[dt][4 * g + 3])};
      *(u32x2*)(dVg + d0) = u32x2{pack_bf16(dVa[dt][4 * g], dVa[dt][4 * g + 1]),
                                  pack_bf16(dVa[dt][4 * g + 2], dVa[dt][4 * g + 3])};
    }
}

hipError_t launch_backward(const BwdArgs& a, int D, hipStream_t s) {
  const int nkb = (a.T + kBwdBlockN - 1) / kBwdBlockN;
  const dim3 grid((unsigned)(a.B * a.H * nkb));
  if (D == 64)
    hipLaunchKernelGGL(bwd_kernel<64>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(bwd_kernel<128>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace mla
