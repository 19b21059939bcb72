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
// operands, plus fp32 dK^T/dV^T accumulators that are rounded to bf16 after every 64-row
// query block (the reference's rounding points). Per query block the workgroup stages Q, dO
// (row-major, swizzled) and lse/D in LDS; each wave computes S and dP for its keys (lane = key),
// forms P and dS in registers, writes dS to LDS as [key][q], and updates dV^T/dK^T with A
// operands read by ds_read_b64_tr_b16 from the dO/Q tiles. After a barrier the workgroup
// computes the dQ block [64 q][D] from dS (tr reads of [key][q]) and the K block staged in LDS,
// one bf16-rounded part per reference key tile, and adds it to dQ with fp32 atomics.
// Query blocks entirely above a wave's keys are skipped (nothing of them is on the causal side).
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
  static constexpr int CH = D / 8;
  static constexpr int KC = D / 16;
  static constexpr int DT = D / 32;
  static constexpr int K_ELEMS = BN * D;
  static constexpr int Q_ELEMS = BM * D;
  static constexpr int DS_ELEMS = BN * BM;
  static constexpr int QLOADS = BM * CH / THREADS;  // 16-byte loads per thread per tensor
  static constexpr int KLOADS = BN * CH / THREADS;
  // dQ tiles (32 q x 32 d) per wave: (BM/32)*(D/32) tiles over 4 waves
  static constexpr int DQ_TILES = (BM / 32) * DT / 4;
};

template <int D>
__global__ void __launch_bounds__(256) bwd_kernel(BwdArgs a) {
  using C = BwdCfg<D>;
  using SwD = SwzTile<D>;
  using SwS = SwzTile<C::BM>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[C::K_ELEMS + 2 * C::Q_ELEMS + C::DS_ELEMS];
  __shared__ __attribute__((aligned(16))) float lse_s[C::BM];
  __shared__ __attribute__((aligned(16))) float dd_s[C::BM];
  uint16_t* Ks = smem;
  uint16_t* Qs = Ks + C::K_ELEMS;
  uint16_t* Gs = Qs + C::Q_ELEMS;
  uint16_t* dSs = Gs + C::Q_ELEMS;

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

  // ---- K block -> LDS (rows past T zero-filled); own K/V rows -> registers ----
#pragma unroll
  for (int i = 0; i < C::KLOADS; ++i) {
    const int idx = tid + i * C::THREADS, row = idx / C::CH, ch = idx % C::CH;
    u32x4 v = {0, 0, 0, 0};
    if (k0 + row < a.T) v = *(const u32x4*)(Kg + (size_t)(k0 + row) * rs + ch * 8);
    *(u32x4*)(Ks + SwD::off(row, ch * 8)) = v;
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

  const int nqb = a.T / C::BM;
  const int qb0 = k0 / C::BM;
  u32x4 qreg[C::QLOADS], greg[C::QLOADS];
  float sreg = 0.0f;
  auto gload = [&](int qb) {
#pragma unroll
    for (int i = 0; i < C::QLOADS; ++i) {
      const int idx = tid + i * C::THREADS, row = idx / C::CH, ch = idx % C::CH;
      const size_t g = (size_t)(qb * C::BM + row) * rs + ch * 8;
      qreg[i] = *(const u32x4*)(Qg + g);
      greg[i] = *(const u32x4*)(Gg + g);
    }
    if (tid < C::BM)
      sreg = lse_g[qb * C::BM + tid];
    else if (tid < 2 * C::BM)
      sreg = dd_g[qb * C::BM + tid - C::BM];
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < C::QLOADS; ++i) {
      const int idx = tid + i * C::THREADS, row = idx / C::CH, ch = idx % C::CH;
      *(u32x4*)(Qs + SwD::off(row, ch * 8)) = qreg[i];
      *(u32x4*)(Gs + SwD::off(row, ch * 8)) = greg[i];
    }
    if (tid < C::BM)
      lse_s[tid] = sreg;
    else if (tid < 2 * C::BM)
      dd_s[tid - C::BM] = sreg;
  };

  gload(qb0);
  lstore();
  __syncthreads();

  const int cb = 16 * ((lane >> 4) & 1);  // column base of this lane's 16-lane group
  for (int qb = qb0; qb < nqb; ++qb) {
    if (qb + 1 < nqb) gload(qb + 1);
    const int qbase = qb * C::BM;
    const bool active = wave_keys && kw <= qbase + C::BM - 1;
    if (active) {
      // ---- S = Q.K^T and dP = dO.V^T for 64 q x this wave's 32 keys (lane = key) ----
      f32x16 S[2], dP[2];
#pragma unroll
      for (int qs = 0; qs < 2; ++qs) {
        S[qs] = zero16();
        dP[qs] = zero16();
#pragma unroll
        for (int c = 0; c < C::KC; ++c) {
          const u32x4 qa = lds_read16(Qs + SwD::off(32 * qs + l32, 16 * c + 8 * h));
          const u32x4 ga = lds_read16(Gs + SwD::off(32 * qs + l32, 16 * c + 8 * h));
          S[qs] = mfma(qa, Kr[c], S[qs]);
          dP[qs] = mfma(ga, Vr[c], dP[qs]);
        }
      }
      // ---- P and dS (rows q = 32qs + 8g + 4h + i) ----
      const bool diag = kw + 31 > qbase;
      uint32_t Pw[2][8], dSw[2][8];
#pragma unroll
      for (int qs = 0; qs < 2; ++qs)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ql = 32 * qs + 8 * g + 4 * h;
          const f32x4 lv = *(const f32x4*)(lse_s + ql);
          const f32x4 dv = *(const f32x4*)(dd_s + ql);
          float sv[4], pv[4], dpv[4], dsv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sv[i] = S[qs][4 * g + i];
            dpv[i] = dP[qs][4 * g + i];
          }
          round_pair(sv[0], sv[1]);
          round_pair(sv[2], sv[3]);
          round_pair(dpv[0], dpv[1]);
          round_pair(dpv[2], dpv[3]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float xs = sv[i] * a.scale;
            float p = exp2_hw((xs - lv[i]) * kLog2e);
            if (diag && key > qbase + ql + i) p = 0.0f;
            pv[i] = p;
            const float t1 = p * (dpv[i] - dv[i]);
            dsv[i] = t1 * a.scale;
          }
          Pw[qs][2 * g] = pack_bf16(pv[0], pv[1]);
          Pw[qs][2 * g + 1] = pack_bf16(pv[2], pv[3]);
          dSw[qs][2 * g] = pack_bf16(dsv[0], dsv[1]);
          dSw[qs][2 * g + 1] = pack_bf16(dsv[2], dsv[3]);
          *(u32x2*)(dSs + SwS::off(32 * wave + l32, ql)) = u32x2{dSw[qs][2 * g], dSw[qs][2 * g + 1]};
        }
      // ---- dV^T += dO^T.P and dK^T += Q^T.dS (m = d, n = key, k = q) ----
#pragma unroll
      for (int cq = 0; cq < 4; ++cq) {
        const int qs = cq >> 1, w0 = 4 * (cq & 1);
        const u32x4 Bp = {Pw[qs][w0], Pw[qs][w0 + 1], Pw[qs][w0 + 2], Pw[qs][w0 + 3]};
        const u32x4 Bs = {dSw[qs][w0], dSw[qs][w0 + 1], dSw[qs][w0 + 2], dSw[qs][w0 + 3]};
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const u32x2 glo = lds_tr(tr_addr<D>(Gs, 16 * cq + 4 * h, 32 * dt + cb, lane));
          const u32x2 ghi = lds_tr(tr_addr<D>(Gs, 16 * cq + 8 + 4 * h, 32 * dt + cb, lane));
          dVa[dt] = mfma(u32x4{glo[0], glo[1], ghi[0], ghi[1]}, Bp, dVa[dt]);
          const u32x2 qlo = lds_tr(tr_addr<D>(Qs, 16 * cq + 4 * h, 32 * dt + cb, lane));
          const u32x2 qhi = lds_tr(tr_addr<D>(Qs, 16 * cq + 8 + 4 * h, 32 * dt + cb, lane));
          dKa[dt] = mfma(u32x4{qlo[0], qlo[1], qhi[0], qhi[1]}, Bs, dKa[dt]);
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
    } else {
      // keys of this wave see nothing of this query block: dS rows are zero
#pragma unroll
      for (int g = 0; g < 8; ++g)
        *(u32x2*)(dSs + SwS::off(32 * wave + l32, 8 * g + 4 * h)) = u32x2{0, 0};
    }
    __syncthreads();  // dS complete; Q/dO tiles no longer read
    if (qb + 1 < nqb) lstore();

    // ---- dQ block: one bf16 part per reference key tile (64 keys), fp32 atomic add ----
#pragma unroll
    for (int t = 0; t < C::DQ_TILES; ++t) {
      const int tile = wave * C::DQ_TILES + t;
      const int qs = tile / C::DT, dt = tile % C::DT;
      f32x16 sum = zero16();
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int kref = k0 / kTile + half;  // the reference key tile of these 64 keys
        if (k0 + 64 * half >= a.T || kref > qb) continue;
        f32x16 acc = zero16();
#pragma unroll
        for (int ck = 0; ck < 4; ++ck) {
          const int kr = 64 * half + 16 * ck + 8 * h;
          const u32x2 slo = lds_tr(tr_addr<C::BM>(dSs, kr, 32 * qs + cb, lane));
          const u32x2 shi = lds_tr(tr_addr<C::BM>(dSs, kr + 4, 32 * qs + cb, lane));
          const u32x2 klo = lds_tr(tr_addr<D>(Ks, kr, 32 * dt + cb, lane));
          const u32x2 khi = lds_tr(tr_addr<D>(Ks, kr + 4, 32 * dt + cb, lane));
          acc = mfma(u32x4{slo[0], slo[1], shi[0], shi[1]}, u32x4{klo[0], klo[1], khi[0], khi[1]}, acc);
        }
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
