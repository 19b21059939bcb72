// attn_bwd.hip -- the dK/dV half of flashAttentionBackward on gfx950 (key-owner kernel).
//
// Reference: /root/reference/attention.metal:198-299. For each 64-key tile kt and each 64-row
// query tile qt >= kt:
//   dP = bf16(dO.V^T), S = bf16(Q.K^T)                           (:274-275)
//   p = exp(S*scale - lse[q]), p = 0 where key > q (diagonal), P = bf16(p)
//   dS = bf16(p * (dP - D[q]) * scale)                            (:277-286)
//   dK = bf16(dK + dS^T.Q), dV = bf16(dV + P^T.dO)   once per query tile (:289-290)
// The key-tile owner accumulates dK/dV race-free. dQ (:288,292-296) is computed by a query-owner
// kernel launched after this one: attn_bwd_dq.hip recomputes dS (flashAttentionBackward), or,
// when the caller provides a workspace (flashAttentionBackwardWorkspace), this kernel also
// stores every dS tile it computes, bf16, and attn_bwd_dqs.hip computes dQ = dS.K from them.
//
// Work split: 4 waves x 32 keys per workgroup, two workgroups per CU (three at D = 64). Wave w
// owns keys 32w..32w+31 of the block: it keeps their K and V rows in registers as matrix-core
// B operands and computes S and dP with lane = key (the query tile's Q and dO rows are A
// operands from LDS), so P and dS come out of the accumulators already laid out as the B
// operands of dV^T += dO^T.P and dK^T += Q^T.dS: no LDS round trip. dO^T and Q^T are read with
// ds_read_b64_tr_b16 from the row-major tiles, four queries per read, in the order
// {8g + 4h + i} that lane half h holds. Between query tiles dK and dV are bf16 values (the
// reference stores them as bf16 after every query tile), carried packed two per register and
// widened to fp32 for one 32-row d slice at a time.
//
// Per query tile: S and dP of query rows 0-31, their p, P and dS, the same for rows 32-63, then
// the dK/dV products. Query tiles stream through LDS two stages deep by
// global_load_lds_dwordx4: Q and dO rows, and lse and D of the tile (lse scaled by log2(e) in
// place once it lands).
//
// Matrix-core passes, as the oracle models them: S and dP sum d in passes of 8 consecutive
// values; dK/dV sum q in passes {16c+0..3, 16c+8..11} then {16c+4..7, 16c+12..15}.
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

template <int D>
struct BwdCfg {
  static constexpr int BN = kBwdBlockN;  // keys per workgroup (128)
  static constexpr int BM = kTile;       // query rows per tile (the reference's query tile)
  static constexpr int THREADS = 256;
  // Q/dO row pitch: the 16-byte row reads are conflict-free; the transposing reads take 2-way
  // conflicts (no pitch clears both)
  static constexpr int P = (D == 128) ? D + 24 : D + 8;
  static constexpr int TBYTES = BM * P * 2;              // one padded tile
  static constexpr int SLOTS = P / 8;                    // 16-byte slots of a padded row
  static constexpr int LPW = (SLOTS + 3) / 4;            // row-copy instructions per wave per tile (max)
  static constexpr int STAT = 2 * TBYTES;                // lse (64 fp32), D (64 fp32), + 512 B the copy spills
  static constexpr int STAGE = 2 * TBYTES + 1024;
  static constexpr int KC = D / 16;
  static constexpr int DT = D / 32;
};

typedef __attribute__((address_space(3))) uint16_t lds_u16b;
__device__ __forceinline__ uint32_t lds_addr_b(const void* p) { return (uint32_t)(uintptr_t)(const lds_u16b*)p; }
__device__ __forceinline__ u32x4 lds_b128_b(uint32_t byte_addr) {
  return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)byte_addr;
}
__device__ __forceinline__ f32x4 lds_f4_b(uint32_t byte_addr) {
  return *(const __attribute__((address_space(3))) f32x4*)(uintptr_t)byte_addr;
}
__device__ __forceinline__ u32x2 lds_tr_b(uint32_t byte_addr) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (__attribute__((address_space(3))) i16x4*)(uintptr_t)byte_addr));
}


template <bool V>
struct DiagTag {
  static constexpr bool value = V;
};

// D = 64: three workgroups per CU (168 VGPRs, a few spilled outside the product loop), 6-8%
// faster than two; D = 128 needs its 244-253 VGPRs and runs two.
template <int D, bool DS>
__global__ void __launch_bounds__(256, D == 64 ? 3 : 2) bwd_kernel(BwdArgs a) {
  using C = BwdCfg<D>;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const int nkb = (a.T + C::BN - 1) / C::BN;
  int pair, kb;
  decode_workgroup(blockIdx.x, a.B * a.H, nkb, false, pair, kb);
  const int b = pair / a.H, hd = pair - b * a.H;
  const int rs = a.H * D;
  const size_t base = ((size_t)b * a.T * a.H + hd) * D;
  const char* Qg = (const char*)(a.q + base);
  const char* Gg = (const char*)(a.dO + base);
  const uint16_t* Kg = a.k + base;
  const uint16_t* Vg = a.v + base;
  const float* lse_g = a.lse + (size_t)pair * a.T;
  const float* dd_g = a.Dv + (size_t)pair * a.T;
  const size_t tile_bytes = (size_t)C::BM * rs * 2;

  const int k0 = kb * C::BN;
  const int kw = k0 + 32 * wave;  // the wave's first key
  const bool wave_keys = kw < a.T;  // false only in the last block when T % 128 == 64
  const int key = kw + l32;
  const int key_ld = min(key, a.T - 1);  // rows of keys past T are read in bounds, never stored

  // own K and V rows as B operands: lane holds row `key`, d = 16c + 8h .. +7
  u32x4 Kr[C::KC], Vr[C::KC];
#pragma unroll
  for (int c = 0; c < C::KC; ++c) {
    Kr[c] = *(const u32x4*)(Kg + (size_t)key_ld * rs + 16 * c + 8 * h);
    Vr[c] = *(const u32x4*)(Vg + (size_t)key_ld * rs + 16 * c + 8 * h);
  }
  // dK^T, dV^T (m = d, n = key) as packed bf16 pairs of accumulator rows (r, r+1)
  uint32_t dKp[C::DT][8], dVp[C::DT][8];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dKp[dt][i] = 0u;
      dVp[dt][i] = 0u;
    }

  // Query-tile copy. Q and dO rows: instruction i covers 16-byte slots 64i..64i+63 of the padded
  // tile (slot s = row s / SLOTS, chunk s % SLOTS; pad chunks re-read the row's last chunk).
  // lse and D of the tile: wave 0, lanes 0-15 and 16-31 (lanes 32-63 repeat them).
  uint32_t off[C::LPW];
#pragma unroll
  for (int j = 0; j < C::LPW; ++j) {
    const int s = 64 * (wave + 4 * j) + lane, row = s / C::SLOTS, c = min(s % C::SLOTS, D / 8 - 1);
    off[j] = (uint32_t)(row * rs * 2 + c * 16);
  }
  const int nqb = a.T / C::BM;
  const int qb0 = k0 / C::BM;
  const uint32_t smem_a = lds_addr_b(smem);
  auto issue_tile = [&](int qb, int stage) {
    const char* qs = Qg + (size_t)qb * tile_bytes;
    const char* gs = Gg + (size_t)qb * tile_bytes;
    const uint32_t dst = smem_a + stage * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::LPW; ++j)
      if (wave + 4 * j < C::SLOTS) {
        dma16(off[j], qs, dst + 1024 * (wave + 4 * j));
        dma16(off[j], gs, dst + C::TBYTES + 1024 * (wave + 4 * j));
      }
    if (wave == 0) {
      const int l = lane & 31;
      const float* src = (l < 16 ? lse_g : dd_g) + qb * C::BM + 4 * (l & 15);
      dma16_v(src, dst + C::STAT);
    }
  };
  // lse -> lse*log2(e) in place (exponents are base 2) and, for D = 128, D -> D*scale, by wave 0
  // once its copy has landed
  auto scale_lse = [&](int stage) {
    if (wave == 0) {
      float* l2 = (float*)(smem + stage * C::STAGE + C::STAT);
      l2[lane] = l2[lane] * kLog2e;
      if (D != 64) l2[64 + lane] = l2[64 + lane] * a.scale;
    }
  };

  // LDS operand addresses (bytes within a stage)
  const uint32_t row_rd = 2 * (l32 * C::P + 8 * h);  // S / dP A operand: row = q, 8 d at 16c + 8h
  // dV^T / dK^T A operand (dO^T, Q^T) by tr reads: group g = lane/16 covers d = 16(g%2) .. +15 of
  // a 32-d tile; source lane s = lane%16 points at query row 4h + s/4 (+8 for the second read)
  const int g16 = lane >> 4, s16 = lane & 15;
  const uint32_t tr_rd = 2 * ((4 * h + (s16 >> 2)) * C::P + 16 * (g16 & 1) + 4 * (s16 & 3));
  const uint32_t st_rd = 4 * (4 * h);  // statistics of query row 32t + 8g + 4h + i at +4(32t + 8g + i)
  const float sl = a.scale * kLog2e;
  const float scale = a.scale;

  // Update accumulators: chain n (dV of d tile n for n < DT, else dK of d tile n - DT) runs in
  // block n % 2; while it runs, the other block's previous chain is rounded back into the bf16
  // state and the next chain's state is widened into it.
  f32x16 acc[2] = {zero16(), zero16()};
  auto state = [&](int n) -> uint32_t* { return n < C::DT ? dVp[n] : dKp[n - C::DT]; };
  auto pack_pairs = [&](int n, int u0, int u1) {  // state(n)[u] = bf16 pair of block n % 2
#pragma unroll
    for (int u = u0; u < u1; ++u) {
      uint32_t v = pack_bf16(acc[n & 1][2 * u], acc[n & 1][2 * u + 1]);
      pin(v);
      state(n)[u] = v;
    }
  };
  auto unpack_pairs = [&](int n, int u0, int u1) {  // block n % 2 = widened state(n)
#pragma unroll
    for (int u = u0; u < u1; ++u) {
      float lo = bf_lo(state(n)[u]), hi = bf_hi(state(n)[u]);
      pin(lo, hi);
      acc[n & 1][2 * u] = lo;
      acc[n & 1][2 * u + 1] = hi;
    }
  };

  // One query tile: NS matrix-core instructions in a fixed order, one per slot, each slot also
  // doing a slice of vector work that does not depend on it. Slots:
  //   [0, KC) S of rows 0-31, d step c     [KC, 2KC) dP of rows 0-31
  //   [2KC, 3KC) S of rows 32-63           [3KC, 4KC) dP of rows 32-63
  //   [4KC, NS) update chain n = (i - 4KC) / 4, query step j = (i - 4KC) % 4
  // S[t], dP[t] hold rows q = 32t + 8(r/4) + 4h + r%4 of the tile, lane = key.
  // dS of the latest query tile, packed bf16 (index 8t + r/2); with DS it is stored in the first
  // slots of the next tile (or after the last one), so the end-of-tile wait never waits for it
  uint32_t dS[16];
  // this wave's 32 keys are half hw of key tile ktw; dS tile (qt, ktw) of the pair's triangle
  const int ktw = kb * (C::BN / 64) + (wave >> 1), hw = wave & 1;
  const int nqt = a.T / 64;
  const size_t tri = (size_t)pair * ((size_t)nqt * (nqt + 1) / 2);
  auto ds_addr = [&](int qt) -> char* {
    if (!DS || !wave_keys || ktw > qt) return nullptr;
    return (char*)a.dS + (tri + (size_t)qt * (qt + 1) / 2 + ktw) * 8192 + hw * 4096 + lane * 16;
  };
  auto store_ds = [&](char* dst, int s) {  // streaming store: the tile is read once, by another kernel
    __builtin_nontemporal_store(u32x4{dS[4 * s], dS[4 * s + 1], dS[4 * s + 2], dS[4 * s + 3]}, (u32x4*)(dst + 1024 * s));
  };

  auto qtile = [&](int qb, int stage, auto diag_tag, char* ds_prev) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    constexpr int NS = 4 * C::KC + 8 * C::DT;
    constexpr int PPS = 8 / C::KC;  // score pairs of vector work per S/dP slot
    // per-lane LDS bases of this stage, computed once and anchored so that every operand address
    // below is base + constant (the constant goes into the instruction's offset field)
    const uint32_t qbase_a = lds_addr_b(smem + stage * C::STAGE);
    uint32_t row_a = qbase_a + row_rd, tr_a = qbase_a + tr_rd, stat_a = qbase_a + C::STAT + st_rd;
    pin(row_a);
    pin(tr_a);
    pin(stat_a);
    const int qrow = qb * C::BM + 4 * h - key;  // q - key = qrow + 32t + 8g + i
    f32x16 x0 = zero16(), x1 = zero16(), y0 = zero16(), y1 = zero16();
    uint32_t Pp[16];  // packed bf16: index 8t + r/2

    auto operand = [&](int i) -> u32x4 {
      if (i < 4 * C::KC) {
        const int seg = i / C::KC, t = seg >> 1, c = i % C::KC;
        return lds_b128_b(row_a + ((seg & 1) ? C::TBYTES : 0) + 2 * (32 * t * C::P + 16 * c));
      }
      const int k = i - 4 * C::KC, n = k / 4, j = k % 4, dt = n % C::DT;
      const uint32_t src = tr_a + (n >= C::DT ? 0 : C::TBYTES) + 2 * (16 * j * C::P + 32 * dt);
      const u32x2 lo = lds_tr_b(src), hi = lds_tr_b(src + 2 * 8 * C::P);
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    // Score pairs of vector work in slot i: kind 1 = p of half t, kind 2 = dS of half t; pairs
    // r = 2u for u in [u0, u0 + cnt).
    struct Work {
      int kind, t, u0, cnt;
    };
    auto work = [&](int i) -> Work {
      if (i < 4 * C::KC) {
        const int seg = i / C::KC, u0 = (i % C::KC) * PPS;
        if (seg == 1) return {1, 0, u0, PPS};
        if (seg == 2) return {2, 0, u0, PPS};
        if (seg == 3) return {1, 1, u0, PPS};
        return {0, 0, 0, 0};
      }
      const int k = i - 4 * C::KC;  // dS of half 1 spread over the dV chains' 4DT slots
      if (k < 4 * C::DT) {
        constexpr int SPAN = (4 * C::DT) / 8;  // slots per pair (1 or 2)
        if (k % SPAN == 0) return {2, 1, k / SPAN, 1};
      }
      return {0, 0, 0, 0};
    };
    // lse (kind 1) or D (kind 2) of the rows of the pairs of slot i (read one slot ahead)
    auto stats = [&](int i) -> f32x4 {
      const Work w = work(i);
      const uint32_t ad = stat_a + (w.kind == 2 ? 256 : 0) + 4 * (32 * w.t + 8 * (w.u0 >> 1) + 2 * (w.u0 & 1));
      if (w.cnt == 2) return lds_f4_b(ad);
      const f32x2 v = *(const __attribute__((address_space(3))) f32x2*)(uintptr_t)ad;
      return f32x4{v[0], v[1], 0.0f, 0.0f};
    };
    auto p_pair = [&](f32x16& x, int t, int u, float l0, float l1) {
      const int r = 2 * u;
      x[r] = round_bf16(x[r]);
      x[r + 1] = round_bf16(x[r + 1]);
      float p0 = exp2_hw(fmaf(x[r], sl, -l0));
      float p1 = exp2_hw(fmaf(x[r + 1], sl, -l1));
      if (DIAG) {
        const int d = qrow + 32 * t + 8 * (r >> 2) + (r & 3);  // q - key of element r
        if (d < 0) p0 = 0.0f;
        if (d + 1 < 0) p1 = 0.0f;
      }
      pin(p0, p1);
      x[r] = p0;
      x[r + 1] = p1;
      uint32_t pk = pack_bf16(p0, p1);
      pin(pk);
      Pp[8 * t + u] = pk;
    };
    auto ds_pair = [&](const f32x16& x, f32x16& y, int t, int u, float d0_, float d1_) {
      const int r = 2 * u;
      y[r] = round_bf16(y[r]);
      y[r + 1] = round_bf16(y[r + 1]);
      // D = 64: scale = 1/8 is a power of two, so bf16(v * scale) = bf16(v) / 8 exactly (above the
      // subnormal range); dS is carried times 8 and dK, and dQ from the stored dS, are scaled once
      // when they are stored. D = 128: p * (dP*scale - D*scale) with D*scale precomputed (one fma
      // for the reference's subtraction and multiply, :284; the fp32 value differs from
      // (p*(dP - D))*scale by a few fp32 ulps, below the bf16 rounding that follows)
      const float d0 = D == 64 ? x[r] * (y[r] - d0_) : x[r] * fmaf(y[r], scale, -d0_);
      const float d1 = D == 64 ? x[r + 1] * (y[r + 1] - d1_) : x[r + 1] * fmaf(y[r + 1], scale, -d1_);
      uint32_t pk = pack_bf16(d0, d1);
      pin(pk);
      dS[8 * t + u] = pk;
    };

    // operand reads run ahead(i) products ahead: four during the first S segment (almost no
    // vector work there to cover the LDS latency), then two at D = 128 and one at D = 64; the
    // statistics SA slots ahead (D = 64 has no registers for more at three workgroups per CU)
    constexpr int RING = 5;
    constexpr int SA = D == 128 ? 2 : 1;  // statistics lookahead (slots)
    auto ahead = [](int i) { return i < C::KC ? 4 : (D == 128 ? 2 : 1); };
    u32x4 ring[RING];
    f32x4 sring[SA + 1];
#pragma unroll
    for (int k = 0; k <= ahead(0); ++k) ring[k] = operand(k);
    sring[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NS; ++i) {
#pragma unroll
      for (int k = (i ? i - 1 + ahead(i - 1) : ahead(0)) + 1; k <= i + ahead(i) && k < NS; ++k)
        ring[k % RING] = operand(k);
      if (i + SA < NS && work(i + SA).kind) sring[(i + SA) % (SA + 1)] = stats(i + SA);
      const u32x4& op = ring[i % RING];
      if (i < 4 * C::KC) {
        const int seg = i / C::KC, c = i % C::KC;
        if (seg == 0) x0 = mfma(op, Kr[c], x0);
        else if (seg == 1) y0 = mfma(op, Vr[c], y0);
        else if (seg == 2) x1 = mfma(op, Kr[c], x1);
        else y1 = mfma(op, Vr[c], y1);
      } else {
        const int k = i - 4 * C::KC, n = k / 4, j = k % 4;
        const uint32_t* src = n >= C::DT ? dS : Pp;
        acc[n & 1] = mfma(op, u32x4{src[4 * j], src[4 * j + 1], src[4 * j + 2], src[4 * j + 3]}, acc[n & 1]);
      }
      // vector work of this slot
      const Work w = work(i);
      const f32x4 st = sring[i % (SA + 1)];
#pragma unroll
      for (int v = 0; v < w.cnt; ++v) {
        if (w.kind == 1)
          p_pair(w.t ? x1 : x0, w.t, w.u0 + v, st[2 * v], st[2 * v + 1]);
        else if (w.kind == 2)
          ds_pair(w.t ? x1 : x0, w.t ? y1 : y0, w.t, w.u0 + v, st[2 * v], st[2 * v + 1]);
      }
      if (DS && i < 4 && ds_prev) store_ds(ds_prev, i);  // previous tile's dS (rewritten from slot 2KC on)
      if (i < C::KC) {
        // the previous tile's last chain (dK of d tile DT-1, block 1) back into the state
        pack_pairs(2 * C::DT - 1, (i * 8) / C::KC, ((i + 1) * 8) / C::KC);
      } else if (i >= 3 * C::KC && i < 4 * C::KC) {
        // widen the first two chains' state (dV of d tiles 0 and 1)
        const int s_ = i - 3 * C::KC, per = 16 / C::KC, u0 = s_ * per;
#pragma unroll
        for (int u = u0; u < u0 + per; ++u) unpack_pairs(u < 8 ? 0 : 1, u & 7, (u & 7) + 1);
      } else if (i >= 4 * C::KC) {
        const int k = i - 4 * C::KC, n = k / 4, j = k % 4;
        if (n >= 1 && j == 1) pack_pairs(n - 1, 0, 8);
        if (n + 1 < 2 * C::DT && n >= 1 && j >= 2) unpack_pairs(n + 1, 4 * (j - 2), 4 * (j - 2) + 4);
      }
      // D = 128: raised issue priority while S and dP are computed (their chains have little
      // vector work of their own; the other wave on the SIMD issues its vector work around them)
      if (D == 128 && i == 0) __builtin_amdgcn_s_setprio(1);
      if (D == 128 && i + 1 == 4 * C::KC) __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- query tiles qb0 .. nqb-1 ----
  // Every wave runs every tile (no per-wave branch: the state stays in place across tiles). The
  // first two tiles hold the block's diagonal and run masked: a wave whose keys all lie above
  // the tile gets p = 0 there and leaves its state unchanged (adding exact zeros). Keys past T
  // (last block, T % 128 == 64) compute on clamped rows and are never stored.
  issue_tile(qb0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  scale_lse(0);
  __syncthreads();
  int qb = qb0, it = 0;
  char* ds_prev = nullptr;
  for (; qb < nqb && qb < qb0 + 2; ++qb, ++it) {
    if (qb + 1 < nqb) issue_tile(qb + 1, (it + 1) & 1);
    qtile(qb, it & 1, DiagTag<true>(), ds_prev);
    ds_prev = ds_addr(qb);
    __builtin_amdgcn_s_waitcnt(0);
    if (qb + 1 < nqb) scale_lse((it + 1) & 1);
    __syncthreads();
  }
  for (; qb < nqb; ++qb, ++it) {
    if (qb + 1 < nqb) issue_tile(qb + 1, (it + 1) & 1);
    qtile(qb, it & 1, DiagTag<false>(), ds_prev);
    ds_prev = ds_addr(qb);
    __builtin_amdgcn_s_waitcnt(0);
    if (qb + 1 < nqb) scale_lse((it + 1) & 1);
    __syncthreads();
  }
  pack_pairs(2 * C::DT - 1, 0, 8);
  if (DS && ds_prev)
    for (int s = 0; s < 4; ++s) store_ds(ds_prev, s);

  // ---- dK, dV: lane = key, rows d = 32dt + 8g + 4h + i ----
  if (!wave_keys) return;
  uint16_t* dKg = a.dK + base + (size_t)key * rs;
  uint16_t* dVg = a.dV + base + (size_t)key * rs;
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = 32 * dt + 8 * g + 4 * h;
      if (D == 64) {  // dK was carried times 8 (see ds_pair); the division is exact
        for (int u = 2 * g; u < 2 * g + 2; ++u) dKp[dt][u] = pack_bf16(bf_lo(dKp[dt][u]) * 0.125f, bf_hi(dKp[dt][u]) * 0.125f);
      }
      *(u32x2*)(dKg + d0) = u32x2{dKp[dt][2 * g], dKp[dt][2 * g + 1]};
      *(u32x2*)(dVg + d0) = u32x2{dVp[dt][2 * g], dVp[dt][2 * g + 1]};
    }
}

hipError_t launch_backward(const BwdArgs& a, int D, hipStream_t s) {
  const int nkb = (a.T + kBwdBlockN - 1) / kBwdBlockN;
  const dim3 grid((unsigned)(a.B * a.H * nkb));
  if (a.dS) {
    if (D == 64)
      hipLaunchKernelGGL((bwd_kernel<64, true>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((bwd_kernel<128, true>), grid, dim3(256), 0, s, a);
  } else {
    if (D == 64)
      hipLaunchKernelGGL((bwd_kernel<64, false>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((bwd_kernel<128, false>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace mla
