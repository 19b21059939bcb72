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
// Work split: 4 waves x 32 keys per workgroup, two workgroups per CU (three at D = 64 without the
// dS store). Wave w owns keys 32w..32w+31 of the block: it keeps their K and V rows in registers
// as matrix-core B operands and computes S and dP with lane = key (the query tile's Q and dO rows
// are A operands from LDS), so P and dS come out of the accumulators already laid out as the B
// operands of dV^T += dO^T.P and dK^T += Q^T.dS: no LDS round trip. dO^T and Q^T are read with
// ds_read_b64_tr_b16 from the row-major tiles, four queries per read, in the order {8g + 4h + i}
// that lane half h holds. Between query tiles dK and dV are bf16 values (the reference stores
// them as bf16 after every query tile), carried packed two per register and widened to fp32 for
// one 32-row d slice at a time, or (D = 64 with the dS store, and the fused short-sequence
// kernel) held as bf16-exact fp32 values and rounded in place.
//
// Per query tile: S and dP of query rows 0-31, their p, P and dS, the same for rows 32-63, then
// the dK/dV products. Query tiles stream through LDS two stages deep by
// global_load_lds_dwordx4: Q and dO rows, and lse and D of the tile (lse scaled by log2(e) in
// place once it lands).
//
// Matrix-core passes, as the oracle models them: S and dP sum d in passes of 8 consecutive
// values; dK/dV sum q in passes {16c+0..3, 16c+8..11} then {16c+4..7, 16c+12..15}.
#include <algorithm>
#include <type_traits>

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

// Where a query tile's dS goes (stored during the first four slots of the next tile, so the
// end-of-tile wait never waits for it): nowhere, the workspace in global memory (non-temporal:
// another kernel reads it once), or a tile slot in LDS.
struct NoDsSink {
  static constexpr bool kOn = false;
  __device__ bool on() const { return false; }
  __device__ void store(int, const uint32_t*) const {}
};
struct GlobalDsSink {
  static constexpr bool kOn = true;
  char* p;  // this lane's 16 bytes of chunk row 0 of the wave's half tile, or NULL
  __device__ bool on() const { return p != nullptr; }
  __device__ void store(int s, const uint32_t* v) const {
    __builtin_nontemporal_store(u32x4{v[4 * s], v[4 * s + 1], v[4 * s + 2], v[4 * s + 3]}, (u32x4*)(p + 1024 * s));
  }
};
struct LdsDsSink {
  static constexpr bool kOn = true;
  uint32_t half;    // LDS byte address of the wave's half tile (1 KB aligned)
  uint32_t lane16;  // 16 * lane
  bool valid;
  __device__ bool on() const { return valid; }
  // chunk row s of the half tile: the lane's 16 bytes go to slot lane ^ 4s, the swizzle under
  // which the dQ-from-dS kernel's transposing reads are conflict-free (attn_bwd_dqs.hip)
  __device__ void store(int s, const uint32_t* v) const {
    const uint32_t ad = half + 1024 * s + (lane16 ^ (64u * s));
    *(__attribute__((address_space(3))) u32x4*)(uintptr_t)ad = u32x4{v[4 * s], v[4 * s + 1], v[4 * s + 2], v[4 * s + 3]};
  }
};

// The per-wave part of the key-owner backward: 32 keys of one (b,h), their K and V rows as
// matrix-core B operands, their dK/dV state and the query-tile step over a query tile staged in
// LDS (a "stage": Q tile, dO tile, then lse*log2(e) and D of its 64 rows, in the BwdCfg layout).
// Used by bwd_kernel (streamed query tiles) and bwd_short_kernel (all query tiles of a short
// sequence resident). F32S_ (D = 64 only) holds the state as fp32 (see below).
template <int D, bool F32S_ = false>
struct DkdvWave {
  using C = BwdCfg<D>;
  static_assert(!F32S_ || D == 64, "the fp32 state fits the register budget at D = 64 only");
  int h, key;
  float scale, sl;
  uint32_t row_rd, tr_rd, st_rd;
  u32x4 Kr[C::KC], Vr[C::KC];
  // dK^T, dV^T (m = d, n = key), chain n = dV of d tile n for n < DT, else dK of d tile n - DT.
  // Packed: bf16 pairs of accumulator rows (r, r+1); chain n runs in update block n % 2, and
  // while it runs the other block's previous chain is rounded back into the bf16 state and the
  // next chain's state is widened into it. F32S: the state is held as fp32 values that are
  // bf16-exact (at D = 64 as many registers as the packed state plus the two blocks), each
  // chain's products accumulate into it directly and it is rounded in place after every query
  // tile, one instruction per value instead of a widening and a packing; bit-identical results.
  static constexpr bool F32S = F32S_;
  uint32_t dKp[F32S ? 1 : C::DT][8], dVp[F32S ? 1 : C::DT][8];
  f32x16 acc[2];
  f32x16 st32[F32S ? 2 * C::DT : 1];
  // dS of the latest query tile, packed bf16 (index 8t + r/2); stored by the sink in the first
  // slots of the next tile (or after the last one)
  uint32_t dS[16];

  __device__ __forceinline__ void init(int lane, int key_, float scale_) {
    h = lane >> 5;
    key = key_;
    scale = scale_;
    sl = scale_ * kLog2e;
    const int l32 = lane & 31, g16 = lane >> 4, s16 = lane & 15;
    row_rd = 2 * (l32 * C::P + 8 * h);  // S / dP A operand: row = q, 8 d at 16c + 8h
    // dV^T / dK^T A operand (dO^T, Q^T) by tr reads: group g = lane/16 covers d = 16(g%2) .. +15
    // of a 32-d tile; source lane s = lane%16 points at query row 4h + s/4 (+8 for the second read)
    tr_rd = 2 * ((4 * h + (s16 >> 2)) * C::P + 16 * (g16 & 1) + 4 * (s16 & 3));
    st_rd = 4 * (4 * h);  // statistics of query row 32t + 8g + 4h + i at +4(32t + 8g + i)
    if constexpr (F32S) {
#pragma unroll
      for (int n = 0; n < 2 * C::DT; ++n) st32[n] = zero16();
    } else {
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dKp[dt][i] = 0u;
          dVp[dt][i] = 0u;
        }
      acc[0] = zero16();
      acc[1] = zero16();
    }
  }
  // own K and V rows: lane holds row `key_ld`, d = 16c + 8h .. +7
  __device__ __forceinline__ void load_rows(const uint16_t* Kg, const uint16_t* Vg, int key_ld, int rs) {
#pragma unroll
    for (int c = 0; c < C::KC; ++c) {
      Kr[c] = *(const u32x4*)(Kg + (size_t)key_ld * rs + 16 * c + 8 * h);
      Vr[c] = *(const u32x4*)(Vg + (size_t)key_ld * rs + 16 * c + 8 * h);
    }
  }
  __device__ __forceinline__ uint32_t* state(int n) { return n < C::DT ? dVp[n] : dKp[n - C::DT]; }
  __device__ __forceinline__ void pack_pairs(int n, int u0, int u1) {  // state(n)[u] = bf16 pair of block n % 2
#pragma unroll
    for (int u = u0; u < u1; ++u) {
      uint32_t v = pack_bf16(acc[n & 1][2 * u], acc[n & 1][2 * u + 1]);
      pin(v);
      state(n)[u] = v;
    }
  }
  __device__ __forceinline__ void unpack_pairs(int n, int u0, int u1) {  // block n % 2 = widened state(n)
#pragma unroll
    for (int u = u0; u < u1; ++u) {
      float lo = bf_lo(state(n)[u]), hi = bf_hi(state(n)[u]);
      pin(lo, hi);
      acc[n & 1][2 * u] = lo;
      acc[n & 1][2 * u + 1] = hi;
    }
  }
  // F32S: values r0 .. r1-1 of chain n rounded in place to bf16
  __device__ __forceinline__ void round_chain(int n, int r0, int r1) {
#pragma unroll
    for (int r = r0; r < r1; r += 2) {
      float a = round_bf16(st32[n][r]), b = round_bf16(st32[n][r + 1]);
      pin(a, b);
      st32[n][r] = a;
      st32[n][r + 1] = b;
    }
  }
  // the last chain of the last query tile back into the state
  __device__ __forceinline__ void finish() {
    if constexpr (F32S)
      round_chain(2 * C::DT - 1, 0, 16);
    else
      pack_pairs(2 * C::DT - 1, 0, 8);
  }
  // dK, dV rows of this lane's key (d = 32dt + 8g + 4h + i)
  __device__ __forceinline__ void store_rows(uint16_t* dKg, uint16_t* dVg) {
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = 32 * dt + 8 * g + 4 * h;
        // D = 64: dK was carried times 8 (see ds_pair); the division is exact
        if constexpr (F32S) {
          const f32x16& k_ = st32[C::DT + dt];
          const f32x16& v_ = st32[dt];
          *(u32x2*)(dKg + d0) = u32x2{pack_bf16(k_[4 * g] * 0.125f, k_[4 * g + 1] * 0.125f),
                                      pack_bf16(k_[4 * g + 2] * 0.125f, k_[4 * g + 3] * 0.125f)};
          *(u32x2*)(dVg + d0) = u32x2{pack_bf16(v_[4 * g], v_[4 * g + 1]), pack_bf16(v_[4 * g + 2], v_[4 * g + 3])};
        } else {
          if (D == 64)
            for (int u = 2 * g; u < 2 * g + 2; ++u) dKp[dt][u] = pack_bf16(bf_lo(dKp[dt][u]) * 0.125f, bf_hi(dKp[dt][u]) * 0.125f);
          *(u32x2*)(dKg + d0) = u32x2{dKp[dt][2 * g], dKp[dt][2 * g + 1]};
          *(u32x2*)(dVg + d0) = u32x2{dVp[dt][2 * g], dVp[dt][2 * g + 1]};
        }
      }
  }

  // One query tile (rows qb*64 ..) staged at LDS byte address qbase_a: NS matrix-core
  // instructions in a fixed order, one per slot, each slot also doing a slice of vector work that
  // does not depend on it. Slots:
  //   [0, KC) S of rows 0-31, d step c     [KC, 2KC) dP of rows 0-31
  //   [2KC, 3KC) S of rows 32-63           [3KC, 4KC) dP of rows 32-63
  //   [4KC, NS) update chain n = (i - 4KC) / 4, query step j = (i - 4KC) % 4
  // S[t], dP[t] hold rows q = 32t + 8(r/4) + 4h + r%4 of the tile, lane = key. The previous
  // tile's dS goes to `prev` in slots 0-3 (it is rewritten from slot 2KC on).
  template <bool DIAG, class Sink>
  __device__ __forceinline__ void qtile(int qb, uint32_t qbase_a, const Sink& prev) {
    constexpr int NS = 4 * C::KC + 8 * C::DT;
    constexpr int PPS = 8 / C::KC;  // score pairs of vector work per S/dP slot
    // per-lane LDS bases of this stage, computed once and anchored so that every operand address
    // below is base + constant (the constant goes into the instruction's offset field)
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
        if constexpr (F32S)
          st32[n] = mfma(op, u32x4{src[4 * j], src[4 * j + 1], src[4 * j + 2], src[4 * j + 3]}, st32[n]);
        else
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
      if (Sink::kOn && i < 4 && prev.on()) prev.store(i, dS);  // previous tile's dS (rewritten from slot 2KC on)
      if constexpr (F32S) {
        // the previous tile's last chain rounded in the first KC slots, chain n - 1 while chain n
        // runs (its first two query steps)
        if (i < C::KC) {
          round_chain(2 * C::DT - 1, (i * 16) / C::KC, ((i + 1) * 16) / C::KC);
        } else if (i >= 4 * C::KC) {
          const int k = i - 4 * C::KC, n = k / 4, j = k % 4;
          if (n >= 1 && j < 2) round_chain(n - 1, 8 * j, 8 * j + 8);
        }
      } else if (i < C::KC) {
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
  }
};

// D = 64 without the dS store: three workgroups per CU (168 VGPRs, a few spilled outside the
// product loop), 6-8% faster than two. D = 64 with the dS store: two workgroups per CU and the
// fp32 dK/dV state. D = 128 needs its 244-253 VGPRs and runs two.
template <int D, bool DS>
__global__ void __launch_bounds__(256, (D == 64 && !DS) ? 3 : 2) bwd_kernel(BwdArgs a) {
  using C = BwdCfg<D>;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkb = (a.T + C::BN - 1) / C::BN;
  int pair, kb;
  decode_workgroup(blockIdx.x, a.B * a.H, nkb, false, bwd_dispatch_round(D), pair, kb);
  const int b = pair / a.H, hd = pair - b * a.H;
  const int rs = a.H * D;
  const size_t base = ((size_t)b * a.T * a.H + hd) * D;
  const char* Qg = (const char*)(a.q + base);
  const char* Gg = (const char*)(a.dO + base);
  const float* lse_g = a.lse + (size_t)pair * a.T;
  const float* dd_g = a.Dv + (size_t)pair * a.T;
  const size_t tile_bytes = (size_t)C::BM * rs * 2;

  const int k0 = kb * C::BN;
  const int kw = k0 + 32 * wave;  // the wave's first key
  const bool wave_keys = kw < a.T;  // false only in the last block when T % 128 == 64
  const int key = kw + (lane & 31);
  DkdvWave<D, D == 64 && DS> wv;
  wv.init(lane, key, a.scale);
  wv.load_rows(a.k + base, a.v + base, min(key, a.T - 1), rs);  // rows past T are read in bounds, never stored

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

  // this wave's 32 keys are half hw of key tile ktw; dS tile (qt, ktw) of the pair's triangle
  const int ktw = kb * (C::BN / 64) + (wave >> 1), hw = wave & 1;
  const int nqt = a.T / 64;
  const size_t tri = (size_t)pair * ((size_t)nqt * (nqt + 1) / 2);
  auto ds_sink = [&](int qt) -> GlobalDsSink {
    if (!DS || !wave_keys || ktw > qt) return GlobalDsSink{nullptr};
    return GlobalDsSink{(char*)a.dS + (tri + (size_t)qt * (qt + 1) / 2 + ktw) * 8192 + hw * 4096 + lane * 16};
  };
  using Sink = typename std::conditional<DS, GlobalDsSink, NoDsSink>::type;
  auto sink_of = [&](int qt) -> Sink {
    if constexpr (DS) return ds_sink(qt);
    else return NoDsSink{};
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
  Sink prev = sink_of(-1);
  for (; qb < nqb && qb < qb0 + 2; ++qb, ++it) {
    if (qb + 1 < nqb) issue_tile(qb + 1, (it + 1) & 1);
    wv.template qtile<true>(qb, smem_a + (it & 1) * C::STAGE, prev);
    prev = sink_of(qb);
    __builtin_amdgcn_s_waitcnt(0);
    if (qb + 1 < nqb) scale_lse((it + 1) & 1);
    __syncthreads();
  }
  for (; qb < nqb; ++qb, ++it) {
    if (qb + 1 < nqb) issue_tile(qb + 1, (it + 1) & 1);
    wv.template qtile<false>(qb, smem_a + (it & 1) * C::STAGE, prev);
    prev = sink_of(qb);
    __builtin_amdgcn_s_waitcnt(0);
    if (qb + 1 < nqb) scale_lse((it + 1) & 1);
    __syncthreads();
  }
  wv.finish();
  if (Sink::kOn && prev.on())
    for (int s = 0; s < 4; ++s) prev.store(s, wv.dS);

  // ---- dK, dV: lane = key, rows d = 32dt + 8g + 4h + i ----
  if (!wave_keys) return;
  wv.store_rows(a.dK + base + (size_t)key * rs, a.dV + base + (size_t)key * rs);
}


// Short sequences (D = 64, T <= 256; the reference's own shape is T = 256): one persistent
// workgroup of 8 waves per CU takes (b,h) pairs in turn and does each pair's whole backward, in
// one launch and without a workspace. LDS holds all query tiles of the pair (bwd_kernel's stage
// layout, one stage per tile), the pair's K rows and the dS tiles of one query tile.
//   * Step qt (all waves in step): wave w owns one 32-key group and, when the group lies at or
//     below query tile qt, runs the DkdvWave step on it and leaves its dS tile in LDS (the
//     workspace's layout, swizzled as the dQ-from-dS kernel's copies are). Waves w and w + 4
//     share a SIMD and own key groups g and nkg - 1 - g.
//   * Then waves 0-3, one per SIMD, compute dQ of query tile qt = dS.K over its key tiles (a
//     32 d x 32 query block each), in the order of attn_bwd_dqs.hip.
//   * The next pair's tile qt - 1 is copied into the stage step qt - 1 freed, and its K and V rows
//     are loaded after the last step, so every copy has the rest of the pair to land.
// dK and dV are bit-identical to bwd_kernel's, dQ to the dQ-from-dS kernel's; with ACC the result
// is added into dQ (flashAttentionBackward's contract), else written.
constexpr int kShortT = 256;
constexpr int kShortQT = kShortT / 64;

template <bool ACC>
__global__ void __launch_bounds__(512, 1) bwd_short_kernel(BwdArgs a) {
  constexpr int D = 64;
  using C = BwdCfg<D>;
  constexpr int KREG = kShortQT * C::STAGE;   // K rows of the pair: key * 2D bytes, 32 KB
  constexpr int DSB = KREG + kShortT * 2 * D;  // dS tiles (qt, kt) of the current query tile at DSB + kt * 8 KB
  static_assert(C::STAGE % 1024 == 0 && C::TBYTES % 1024 == 0 && KREG % 1024 == 0 && DSB % 1024 == 0, "1 KB granules");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[DSB + kShortQT * 8192];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31, g16 = lane >> 4, s16 = lane & 15;
  const int npairs = a.B * a.H;
  const int rs = a.H * D;
  const size_t tile_bytes = (size_t)C::BM * rs * 2;
  const int nqt = a.T / 64, nkg = a.T / 32;
  const uint32_t smem_a = lds_addr_b(smem);
  auto base_of = [&](int pair) -> size_t {
    const int b = pair / a.H, hd = pair - b * a.H;
    return ((size_t)b * a.T * a.H + hd) * D;
  };

  // Stage copies: 2*PER row instructions (Q then dO, bwd_kernel's padded slot order) spread over
  // the 8 waves, instruction n by wave n % 8; lse and D by wave 2 (lanes 0-15 and 16-31; 32-63
  // repeat them).
  constexpr int PER = C::TBYTES / 1024;
  constexpr int NCP = (2 * PER + 7) / 8;
  uint32_t off[NCP];
#pragma unroll
  for (int j = 0; j < NCP; ++j) {
    const int n = wave + 8 * j, i = n >= PER ? n - PER : n;
    const int sl = 64 * i + lane, row = sl / C::SLOTS, c = min(sl % C::SLOTS, D / 8 - 1);
    off[j] = (uint32_t)(row * rs * 2 + c * 16);
  }
  auto issue_tile = [&](int pair, int qt) {  // tile qt of `pair` into stage qt
    const size_t bq = base_of(pair) * 2 + (size_t)qt * tile_bytes;
    const uint32_t dst = smem_a + qt * C::STAGE;
#pragma unroll
    for (int j = 0; j < NCP; ++j) {
      const int n = wave + 8 * j;
      if (n < 2 * PER) {
        const bool go = n >= PER;
        const int i = go ? n - PER : n;
        dma16(off[j], (const char*)(go ? a.dO : a.q) + bq, dst + (go ? C::TBYTES : 0) + 1024 * i);
      }
    }
    if (wave == 2) {
      const float* src = (l32 < 16 ? a.lse : a.Dv) + (size_t)pair * a.T + qt * C::BM + 4 * (l32 & 15);
      dma16_v(src, dst + C::STAT);
    }
  };

  // key group of this wave: g and nkg - 1 - g share a SIMD (waves w and w + 4)
  const int g = wave < 4 ? (wave < nkg ? wave : -1) : (nkg - 1 - (wave - 4) >= 4 ? nkg - 1 - (wave - 4) : -1);
  const int kt = g >> 1, hw = g & 1;
  const int key = 32 * (g < 0 ? 0 : g) + l32;
  // dQ block of waves 0-3: d half wd, query half nq (32 d x 32 queries of the query tile)
  const int wd = wave & 1, nq = (wave >> 1) & 1;
  // operand lanes as in attn_bwd_dqs.hip; K row r holds chunk p at LDS chunk p ^ kx(r)
  auto kx = [](int r) { return 4 * ((r >> 1) & 1); };
  const int ra = 8 * (g16 >> 1) + (s16 >> 2);
  const int ca = (wd * 32) / 8 + 2 * (g16 & 1) + ((s16 & 3) >> 1);
  const uint32_t a_lane = (uint32_t)(ra * 2 * D + 16 * (ca ^ kx(ra)) + 8 * (s16 & 1));
  const int cr = 2 * (g16 & 1) + ((s16 & 3) >> 1), slq = 8 * (g16 >> 1) + (s16 >> 2);
  uint32_t b_lane[2];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
    b_lane[hi] = (uint32_t)(cr * 1024 + 16 * ((slq + 4 * hi) ^ (4 * cr)) + 8 * (s16 & 1) + (32 * nq) * 16);
  const int qin = 32 * (l32 >> 4) + 8 * ((l32 >> 2) & 3) + 4 * nq + (l32 & 3);  // this lane's query row

  int pair = blockIdx.x;
  if (pair >= npairs) return;
  DkdvWave<D, true> wv;
  wv.init(lane, key, a.scale);
  for (int t = 0; t < nqt; ++t) issue_tile(pair, t);
  if (g >= 0) wv.load_rows(a.k + base_of(pair), a.v + base_of(pair), key, rs);
  for (;;) {
    const size_t base = base_of(pair);
    const int next = pair + (int)gridDim.x;
    const bool more = next < npairs;
    __builtin_amdgcn_s_waitcnt(0);  // this pair's tiles and rows (copied during the previous pair)
    if (wave == 2) {                // lse -> lse*log2(e), by the wave that copied it: exponents are base 2
      for (int t = 0; t < nqt; ++t) {
        float* l2 = (float*)(smem + t * C::STAGE + C::STAT);
        l2[lane] = l2[lane] * kLog2e;
      }
    }
    if (g >= 0) {
#pragma unroll
      for (int c = 0; c < C::KC; ++c)
        *(__attribute__((address_space(3))) u32x4*)(uintptr_t)(smem_a + KREG + key * 2 * D + 16 * ((2 * c + h) ^ kx(key))) =
            wv.Kr[c];
    }
    __syncthreads();

    for (int qt = 0; qt < nqt; ++qt) {
      if (qt >= 1 && more) issue_tile(next, qt - 1);  // stage qt - 1 was last read in step qt - 1
      // dK/dV step of the wave's key group; its dS tile (qt, kt) into LDS
      if (g >= 0 && kt <= qt) {
        if (qt == kt)
          wv.template qtile<true>(qt, smem_a + qt * C::STAGE, NoDsSink{});
        else
          wv.template qtile<false>(qt, smem_a + qt * C::STAGE, NoDsSink{});
        const LdsDsSink sink{smem_a + DSB + (uint32_t)(kt * 8192 + hw * 4096), 16u * lane, true};
#pragma unroll
        for (int s = 0; s < 4; ++s) sink.store(s, wv.dS);
      }
      __syncthreads();  // every dS tile of query tile qt is in LDS
      if (wave < 4) {
        float* dQg = a.dQ + base + (size_t)qt * 64 * rs + wd * 32 + 4 * h + (size_t)qin * rs;
        f32x4 old[4];
        if (ACC) {  // loads in flight during the products
#pragma unroll
          for (int gg = 0; gg < 4; ++gg) old[gg] = *(const f32x4*)(dQg + 8 * gg);
        }
        // products i = 4 k2 + ks in order, each one's operands read one product ahead
        auto operands = [&](int i, u32x4& A, u32x4& Bv) {
          const int k2 = i >> 2, ks = i & 3;
          const uint32_t da = smem_a + DSB + k2 * 8192 + b_lane[0] + 4 * (ks >> 1) * 1024 + (16 * (ks & 1)) * 16;
          const uint32_t ad = smem_a + KREG + k2 * 8192 + a_lane + 16 * ks * 2 * D;
          const u32x2 blo = lds_tr_b(da), bhi = lds_tr_b(da - b_lane[0] + b_lane[1]);
          const u32x2 alo = lds_tr_b(ad), ahi = lds_tr_b(ad + 4 * 2 * D);
          A = u32x4{alo[0], alo[1], ahi[0], ahi[1]};
          Bv = u32x4{blo[0], blo[1], bhi[0], bhi[1]};
        };
        f32x16 acc = zero16();
        const int np = 4 * (qt + 1);
        u32x4 A0, B0, A1, B1;
        operands(0, A0, B0);
        for (int i = 0; i < np; i += 2) {  // np is a multiple of 4
          operands(i + 1, A1, B1);
          acc = mfma(A0, B0, acc);
          if (i + 2 < np) operands(i + 2, A0, B0);
          acc = mfma(A1, B1, acc);
        }
        // the stored dS are 8 dS (power-of-two scale folded): dQ = acc / 8 exactly
#pragma unroll
        for (int gg = 0; gg < 4; ++gg) {
          f32x4 v = f32x4{acc[4 * gg], acc[4 * gg + 1], acc[4 * gg + 2], acc[4 * gg + 3]} * 0.125f;
          if (ACC) v = old[gg] + v;
          *(f32x4*)(dQg + 8 * gg) = v;
        }
      }
      __syncthreads();  // the dS tiles are free for the next step
    }
    if (g >= 0) {
      wv.finish();
      wv.store_rows(a.dK + base + (size_t)key * rs, a.dV + base + (size_t)key * rs);
    }
    if (!more) break;
    issue_tile(next, nqt - 1);
    wv.init(lane, key, a.scale);
    if (g >= 0) wv.load_rows(a.k + base_of(next), a.v + base_of(next), key, rs);
    pair = next;
  }
}

bool backward_is_short(int T, int D) { return D == 64 && T <= kShortT; }

hipError_t launch_backward_short(const BwdArgs& a, bool accumulate, hipStream_t s) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    return hipErrorInvalidDevice;
  const dim3 grid((unsigned)std::min(a.B * a.H, cus));  // one persistent workgroup per CU
  if (accumulate)
    hipLaunchKernelGGL((bwd_short_kernel<true>), grid, dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((bwd_short_kernel<false>), grid, dim3(512), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_backward(const BwdArgs& a, int D, hipStream_t s) {
  const int nkb = (a.T + kBwdBlockN - 1) / kBwdBlockN;
  const dim3 grid((unsigned)(a.B * a.H * nkb));
  if (a.dS) {
    // at D = 64 the workspace entry point stores no dS (workspace_recomputes, backward_is_short)
    if (D == 64) return hipErrorInvalidValue;
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
