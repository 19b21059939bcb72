// attn_bwd_dq.hip -- the dQ half of flashAttentionBackward on gfx950 (query-owner kernel).
//
// Reference: /root/reference/attention.metal:270-296. For a query row q and every key k <= q:
//   S = bf16(Q.K^T), dP = bf16(dO.V^T)                              (:274-275)
//   p = exp(S*scale - lse[q]) (0 above the diagonal)                 (:277-282)
//   dS = bf16(p * (dP - D[q]) * scale)                               (:284)
//   dQ[q] += dS.K    (fp32 atomic add into the caller-zeroed dQ, :288,292-296)
// The reference computes dS inside the key-tile owner and adds one dQ part per (key tile,
// query tile) with fp32 atomics into dQ. Here a query-owner workgroup recomputes S, dP and dS for
// its 128 query rows over all keys, keeps dQ in matrix-core accumulators, and adds its sum to its
// rows of dQ with one read-add-write per element (the only writer of those rows, so no atomics:
// the device executes about 0.33e12 fp32 atomic adds per second, and the owner-side form, one
// atomic per element per key tile, would cost more than the whole kernel at long sequences). For
// flashAttentionBackward dQ keeps the reference's contract: the result is added to what the
// caller's buffer holds. The workspace entry point at D = 64 runs this kernel writing dQ instead.
// The dQ product sums each query's keys in fp32 across key tiles (the reference rounds each
// 64-key part to bf16 first, :288; the difference is far inside the gradient tolerance).
//
// Work split: 4 waves x 32 query rows per workgroup, two workgroups per CU (two waves per SIMD
// hide each other's LDS and barrier waits). Lane = query: the wave computes S^T and dP^T
// (keys x queries) with K and V rows from LDS as A operands and its own Q and dO rows as
// register B operands, so p, dS and the statistics lse[q], D[q] are per-lane scalars. dS^T,
// packed to bf16, is directly the B operand of dQ^T += K^T.dS^T; K^T is read with
// ds_read_b64_tr_b16 from the row-major K tile, four keys per read, in the order {8g + 4h + i}
// that lane half h of a 32-key subtile holds.
//
// Per 64-key tile the 48 matrix-core instructions (D=128) run in a fixed order, one per slot,
// each with a slice of the vector work it does not depend on: S and dP of keys 0-31, then of
// keys 32-63, then the dQ products; p and dS of the first 32 keys are computed while the
// second half's products run, and dS of the second half while the first dQ products run.
// Scheduling fences keep that order. K and V tiles go global -> LDS by
// global_load_lds_dwordx4 (no registers, untracked by the compiler), two stages: tile j+1 is
// copied while tile j is used. At the end each wave reads its 32 rows of the old dQ with
// 16-byte loads, all issued before the accumulators are transposed through LDS, and writes
// old + sum back with 16-byte stores (element-wise loads, a few in flight at a time, took a
// sixth of the kernel at T = 4096 and half of it at T = 1024).
//
// Matrix-core passes: S and dP sum d in passes of 8 consecutive values; dQ sums keys in passes
// {16c+0..3, 16c+8..11} then {16c+4..7, 16c+12..15}.
#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

template <int D>
struct DqCfg {
  static constexpr int BM = kDqBlockM;  // query rows per workgroup (128)
  static constexpr int BN = kTile;      // keys per tile (64)
  static constexpr int THREADS = 256;
  static constexpr int P = (D == 128) ? D + 24 : D + 8;  // K, V row pitch: b128 row and tr reads conflict-free
  static constexpr int TBYTES = kTile * P * 2;           // one padded tile
  static constexpr int STAGE = 2 * TBYTES;               // K, V
  static constexpr int SLOTS = P / 8;                    // 16-byte slots of a padded row (19 / 9)
  static constexpr int LPW = (SLOTS + 3) / 4;            // row-copy instructions per wave per tile (max)
  static constexpr int KC = D / 16;                      // 16-deep steps over d
  static constexpr int DT = D / 32;                      // 32-wide d tiles of dQ
  static constexpr int NM = 4 * KC + 4 * DT;             // matrix-core instructions per tile
  static constexpr int DQP = D + 4;                      // fp32 pitch of the dQ transpose buffer
  // Vector-work schedule: score pair p of half t enters its four stages in slot enter(t, p) and
  // packs dS in slot enter + 3; pairs per slot PPS (two at D=64, where there are fewer products).
  static constexpr int PPS = D == 64 ? 2 : 1;
  static constexpr int enter(int t, int p) { return (t ? 4 * KC : 2 * KC) + p / PPS; }
  // slot of dQ product k (key chunk c = k / DT, d tile k % DT): in order, after the slot that
  // packs the last dS pair of chunk c (pairs 4(c%2) .. +3 of half c/2)
  static constexpr int dq_slot(int k) {
    int slot = 4 * KC - 1;
    for (int j = 0; j <= k; ++j) {
      const int c = j / DT, ready = enter(c / 2, 4 * (c % 2) + 3) + 3;
      slot = (slot + 1 > ready + 1) ? slot + 1 : ready + 1;
    }
    return slot;
  }
  static constexpr int NV = dq_slot(4 * DT - 1) + 1;  // slots per tile
  // matrix-core product of slot i (S/dP: i < 4KC; dQ: 4KC + k), or -1
  static constexpr int product_at(int i) {
    if (i < 4 * KC) return i;
    for (int k = 0; k < 4 * DT; ++k)
      if (dq_slot(k) == i) return 4 * KC + k;
    return -1;
  }
};

typedef __attribute__((address_space(3))) uint16_t lds_u16;
__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_u16*)p; }
__device__ __forceinline__ u32x4 lds_b128_at(uint32_t byte_addr) {
  return *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)byte_addr;
}
__device__ __forceinline__ u32x2 lds_tr_at(uint32_t byte_addr) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (__attribute__((address_space(3))) i16x4*)(uintptr_t)byte_addr));
}

template <bool V>
struct BoolTag {
  static constexpr bool value = V;
};

// ACC: add the result into dQ (flashAttentionBackward's contract); otherwise write dQ.
template <int D, bool ACC>
__global__ void __launch_bounds__(256, 2) bwd_dq_kernel(BwdArgs a) {
  using C = DqCfg<D>;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31;
  const int nqb = (a.T + C::BM - 1) / C::BM;
  int pair, qb;
  decode_workgroup(blockIdx.x, a.B * a.H, nqb, true, bwd_dispatch_round(D), pair, qb);
  const int b = pair / a.H, hd = pair - b * a.H;
  const int rs = a.H * D;
  const size_t base = ((size_t)b * a.T * a.H + hd) * D;
  const uint16_t* Qg = a.q + base;
  const uint16_t* Gg = a.dO + base;
  const char* Kg = (const char*)(a.k + base);
  const char* Vg = (const char*)(a.v + base);
  const size_t tile_bytes = (size_t)C::BN * rs * 2;

  const int q0 = qb * C::BM;
  const int qw = q0 + 32 * wave;
  const bool wave_active = qw < a.T;
  const int n_tiles = (min(q0 + C::BM, a.T) - 1) / C::BN + 1;
  const int my_tiles = wave_active ? qw / C::BN + 1 : 0;  // the last one is the diagonal tile
  const int q = qw + l32;

  // Q^T and dO^T as B operands: lane holds row q, d = 16c + 8h .. +7.
  u32x4 Qr[C::KC], Gr[C::KC];
#pragma unroll
  for (int c = 0; c < C::KC; ++c) {
    Qr[c] = wave_active ? *(const u32x4*)(Qg + (size_t)q * rs + 16 * c + 8 * h) : u32x4{0, 0, 0, 0};
    Gr[c] = wave_active ? *(const u32x4*)(Gg + (size_t)q * rs + 16 * c + 8 * h) : u32x4{0, 0, 0, 0};
  }
  const float lse2 = wave_active ? a.lse[(size_t)pair * a.T + q] * kLog2e : 0.0f;  // exponent in base 2
  const float dq = wave_active ? a.Dv[(size_t)pair * a.T + q] : 0.0f;
  const float dq_scaled = dq * a.scale;  // D = 128: dS = bf16(p * fma(dP, scale, -D*scale))
  const float sl = a.scale * kLog2e;
  const float scale = a.scale;

  // Tile copy: instruction i of a tile covers 16-byte slots 64i..64i+63 of the padded tile;
  // slot s is row s / SLOTS, chunk s % SLOTS; pad chunks re-read the row's last chunk.
  uint32_t off[C::LPW];
#pragma unroll
  for (int j = 0; j < C::LPW; ++j) {
    const int sl_ = 64 * (wave + 4 * j) + lane, row = sl_ / C::SLOTS, c = min(sl_ % C::SLOTS, D / 8 - 1);
    off[j] = (uint32_t)(row * rs * 2 + c * 16);
  }
  // untracked copies (dma16): the s_waitcnt before each barrier covers them, and the LDS reads
  // of the current tile do not wait for the next tile's copy
  auto issue_tile = [&](int kt) {
    const char* ks = Kg + (size_t)kt * tile_bytes;
    const char* vs = Vg + (size_t)kt * tile_bytes;
    const uint32_t dst = lds_addr(smem + (kt & 1) * C::STAGE);
#pragma unroll
    for (int j = 0; j < C::LPW; ++j)
      if (wave + 4 * j < C::SLOTS) {
        dma16(off[j], ks, dst + 1024 * (wave + 4 * j));
        dma16(off[j], vs, dst + C::TBYTES + 1024 * (wave + 4 * j));
      }
  };

  // LDS operand addresses (bytes, within a stage).
  const uint32_t row_rd = 2 * (l32 * C::P + 8 * h);  // S^T / dP^T A operand: row = key, 8 d at 16c + 8h
  // dQ^T A operand (K^T) by tr reads: group g = lane/16 covers d = 16(g%2) .. +15 of a 32-d tile;
  // source lane s = lane%16 points at key row 4h + s/4 (+8 for the second read).
  const int g16 = lane >> 4, s16 = lane & 15;
  const uint32_t tr_rd = 2 * ((4 * h + (s16 >> 2)) * C::P + 16 * (g16 & 1) + 4 * (s16 & 3));

  f32x16 dQa[C::DT];
#pragma unroll
  for (int i = 0; i < C::DT; ++i) dQa[i] = zero16();
  uint32_t dS[16];

  // One key tile (MASK: this wave's diagonal tile). x = S^T, y = dP^T per 32-key half t; pair p
  // of half t is scores (2p, 2p+1) of register block t. Matrix-core slots: [0, 2KC) S and dP of
  // half 0 alternating (d step c = i/2), [2KC, 4KC) the same for half 1, [4KC, NM) dQ ordered by
  // key chunk c (keys 16c..16c+15) then d tile. The vector work of a pair runs in four pipelined
  // stages (1: bf16(S) and the exponent argument; 2: exp2, bf16(dP); 3: dP - D and p*(dP - D);
  // 4: *scale and packed dS), pair p of half t entering in slot DqCfg::enter(t, p); a dQ product
  // of chunk c waits (DqCfg::dq_slot) until the dS pairs of keys 16c.. are packed, which at
  // D=64 inserts slots without a product.
  auto tile = [&](int kt, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const uint32_t kb = lds_addr(smem + (kt & 1) * C::STAGE), vb = kb + C::TBYTES;
    const int key0 = kt * C::BN;
    f32x16 x0 = zero16(), x1 = zero16(), y0 = zero16(), y1 = zero16();
    // operand reads run AHEAD(i) products ahead: five during the first S/dP half (no vector work
    // there to cover the LDS latency), two afterwards
    constexpr int RING = 6;
    auto ahead = [](int i) { return i < 2 * C::KC ? 5 : 2; };
    u32x4 ring[RING];
    auto op_of = [&](int i) -> u32x4 {
      if (i < 4 * C::KC) {  // S / dP: half t, d step c
        const int t = i / (2 * C::KC), isdp = i & 1, c = (i % (2 * C::KC)) >> 1;
        return lds_b128_at((isdp ? vb : kb) + row_rd + 2 * (32 * t * C::P + 16 * c));
      }
      const int k = i - 4 * C::KC, dt = k % C::DT, c = k / C::DT;
      const u32x2 lo = lds_tr_at(kb + tr_rd + 2 * (16 * c * C::P + 32 * dt));
      const u32x2 hi = lds_tr_at(kb + tr_rd + 2 * ((16 * c + 8) * C::P + 32 * dt));
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
#pragma unroll
    for (int i = 0; i <= ahead(0); ++i) ring[i] = op_of(i);
    float da[16], db[16];  // bf16(dP) of the pairs, as fp32 values
    float ta[16], tb[16], pa[16], pb[16], ya[16], yb[16];
    // vector stage st of pair p of half t (pair index u = 8t + p)
    auto stage = [&](int t, int p, int st) {
      f32x16& x = t ? x1 : x0;
      f32x16& y = t ? y1 : y0;
      const int u = 8 * t + p, r = 2 * p;
      if (st == 0) {  // s = bf16(S); exponent argument s*scale*log2e - lse*log2e
        ta[u] = fmaf(round_bf16(x[r]), sl, -lse2);
        tb[u] = fmaf(round_bf16(x[r + 1]), sl, -lse2);
        pin(ta[u], tb[u]);
      } else if (st == 1) {  // p = exp2(.), 0 above the diagonal; bf16(dP)
        float p0 = exp2_hw(ta[u]), p1 = exp2_hw(tb[u]);
        if (MASK) {
          const int k0 = key0 + 32 * t + 8 * (r >> 2) + 4 * h + (r & 3);
          if (k0 > q) p0 = 0.0f;
          if (k0 + 1 > q) p1 = 0.0f;
        }
        pa[u] = p0;
        pb[u] = p1;
        da[u] = round_bf16(y[r]);
        db[u] = round_bf16(y[r + 1]);
        pin(pa[u], pb[u]);
        pin(da[u], db[u]);
      } else if (st == 2) {  // p * (dP - D) (D = 64), p * (dP*scale - D*scale) (D = 128)
        ya[u] = D == 64 ? pa[u] * (da[u] - dq) : pa[u] * fmaf(da[u], scale, -dq_scaled);
        yb[u] = D == 64 ? pb[u] * (db[u] - dq) : pb[u] * fmaf(db[u], scale, -dq_scaled);
        pin(ya[u], yb[u]);
      } else {  // dS = bf16(.); at D = 64 (scale 1/8, a power of two) dS is carried times 8 and dQ
                // divided once when it is stored: exact above the subnormals. At D = 128 the same
                // value as the dK/dV kernel's dS (attn_bwd.hip)
        uint32_t pk = pack_bf16(ya[u], yb[u]);
        pin(pk);
        dS[u] = pk;
      }
    };
#pragma unroll
    for (int slot = 0; slot < C::NV; ++slot) {
      const int i = C::product_at(slot);
      if (i >= 0) {
#pragma unroll
      for (int k = (i ? i - 1 + ahead(i - 1) : ahead(0)) + 1; k <= i + ahead(i) && k < C::NM; ++k)
        ring[k % RING] = op_of(k);
      const u32x4& op = ring[i % RING];
      if (i < 4 * C::KC) {
        const int t = i / (2 * C::KC), c = (i % (2 * C::KC)) >> 1;
        if (i & 1) {
          if (t) y1 = mfma(op, Gr[c], y1);
          else y0 = mfma(op, Gr[c], y0);
        } else {
          if (t) x1 = mfma(op, Qr[c], x1);
          else x0 = mfma(op, Qr[c], x0);
        }
      } else {
        const int k = i - 4 * C::KC, dt = k % C::DT, c = k / C::DT;
        dQa[dt] = mfma(op, u32x4{dS[4 * c], dS[4 * c + 1], dS[4 * c + 2], dS[4 * c + 3]}, dQa[dt]);
      }
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const int st = slot - C::enter(t, p);
          if (st >= 0 && st < 4) stage(t, p, st);
        }
      fence();
    }
  };

  // ---- key tiles 0 .. n_tiles-1; tile j+1 is copied while tile j is used ----
  issue_tile(0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // Tiles below every row of the workgroup run on every wave with one code path (inactive waves
  // of a partial last block compute on zero rows and never store), so the accumulators keep
  // their registers across iterations; the diagonal region (at most two tiles) branches per wave.
  const int full_end = min(q0 / C::BN, n_tiles);
  int j = 0;
  for (; j < full_end; ++j) {
    if (j + 1 < n_tiles) issue_tile(j + 1);
    tile(j, BoolTag<false>());
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  for (; j < n_tiles; ++j) {
    if (j + 1 < n_tiles) issue_tile(j + 1);
    if (j + 1 < my_tiles)
      tile(j, BoolTag<false>());
    else if (j + 1 == my_tiles)
      tile(j, BoolTag<true>());
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // ---- dQ += result (ACC) or dQ = result: transpose through LDS ([q][d] fp32), then row-contiguous writes ----
  // The wave's 32 rows of the old dQ are read first, as 16-byte chunks (chunk u = 64i + lane is
  // row u / (D/4), columns 4(u % (D/4)) .. +3), so the loads are in flight during the transpose.
  constexpr int NCH = 32 * D / 4 / 64;  // 16-byte chunks per lane
  float* dQg = a.dQ + base + (size_t)qw * rs;
  f32x4 old[NCH];
  if (ACC && wave_active) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int u = 64 * i + lane, r = u / (D / 4), c4 = u % (D / 4);
      old[i] = *(const f32x4*)(dQg + (size_t)r * rs + 4 * c4);
    }
  }
  float* buf = (float*)smem + wave * 32 * C::DQP;
  if (wave_active) {
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(f32x4*)(buf + l32 * C::DQP + 32 * dt + 8 * g + 4 * h) =
            f32x4{dQa[dt][4 * g], dQa[dt][4 * g + 1], dQa[dt][4 * g + 2], dQa[dt][4 * g + 3]} * (D == 64 ? 0.125f : 1.0f);
  }
  __syncthreads();
  if (!wave_active) return;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int u = 64 * i + lane, r = u / (D / 4), c4 = u % (D / 4);
    const f32x4 sum = *(const f32x4*)(buf + r * C::DQP + 4 * c4);
    *(f32x4*)(dQg + (size_t)r * rs + 4 * c4) = ACC ? old[i] + sum : sum;
  }
}

hipError_t launch_backward_dq(const BwdArgs& a, int D, bool accumulate, hipStream_t s) {
  const int nqb = (a.T + kDqBlockM - 1) / kDqBlockM;
  const dim3 grid((unsigned)(a.B * a.H * nqb));
  if (D == 64) {
    if (accumulate)
      hipLaunchKernelGGL((bwd_dq_kernel<64, true>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((bwd_dq_kernel<64, false>), grid, dim3(256), 0, s, a);
  } else {
    if (accumulate)
      hipLaunchKernelGGL((bwd_dq_kernel<128, true>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((bwd_dq_kernel<128, false>), grid, dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace mla
