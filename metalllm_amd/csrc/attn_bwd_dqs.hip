// attn_bwd_dqs.hip -- the dQ half of flashAttentionBackward from stored dS tiles (query-owner).
//
// Reference: /root/reference/attention.metal:288,292-296: for each key tile kt <= qt,
// dQ[q] += dS.K, with dS = bf16(p * (dP - D) * scale) the tile the backward already computed
// (:277-286). The dK/dV kernel (attn_bwd.hip) stores every dS tile it computes, bf16, into the
// caller's workspace; this kernel is then a plain causal GEMM dQ = dS.K over that buffer: no
// recomputation of S, P or dP, so it is bound by the bytes of dS it streams (HBM), not by
// vector work. The workspace trades B*H*T^2 bytes of device memory (4.4 GB at B=H=16,
// T=4096) for the second recomputation of the softmax.
//
// dS store layout: per pair, the tiles (qt, kt <= qt) of its lower triangle in order
// qt(qt+1)/2 + kt, 8 KB each. Inside a tile, half hw (keys 32hw..32hw+31) of 4 KB holds four
// 1 KB chunk rows s = 0..3, each 64 lanes x 16 bytes: lane l = key32 + 32h carries the 8 values
// of key 32hw + key32 at query positions p = 32h + 8s + e (e = 0..7), and position p is query
// q(p) = 32t + 8j + 4h + i of the tile with p % 32 = 16t + 4j + i. That is the order the dK/dV
// kernel holds dS in its accumulators, so it stores with four full 16-byte writes per lane.
//
// Work split: a workgroup owns 128 query rows (query tiles qt0 = 2QB, qt1 = 2QB + 1) of one
// (b, h); wave w computes dQ^T of query tile qt0 + w/2 for the d half w%2. Key tiles stream
// through LDS in a two-stage ring (global_load_lds_dwordx4): the K tile (rows padded so the
// transposing reads are conflict-free) and the two dS tiles (qt0, kt), (qt1, kt). The ring is
// small enough for two workgroups per CU, so one streams while the other starts or finishes.
// Both matrix-core operands come from LDS by ds_read_b64_tr_b16: A = K^T (m = d, k = key),
// B = dS^T (k = key, n = query position). dQ goes back through LDS ([q][d] fp32) so that its
// stores are row-contiguous; every row of dQ is written once, in full.
#include <algorithm>
#include <atomic>

#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

template <int D>
struct DqsCfg {
  static constexpr int QT = 2;                       // query tiles per workgroup
  // K row pitch (elements): 320 or 192 bytes, so that the 4 rows x 64 bytes one half-wave of a
  // ds_read_b64_tr_b16 touches (32 lanes, the LDS's 256 bytes per cycle) fall in distinct banks
  static constexpr int KP = (D == 128) ? 160 : 96;
  static constexpr int SLOTS = KP / 8;               // 16-byte slots per padded K row = copy instructions
  static constexpr int KPW = (SLOTS + 3) / 4;        // K copy instructions per wave
  static constexpr int KBYTES = 64 * KP * 2;
  static constexpr int SBLK = 1024 + 64;             // padded 1 KB chunk row of a dS tile
  static constexpr int DSBYTES = 8 * SBLK;           // one dS tile
  static constexpr int STAGE = KBYTES + QT * DSBYTES;
  static constexpr int NSTAGE = 2;
  static constexpr int MB = D / 64;                  // 32-row d blocks per wave
  static constexpr int DH = D / 2;                   // d columns per wave
  static constexpr int DQP = DH + 4;                 // fp32 row pitch of the dQ transpose
};

// dma16 with the non-temporal hint: dS tiles are read once.
__device__ __forceinline__ void dma16_nt(uint32_t voff, const void* sbase, uint32_t m0) {
  asm volatile("global_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

typedef __attribute__((address_space(3))) i16x4 lds_i16x4_q;
__device__ __forceinline__ u32x2 tr_at(uint32_t byte_addr) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_q*)(uintptr_t)byte_addr));
}

template <int D>
__global__ void __launch_bounds__(256, 2) dqs_kernel(BwdArgs a) {
  using C = DqsCfg<D>;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::NSTAGE * C::STAGE];
  static_assert(C::NSTAGE * C::STAGE >= 4 * 64 * C::DQP * 4, "dQ transpose fits in the stages");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31, g16 = lane >> 4, s16 = lane & 15;
  const int nqt = a.T / 64;
  const int nqb = (nqt + C::QT - 1) / C::QT;
  int pair, qblk;
  decode_workgroup(blockIdx.x, a.B * a.H, nqb, true, pair, qblk);
  const int b = pair / a.H, hd = pair - b * a.H;
  const int rs = a.H * D;
  const size_t base = ((size_t)b * a.T * a.H + hd) * D;
  const int qt0 = C::QT * qblk;
  const int nk = min(qt0 + C::QT, nqt);  // key tiles 0 .. last query tile of the block
  const int wq = wave >> 1, wd = wave & 1;
  const int qtw = qt0 + wq;
  const bool wave_q = qtw < nqt;
  const char* Kg = (const char*)(a.k + base);
  const char* dsg = (const char*)a.dS + (size_t)pair * ((size_t)nqt * (nqt + 1) / 2) * 8192;

  // K copy: slot s -> row s / SLOTS, chunk s % SLOTS (pad chunks re-read the row's last chunk);
  // a wave whose last instruction index is past SLOTS repeats its first one
  uint32_t koff[C::KPW], kdst[C::KPW];
#pragma unroll
  for (int j = 0; j < C::KPW; ++j) {
    const int ins = wave + 4 * j < C::SLOTS ? wave + 4 * j : wave;
    const int s = 64 * ins + lane, row = s / C::SLOTS, c = min(s % C::SLOTS, D / 8 - 1);
    koff[j] = (uint32_t)(row * rs * 2 + c * 16);
    kdst[j] = 1024u * ins;
  }
  const uint32_t smem_a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)smem;
  auto issue = [&](int kt, int stage) {
    const uint32_t dst = smem_a + stage * C::STAGE;
    const char* ks = Kg + (size_t)kt * 64 * rs * 2;
#pragma unroll
    for (int j = 0; j < C::KPW; ++j) dma16(koff[j], ks, dst + kdst[j]);
    // dS tiles (qt0 + t, kt); a tile outside the triangle (or past T) reads the pair's first tile
    // instead and is never used
#pragma unroll
    for (int j = 0; j < 2 * C::QT; ++j) {
      const int ins = wave + 4 * j, t = ins >> 3, row = ins & 7;
      const int qt = qt0 + t;
      const bool valid = qt < nqt && kt <= qt;
      const char* src = dsg + (valid ? ((size_t)qt * (qt + 1) / 2 + kt) * 8192 : 0);
      dma16_nt((uint32_t)(lane * 16 + row * 1024), src, dst + C::KBYTES + t * C::DSBYTES + row * C::SBLK);
    }
  };

  // per-lane operand addresses (bytes within a stage)
  // A = K^T: group g16 covers d 16(g16%2)..+15 of a 32-d block, source lane s16 reads key
  // 8(g16/2) + s16/4 (+4 for the second read), d 4(s16%4)..+3
  const uint32_t a_lane =
      2 * ((8 * (g16 >> 1) + (s16 >> 2)) * C::KP + 16 * (g16 & 1) + 4 * (s16 & 3)) + wd * D;
  // B = dS^T: the same keys; query positions p = 32nb + 16(g16%2) + 4(s16%4)..+3
  const uint32_t b_lane = C::KBYTES + wq * C::DSBYTES + (2 * (g16 & 1) + ((s16 & 3) >> 1)) * C::SBLK +
                          (8 * (g16 >> 1) + (s16 >> 2)) * 16 + 8 * (s16 & 1);

  f32x16 acc[C::MB][2];
#pragma unroll
  for (int m = 0; m < C::MB; ++m) acc[m][0] = acc[m][1] = zero16();

  auto compute = [&](int stage) {
    const uint32_t sa = smem_a + stage * C::STAGE;
    const uint32_t ab = sa + a_lane, bb = sa + b_lane;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 Bo[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const uint32_t bd = bb + 4 * (ks >> 1) * C::SBLK + (16 * (ks & 1) + 32 * nb) * 16;
        const u32x2 lo = tr_at(bd), hi = tr_at(bd + 4 * 16);
        Bo[nb] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
#pragma unroll
      for (int m = 0; m < C::MB; ++m) {
        const uint32_t ad = ab + 2 * (16 * ks * C::KP + 32 * m);
        const u32x2 lo = tr_at(ad), hi = tr_at(ad + 2 * 4 * C::KP);
        const u32x4 A = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[m][nb] = mfma(A, Bo[nb], acc[m][nb]);
      }
    }
  };

  issue(0, 0);
  for (int kt = 0; kt < nk; ++kt) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of stage kt landed (the only ones in flight)
    __syncthreads();                // everyone's landed; everyone is done with stage kt - 1
    if (kt + 1 < nk) issue(kt + 1, (kt + 1) & 1);
    if (wave_q && kt <= qtw) compute(kt & 1);
  }

  // ---- dQ = dQ^T of this wave, through LDS: lane holds query position p = 32nb + l32 ----
  __syncthreads();  // every wave is done reading the stages
  float* buf = (float*)smem + wave * 64 * C::DQP;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int qin = 32 * (l32 >> 4) + 8 * ((l32 >> 2) & 3) + 4 * nb + (l32 & 3);
#pragma unroll
    for (int m = 0; m < C::MB; ++m)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(f32x4*)(buf + qin * C::DQP + 32 * m + 8 * g + 4 * h) =
            f32x4{acc[m][nb][4 * g], acc[m][nb][4 * g + 1], acc[m][nb][4 * g + 2], acc[m][nb][4 * g + 3]};
  }
  __builtin_amdgcn_s_waitcnt(0);  // own LDS writes done (each wave reads back only its own rows)
  if (!wave_q) return;
  float* dQg = a.dQ + base + (size_t)qtw * 64 * rs + wd * C::DH;
  constexpr int LPR = C::DH / 4;      // lanes per row (4 floats each)
  constexpr int RPI = 64 / LPR;       // rows per instruction
  const int rl = lane / LPR, cl = 4 * (lane % LPR);
#pragma unroll 4
  for (int r = 0; r < 64; r += RPI) {
    *(f32x4*)(dQg + (size_t)(r + rl) * rs + cl) = *(const f32x4*)(buf + (r + rl) * C::DQP + cl);
  }
}

// Persistent form of dqs_kernel (same work split, operands and results), used when the pair
// count is a multiple of 8: a grid of two workgroups per CU, where the workgroups on XCD x serve
// the pairs p = x (mod 8), so each pair's K tiles stay in one L2. That XCD's (pair, query block)
// items are listed pair by pair, each pair's blocks largest first, and dealt in snake order
// across its workgroups. Workgroups working at the same time then share one or two pairs'
// K tiles, and every workgroup gets about the same number of key tiles (a large block in one row
// of the deal meets a small one in the next). Stages
// run back to back across item boundaries: the first stage of the next item is copied while the
// last one of the current item is computed, and the item's dQ is stored straight from the
// accumulators (16-byte stores, row segments that L2 merges into whole lines), those stores
// completing while the next item's first stage is computed.
template <int D>
__global__ void __launch_bounds__(256, 2) dqs_persistent_kernel(BwdArgs a) {
  using C = DqsCfg<D>;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::NSTAGE * C::STAGE];
  constexpr int NSTORE = C::MB * 2 * 4;  // dQ store instructions per wave per item

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31, g16 = lane >> 4, s16 = lane & 15;
  const int nqt = a.T / 64;
  const int nqb = (nqt + C::QT - 1) / C::QT;
  const int P8 = a.B * a.H / 8;                         // pairs per XCD
  const int x = blockIdx.x & 7, w = blockIdx.x >> 3, Wx = gridDim.x >> 3;
  const int nlist = P8 * nqb;                           // items on this XCD
  const int rs = a.H * D;
  const int wq = wave >> 1, wd = wave & 1;
  const size_t ntri = (size_t)nqt * (nqt + 1) / 2;

  // item k of this workgroup -> list index (snake order) -> (pair, query block)
  auto list_index = [&](int k) { return k * Wx + ((k & 1) ? Wx - 1 - w : w); };
  struct Item {
    int pair, qt0, nk;
  };
  auto item_at = [&](int m) -> Item {
    const int j = m / nqb, local = m - j * nqb;
    const int qblk = nqb - 1 - local;
    const int qt0 = C::QT * qblk;
    return Item{8 * j + x, qt0, min(qt0 + C::QT, nqt)};
  };
  auto base_of = [&](int pair) -> size_t {
    const int b = pair / a.H, hd = pair - b * a.H;
    return ((size_t)b * a.T * a.H + hd) * D;
  };

  uint32_t koff[C::KPW], kdst[C::KPW];
#pragma unroll
  for (int j = 0; j < C::KPW; ++j) {
    const int ins = wave + 4 * j < C::SLOTS ? wave + 4 * j : wave;
    const int s = 64 * ins + lane, row = s / C::SLOTS, c = min(s % C::SLOTS, D / 8 - 1);
    koff[j] = (uint32_t)(row * rs * 2 + c * 16);
    kdst[j] = 1024u * ins;
  }
  const uint32_t smem_a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)smem;
  auto issue = [&](const Item& it, int kt, int stage) {
    const uint32_t dst = smem_a + stage * C::STAGE;
    const char* ks = (const char*)(a.k + base_of(it.pair)) + (size_t)kt * 64 * rs * 2;
#pragma unroll
    for (int j = 0; j < C::KPW; ++j) dma16(koff[j], ks, dst + kdst[j]);
    const char* dsg = (const char*)a.dS + (size_t)it.pair * ntri * 8192;
#pragma unroll
    for (int j = 0; j < 2 * C::QT; ++j) {
      const int ins = wave + 4 * j, t = ins >> 3, row = ins & 7;
      const int qt = it.qt0 + t;
      const bool valid = qt < nqt && kt <= qt;
      const char* src = dsg + (valid ? ((size_t)qt * (qt + 1) / 2 + kt) * 8192 : 0);
      dma16_nt((uint32_t)(lane * 16 + row * 1024), src, dst + C::KBYTES + t * C::DSBYTES + row * C::SBLK);
    }
  };

  const uint32_t a_lane =
      2 * ((8 * (g16 >> 1) + (s16 >> 2)) * C::KP + 16 * (g16 & 1) + 4 * (s16 & 3)) + wd * D;
  const uint32_t b_lane = C::KBYTES + wq * C::DSBYTES + (2 * (g16 & 1) + ((s16 & 3) >> 1)) * C::SBLK +
                          (8 * (g16 >> 1) + (s16 >> 2)) * 16 + 8 * (s16 & 1);

  f32x16 acc[C::MB][2];
#pragma unroll
  for (int m = 0; m < C::MB; ++m) acc[m][0] = acc[m][1] = zero16();

  auto compute = [&](int stage) {
    const uint32_t sa = smem_a + stage * C::STAGE;
    const uint32_t ab = sa + a_lane, bb = sa + b_lane;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 Bo[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const uint32_t bd = bb + 4 * (ks >> 1) * C::SBLK + (16 * (ks & 1) + 32 * nb) * 16;
        const u32x2 lo = tr_at(bd), hi = tr_at(bd + 4 * 16);
        Bo[nb] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
#pragma unroll
      for (int m = 0; m < C::MB; ++m) {
        const uint32_t ad = ab + 2 * (16 * ks * C::KP + 32 * m);
        const u32x2 lo = tr_at(ad), hi = tr_at(ad + 2 * 4 * C::KP);
        const u32x4 A = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[m][nb] = mfma(A, Bo[nb], acc[m][nb]);
      }
    }
  };

  int k = 0, m = list_index(0);
  if (m >= nlist) return;  // more workgroups than items on this XCD
  Item cur = item_at(m);
  // the next stage to copy: item kn at key tile ktn
  int kn = 0, ktn = 0;
  Item nxt = cur;
  bool have_next = true;
  auto advance_next = [&]() {
    if (++ktn == nxt.nk) {
      ktn = 0;
      const int mn = list_index(++kn);
      have_next = mn < nlist;
      if (have_next) nxt = item_at(mn);
    }
  };
  issue(nxt, ktn, 0);
  advance_next();
  bool stored = false;  // this wave's dQ stores were issued after the copies now awaited
  int kt = 0;
  for (int t = 0;; ++t) {
    if (stored)
      wait_vm<NSTORE>();  // the copies of stage t landed; the previous item's stores may be in flight
    else
      wait_vm<0>();
    __syncthreads();
    if (have_next) {
      issue(nxt, ktn, (t + 1) & 1);
      advance_next();
    }
    const int qtw = cur.qt0 + wq;
    const bool wave_q = qtw < nqt;
    if (wave_q && kt <= qtw) compute(t & 1);
    stored = false;
    if (++kt < cur.nk) continue;
    // ---- item done: dQ = dQ^T of this wave, lane holds query position p = 32nb + l32 ----
    if (wave_q) {
      float* dQg = a.dQ + base_of(cur.pair) + (size_t)qtw * 64 * rs + wd * C::DH + 4 * h;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int qin = 32 * (l32 >> 4) + 8 * ((l32 >> 2) & 3) + 4 * nb + (l32 & 3);
#pragma unroll
        for (int mm = 0; mm < C::MB; ++mm)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            *(f32x4*)(dQg + (size_t)qin * rs + 32 * mm + 8 * g) =
                f32x4{acc[mm][nb][4 * g], acc[mm][nb][4 * g + 1], acc[mm][nb][4 * g + 2], acc[mm][nb][4 * g + 3]};
      }
      stored = true;
    }
#pragma unroll
    for (int mm = 0; mm < C::MB; ++mm) acc[mm][0] = acc[mm][1] = zero16();
    m = list_index(++k);
    if (m >= nlist) break;
    cur = item_at(m);
    kt = 0;
  }
}

hipError_t launch_backward_dqs(const BwdArgs& a, int D, hipStream_t s) {
  const int nqb = (a.T / 64 + 1) / 2;
  const int npairs = a.B * a.H;
  if (npairs % 8 == 0) {
    // CU count of the current device (cached per device; the query does not touch the stream)
    static std::atomic<int> cu_cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipErrorInvalidDevice;
    int cus = dev < 64 ? cu_cache[dev].load(std::memory_order_relaxed) : 0;
    if (cus <= 0) {
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return hipErrorInvalidDevice;
      if (dev < 64) cu_cache[dev].store(cus, std::memory_order_relaxed);
    }
    // two workgroups per CU, a multiple of 8 (one share per XCD), no more than there are items
    const int items = npairs * nqb;
    const int per_xcd = std::max(1, std::min((2 * cus) / 8, items / 8));
    const dim3 grid((unsigned)(8 * per_xcd));
    if (D == 64)
      hipLaunchKernelGGL(dqs_persistent_kernel<64>, grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(dqs_persistent_kernel<128>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)(npairs * nqb));
  if (D == 64)
    hipLaunchKernelGGL(dqs_kernel<64>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(dqs_kernel<128>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace mla
