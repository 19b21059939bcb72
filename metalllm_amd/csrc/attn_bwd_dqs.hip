// attn_bwd_dqs.hip -- the dQ half of flashAttentionBackward from stored dS tiles (query-owner).
//
// Reference: /root/reference/attention.metal:288,292-296: for each key tile kt <= qt,
// dQ[q] += dS.K, with dS = bf16(p * (dP - D) * scale) the tile the backward already computed
// (:277-286). The dK/dV kernel (attn_bwd.hip) stores every dS tile it computes, bf16, into the
// caller's workspace; this kernel is then a plain causal GEMM dQ = dS.K over that buffer: no
// recomputation of S, P or dP, so it is bound by the bytes it copies, not by vector work. The
// workspace trades B*H*T^2 bytes of device memory (4.4 GB at B=H=16, T=4096) for the second
// recomputation of the softmax.
//
// dS store layout: per pair, the tiles (qt, kt <= qt) of its lower triangle in order
// qt(qt+1)/2 + kt, 8 KB each. Inside a tile, half hw (keys 32hw..32hw+31) of 4 KB holds four
// 1 KB chunk rows s = 0..3, each 64 lanes x 16 bytes: lane l = key32 + 32h carries the 8 values
// of key 32hw + key32 at query positions p = 32h + 8s + e (e = 0..7), and position p is query
// q(p) = 32t + 8j + 4h + i of the tile with p % 32 = 16t + 4j + i. That is the order the dK/dV
// kernel holds dS in its accumulators, so it stores with four full 16-byte writes per lane. At
// D = 64 the tiles hold 8 dS (the power-of-two scale 1/8 is applied to dQ when it is stored).
//
// Work split: an item is QT query tiles (64 rows each) of one (b, h); wave w of the workgroup
// computes dQ^T of query tile qt0 + w/2 for the d half w%2, over key tiles 0 .. qt0 + QT - 1.
// Key steps stream through LDS in a ring of NSTAGE stages (global_load_lds_dwordx4), each
// holding the K tile and the QT dS tiles (qt0 + t, kt): step t waits for stage t, copies stage
// t + NSTAGE - 1 and computes stage t. Both matrix-core operands come from LDS by
// ds_read_b64_tr_b16: A = K^T (m = d, k = key), B = dS^T (k = key, n = query position).
// The kernel is bound by the copies: dS streams from HBM once, and each K tile is copied again
// for every item (from L2), so long sequences use QT = 4 with 8 waves, one workgroup per CU and
// three stages (two in flight: the K copies per dS byte halve and the bytes in flight double);
// short ones, whose items would be too few for the CUs, use QT = 2 with 4 waves, two workgroups
// per CU and two stages.
//
// LDS layout, no padding: K rows and dS chunk rows are XOR-swizzled in 16-byte chunks so that
// the transposing reads are conflict-free (the 4 rows x 64 bytes that 32 lanes of one
// ds_read_b64_tr_b16 touch fall in distinct banks). K row r, LDS chunk p holds K chunk
// p ^ kx(r), kx(r) = 4(r % 4) (D = 128, 16 chunks a row) or 4((r / 2) % 2) (D = 64, 8 chunks);
// dS chunk row c, LDS slot s holds the row's slot s ^ 4(c % 4). A copy lane fetches the global
// chunk that belongs at its LDS slot, so the copies stay whole 16-byte transfers within a row.
//
// Scheduling (persistent): when the pair count is a multiple of 8, the workgroups on XCD x
// serve the pairs p = x (mod 8), so each pair's K tiles stay in one L2; otherwise all
// workgroups form one group. A group's (pair, query block) items are listed pair by pair, each
// pair's blocks largest first, and dealt in snake order across its workgroups: workgroups
// working at the same time share one or two pairs' K tiles, and every workgroup gets about the
// same number of key steps. Stages run back to back across item boundaries, and an item's dQ is
// stored straight from the accumulators while the next item's stages are computed. Every row of
// dQ is written once, in full. The products are computed as dQ = dS.K (m = query position, n = d;
// the same operand registers as dQ^T = K^T.dS^T, the same sums bit for bit) so that a lane holds
// one d of 16 rows: each 4-byte store writes 32 consecutive d of a row per half wave, whole
// 128-byte lines (with dQ^T each 16-byte store wrote 32-byte pieces of 32 rows; c3 1.047 ->
// 1.015 ms, c2 0.113 -> 0.109 ms). The vmcnt waits saturate at 63: with 64 stores per item a
// wait may also cover a few of them, which only waits longer.
#include <algorithm>
#include <atomic>

#include "attn_common.hpp"
#include "attn_launch.hpp"

namespace mla {

template <int D, int QT_, int NSTAGE_>
struct DqsCfg {
  static constexpr int QT = QT_;                       // query tiles per item
  static constexpr int NSTAGE = NSTAGE_;               // ring stages
  static constexpr int WAVES = 2 * QT;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int KCH = D / 8;                    // 16-byte chunks per K row
  static constexpr int KBYTES = 64 * D * 2;
  static constexpr int KINS = KBYTES / 1024;           // K copy instructions per stage
  static constexpr int DSBYTES = 8192;
  static constexpr int DSPW = 8 * QT / WAVES;          // dS copy instructions per wave (4)
  static constexpr int STAGE = KBYTES + QT * DSBYTES;
  static constexpr int KPW = KINS / WAVES;             // K copy instructions per wave
  static constexpr int CPW = KPW + DSPW;               // copy instructions per wave and stage
  static constexpr int MB = D / 64;                    // 32-row d blocks per wave
  static constexpr int DH = D / 2;                     // d columns per wave
  static constexpr int NSTORE = MB * 2 * 16;           // dQ store instructions per wave and item
  static constexpr int WG_PER_CU = NSTAGE * STAGE <= 80 * 1024 ? 2 : 1;
  static_assert(KINS % WAVES == 0, "K copies split evenly over the waves");
  static_assert(NSTAGE == 2 || NSTAGE == 3, "ring depth");

};

// dma16 with the non-temporal hint: dS tiles are read once.
__device__ __forceinline__ void dma16_nt(uint32_t voff, const void* sbase, uint32_t m0) {
  asm volatile("global_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

typedef __attribute__((address_space(3))) i16x4 lds_i16x4_q;
__device__ __forceinline__ u32x2 tr_at(uint32_t byte_addr) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_q*)(uintptr_t)byte_addr));
}

// s_waitcnt takes an immediate: waits with the first of Ns equal to n, or with 0 (everything)
// when none is.
// (counts above 63, the counter's range, wait for everything but the last 63)
template <int N, int... Rest>
__device__ __forceinline__ void wait_vm_of(int n) {
  if (n == N) {
    wait_vm<(N < 63 ? N : 63)>();
  } else {
    if constexpr (sizeof...(Rest) > 0)
      wait_vm_of<Rest...>(n);
    else
      wait_vm<0>();
  }
}

template <int D, int QT, int NSTAGE>
__global__ void __launch_bounds__(128 * QT, (NSTAGE * (128 * D + 8192 * QT) <= 80 * 1024 ? 2 : 1))
dqs_kernel(BwdArgs a) {  // (THREADS, WG_PER_CU of DqsCfg)
  using C = DqsCfg<D, QT, NSTAGE>;
  // the stored dS tiles of D = 64 hold 8 dS (the dK/dV kernel folds the power-of-two scale 1/8
  // into the stores of dK and dQ): dQ = (sum of 8 dS . K) / 8, exact
  constexpr float kDsUnit = D == 64 ? 0.125f : 1.0f;
  static_assert(C::THREADS == 128 * QT && C::WG_PER_CU == (NSTAGE * C::STAGE <= 80 * 1024 ? 2 : 1), "launch bounds");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::NSTAGE * C::STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = lane >> 5, l32 = lane & 31, g16 = lane >> 4, s16 = lane & 15;
  const int nqt = a.T / 64;
  const int nqb = (nqt + C::QT - 1) / C::QT;
  const int npairs = a.B * a.H;
  const int G = npairs % 8 == 0 ? 8 : 1;               // groups (XCDs when 8)
  const int x = blockIdx.x % G, w = blockIdx.x / G, Wx = gridDim.x / G;
  const int nlist = npairs / G * nqb;                   // items of this group
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
    const int qt0 = C::QT * (nqb - 1 - local);
    return Item{G * j + x, qt0, min(qt0 + C::QT, nqt)};
  };
  auto base_of = [&](int pair) -> size_t {
    const int b = pair / a.H, hd = pair - b * a.H;
    return ((size_t)b * a.T * a.H + hd) * D;
  };
  auto kx = [](int r) { return D == 128 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); };

  // copies of a stage: K instructions wave + WAVES*j (LDS slot L = 64*ins + lane: row L / KCH,
  // chunk L % KCH); dS instructions d = wave + WAVES*j, tile d / 8, chunk row d % 8
  uint32_t koff[C::KPW], dsoff[C::DSPW], dsdst[C::DSPW];
#pragma unroll
  for (int j = 0; j < C::KPW; ++j) {
    const int L = 64 * (wave + C::WAVES * j) + lane, r = L / C::KCH, p = L % C::KCH;
    koff[j] = (uint32_t)(r * rs * 2 + 16 * (p ^ kx(r)));
  }
#pragma unroll
  for (int j = 0; j < C::DSPW; ++j) {
    const int d = wave + C::WAVES * j, t = d >> 3, row = d & 7;
    dsoff[j] = (uint32_t)(row * 1024 + 16 * (lane ^ (4 * (row & 3))));
    dsdst[j] = (uint32_t)(C::KBYTES + t * C::DSBYTES + row * 1024);
  }
  const uint32_t smem_a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)smem;
  // Copy cursor: the next stage to copy is key tile ktn of item nxt. Its source addresses are
  // set up once per item (set_cursor) and advanced by one tile per stage, so issuing a stage costs
  // a few scalar adds (every wave of the CU shares the scalar unit of its SIMD with the others).
  //   kp       K tile ktn of the item's pair
  //   dsp[j]   dS tile (qt0 + (wave + WAVES*j)/8, ktn) of the pair's triangle
  //   qlim[j]  that query tile, or -1 past T: copy j is valid while ktn <= qlim[j]; an invalid one
  //            reads the pair's first tile (ds0) instead and is never used
  const size_t ktile = (size_t)64 * rs * 2;
  const char* kp = nullptr;
  const char* ds0 = nullptr;
  const char* dsp[C::DSPW];
  int qlim[C::DSPW];
  auto set_cursor = [&](const Item& it) {
    kp = (const char*)(a.k + base_of(it.pair));
    ds0 = (const char*)a.dS + (size_t)it.pair * ntri * 8192;
#pragma unroll
    for (int j = 0; j < C::DSPW; ++j) {
      const int qt = it.qt0 + (wave + C::WAVES * j) / 8;
      qlim[j] = qt < nqt ? qt : -1;
      dsp[j] = ds0 + (qt < nqt ? (size_t)qt * (qt + 1) / 2 * 8192 : 0);
    }
  };
  auto issue = [&](int kt, int stage) {
    const uint32_t dst = smem_a + stage * C::STAGE;
#pragma unroll
    for (int j = 0; j < C::KPW; ++j) dma16(koff[j], kp, dst + 1024 * (wave + C::WAVES * j));
#pragma unroll
    for (int j = 0; j < C::DSPW; ++j) dma16_nt(dsoff[j], kt <= qlim[j] ? dsp[j] : ds0, dst + dsdst[j]);
  };

  // A = K^T: group g16 covers d 16(g16%2)..+15 of 32-d block m, source lane s16 reads key
  // 8(g16/2) + s16/4 (+4 for the second read, +16ks per k step), d 4(s16%4)..+3; the row's
  // swizzle depends on s16/4 only, so each m has one per-lane base
  uint32_t a_lane[C::MB];
#pragma unroll
  for (int m = 0; m < C::MB; ++m) {
    const int r = 8 * (g16 >> 1) + (s16 >> 2);
    const int c = (wd * C::DH + 32 * m) / 8 + 2 * (g16 & 1) + ((s16 & 3) >> 1);
    a_lane[m] = (uint32_t)(r * 2 * D + 16 * (c ^ kx(r)) + 8 * (s16 & 1));
  }
  // B = dS^T: the same keys (chunk row 4(ks/2) + cr), query positions 32nb + 16(g16%2) +
  // 4(s16%4)..+3 (slot 16(ks%2) + 32nb + sl, +4 for the second read)
  const int cr = 2 * (g16 & 1) + ((s16 & 3) >> 1), sl = 8 * (g16 >> 1) + (s16 >> 2);
  uint32_t b_lane[2];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
    b_lane[hi] = (uint32_t)(C::KBYTES + wq * C::DSBYTES + cr * 1024 + 16 * ((sl + 4 * hi) ^ (4 * cr)) + 8 * (s16 & 1));

  f32x16 acc[C::MB][2];
#pragma unroll
  for (int m = 0; m < C::MB; ++m) acc[m][0] = acc[m][1] = zero16();

  auto compute = [&](int stage) {
    const uint32_t sa = smem_a + stage * C::STAGE;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 Bo[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const uint32_t o = 4 * (ks >> 1) * 1024 + (16 * (ks & 1) + 32 * nb) * 16;
        const u32x2 lo = tr_at(sa + b_lane[0] + o), hi = tr_at(sa + b_lane[1] + o);
        Bo[nb] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
#pragma unroll
      for (int m = 0; m < C::MB; ++m) {
        const uint32_t ad = sa + a_lane[m] + 16 * ks * 2 * D;
        const u32x2 lo = tr_at(ad), hi = tr_at(ad + 4 * 2 * D);
        const u32x4 A = u32x4{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[m][nb] = mfma(Bo[nb], A, acc[m][nb]);  // dQ (m = query, n = d)
      }
    }
  };

  int k = 0, m = list_index(0);
  if (m >= nlist) return;  // more workgroups than items in this group
  Item cur = item_at(m);
  // copy cursor: the next stage to copy is item kn at key tile ktn
  int kn = 0, ktn = 0;
  Item nxt = cur;
  bool have_next = true;
  auto advance_next = [&]() {
    if (++ktn == nxt.nk) {
      ktn = 0;
      const int mn = list_index(++kn);
      have_next = mn < nlist;
      if (have_next) {
        nxt = item_at(mn);
        set_cursor(nxt);
      }
    } else {
      kp += ktile;
#pragma unroll
      for (int j = 0; j < C::DSPW; ++j) dsp[j] += 8192;
    }
  };
  set_cursor(nxt);
  issue(ktn, 0);
  advance_next();
  // Vector-memory operations this wave issued after the copies of the stage awaited next (they
  // complete in issue order): with three stages the copies of the stage after it (c1), and the
  // dQ stores of the previous step (s1) and, with three stages, of the step before (s2).
  bool c1 = false, s1 = false, s2 = false;
  if (C::NSTAGE == 3 && have_next) {
    issue(ktn, 1);
    advance_next();
    c1 = true;
  }
  int kt = 0, st = 0;
  for (;;) {
    const int n_after = (c1 ? C::CPW : 0) + (s1 ? C::NSTORE : 0) + (s2 ? C::NSTORE : 0);
    if (C::NSTAGE == 3)
      wait_vm_of<C::CPW, C::NSTORE, C::CPW + C::NSTORE, 2 * C::NSTORE, C::CPW + 2 * C::NSTORE>(n_after);
    else
      wait_vm_of<C::NSTORE>(n_after);
    __syncthreads();  // stage st landed for every wave; every wave is done with the previous stage
    if (C::NSTAGE == 3) c1 = have_next;
    if (have_next) {
      issue(ktn, st == 0 ? C::NSTAGE - 1 : st - 1);  // stage (st + NSTAGE - 1) % NSTAGE
      advance_next();
    }
    const int qtw = cur.qt0 + wq;
    const bool wave_q = qtw < nqt;
    if (wave_q && kt <= qtw) compute(st);
    st = st == C::NSTAGE - 1 ? 0 : st + 1;
    if (C::NSTAGE == 3) s2 = s1;
    s1 = false;
    if (++kt < cur.nk) continue;
    // ---- item done: lane holds d = 32mm + l32 of query positions x = 8(r/4) + 4h + r%4 of block
    // nb (position p = 32nb + x is query row 32(x/16) + 8((x/4)%4) + 4nb + x%4 of the tile); one
    // store writes 32 consecutive d of one row per half wave: whole 128-byte lines ----
    if (wave_q) {
      float* dQg = a.dQ + base_of(cur.pair) + (size_t)qtw * 64 * rs + wd * C::DH + l32;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int x = 8 * (r >> 2) + 4 * h + (r & 3);
          const int qin = 32 * (x >> 4) + 8 * ((x >> 2) & 3) + 4 * nb + (x & 3);
#pragma unroll
          for (int mm = 0; mm < C::MB; ++mm) dQg[(size_t)qin * rs + 32 * mm] = acc[mm][nb][r] * kDsUnit;
        }
      s1 = true;
    }
#pragma unroll
    for (int mm = 0; mm < C::MB; ++mm) acc[mm][0] = acc[mm][1] = zero16();
    m = list_index(++k);
    if (m >= nlist) break;
    cur = item_at(m);
    kt = 0;
  }
}

template <int D, int QT, int NSTAGE>
static hipError_t launch_ring(const BwdArgs& a, int cus, hipStream_t s) {
  using C = DqsCfg<D, QT, NSTAGE>;
  const int npairs = a.B * a.H;
  const int G = npairs % 8 == 0 ? 8 : 1;
  const int items = npairs * ((a.T / 64 + QT - 1) / QT);
  // resident workgroups, a multiple of the group count, no more than there are items
  const int per_group = std::max(1, std::min(C::WG_PER_CU * cus / G, items / G));
  hipLaunchKernelGGL((dqs_kernel<D, QT, NSTAGE>), dim3((unsigned)(G * per_group)), dim3(C::THREADS), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_backward_dqs(const BwdArgs& a, int D, hipStream_t s) {
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
  // four query tiles per item from 512 keys on (T = 256 has a single such item per pair)
  const bool deep = a.T >= 512;
  if (D == 64)
    return deep ? launch_ring<64, 4, 3>(a, cus, s) : launch_ring<64, 2, 2>(a, cus, s);
  return deep ? launch_ring<128, 4, 3>(a, cus, s) : launch_ring<128, 2, 2>(a, cus, s);
}

}  // namespace mla
