// attn_launch.hpp -- host-side launch interface between the C ABI (attn_abi.hip) and the
// kernels (attn_fwd.hip, attn_bwd.hip, attn_computed.hip). Shapes arrive validated.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mla {

// Q/K/V/O/dO/dQ/dK/dV are [B,T,H,D] (row of one token = H*D elements); LSE and D are [B,H,T].
struct FwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  float* lse;
  int T, H, B;
  float scale;  // 1/sqrt(D) in fp32, as the reference computes it (attention.metal:109)
};

struct ComputeDArgs {
  const uint16_t* dO;
  const uint16_t* O;
  float* Dv;
  int T, H, B;
};

struct BwdArgs {
  const uint16_t* dO;
  const float* Dv;
  const float* lse;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  float* dQ;
  uint16_t* dK;
  uint16_t* dV;
  int T, H, B;
  float scale;
  // Optional: the dS tiles of the causal lower triangle, bf16, written by launch_backward and
  // read by launch_backward_dqs (ds_scratch_bytes(); layout in attn_bwd_dqs.hip). NULL: not stored.
  uint16_t* dS = nullptr;
};

// Bytes of the dS tile store for B*H pairs of T rows: one 64x64 bf16 tile per (query tile,
// key tile <= query tile) of every pair.
inline size_t ds_scratch_bytes(int B, int H, int T) {
  const size_t nqt = (size_t)T / 64;
  return (size_t)B * H * (nqt * (nqt + 1) / 2) * 8192;
}

hipError_t launch_forward(const FwdArgs& a, int D, hipStream_t s);
void forward_prepare();  // device queries of launch_forward, done ahead of a stream capture
hipError_t launch_compute_d(const ComputeDArgs& a, int D, hipStream_t s);
hipError_t launch_backward(const BwdArgs& a, int D, hipStream_t s);     // dK, dV (key-owner)
// dQ (query-owner, recomputing dS): added into dQ (accumulate) or written
hipError_t launch_backward_dq(const BwdArgs& a, int D, bool accumulate, hipStream_t s);
hipError_t launch_backward_dqs(const BwdArgs& a, int D, hipStream_t s); // dQ from the stored dS
// Short sequences (D = 64, T <= 256): dK, dV and dQ of a (b,h) pair by one workgroup, one launch,
// no workspace; dQ added into (accumulate) or written.
bool backward_is_short(int T, int D);
// Whether the workspace entry point runs the recomputing kernels (dK/dV without the dS store, then
// dQ written) instead of the dS round trip. Yes at D = 64: the dK/dV kernel without the store runs
// three workgroups per CU and the pair is faster (config 2 step 0.436 -> 0.41 ms, config 4's
// 0.733 -> 0.716 ms); T <= 256 runs the fused short backward instead (backward_is_short). No at
// D = 128, where the round trip saves two of the seven products.
inline bool workspace_recomputes(int T, int D) { return D == 64 && T > 256; }
hipError_t launch_backward_short(const BwdArgs& a, bool accumulate, hipStream_t s);

// Dispatch chunk sizes, in workgroups per XCD group. The backward's is one round of resident
// workgroups: two per CU on the 32 CUs of an MI355X XCD (the three-per-CU D = 64 kernels use the
// same figure). The forward's is two rounds: measured at T = 4096, D = 128 with one round per
// chunk, two and four, the forward took 1.345, 1.275 and 1.29 ms and the dK/dV kernel 2.31,
// 2.39 and 2.37 ms.
constexpr int kFwdDispatchRound = 128;
constexpr int kBwdDispatchRound = 64;
// At D = 64 the backward's kernels (dK/dV without the dS store, the recomputing dQ kernel) run
// three workgroups per CU, 96 per XCD, and their chunks span two such rounds. Measured on one box
// (the workspace backward at config 2 and at config 4's attention shape): chunks of 64, 96, 192
// workgroups and all of an XCD's pairs in one chunk gave 0.317, 0.325, 0.306, 0.303 ms and 0.263,
// 0.272, 0.240, 0.239 ms; with 64 the last chunk's long blocks started late and ran alone.
constexpr int kBwdDispatchRound64 = 192;
__host__ __device__ inline int bwd_dispatch_round(int D) { return D == 64 ? kBwdDispatchRound64 : kBwdDispatchRound; }

// Pairs per dispatch chunk: enough that one chunk's blocks fill a round of resident workgroups.
__host__ __device__ inline int dispatch_chunk(int nblk, int group_slots) {
  const int c = (group_slots + nblk - 1) / nblk;
  return c > 1 ? c : 1;
}

// Workgroup -> (pair = b*H + h, block) decode shared by host tests and kernels. Pairs are
// spread so that every block of one pair lands on the same XCD (workgroups are handed to the
// 8 XCDs round-robin by id). A group's pairs are taken in chunks of dispatch_chunk(nblk, round)
// pairs (round: workgroups per XCD group, kFwdDispatchRound or bwd_dispatch_round(D)); inside
// a chunk the blocks go out block-major, the largest causal work first, across the chunk's pairs:
//   forward : block = query block, longest (last) first
//   backward: block = key block, longest (first) first
// The hardware starts workgroups in id order as slots free up, so the long blocks of the last
// pairs no longer start late and run alone at the end (pair by pair, the tail was up to one long
// block), while the workgroups running at once still share a few pairs' tiles in L2.
__host__ __device__ inline void decode_workgroup(int bid, int npairs, int nblk, bool last_first, int round,
                                                 int& pair, int& blk) {
  const bool grouped = (npairs & 7) == 0;  // 8 groups, one per XCD
  const int g = grouped ? 8 : 1;
  const int x = grouped ? (bid & 7) : 0, slot = grouped ? (bid >> 3) : bid;
  const int npx = npairs / g;  // pairs of this group
  const int C = dispatch_chunk(nblk, grouped ? round : 8 * round);
  const int chunk = slot / (C * nblk);
  const int r = slot - chunk * C * nblk;
  const int cc = C < npx - chunk * C ? C : npx - chunk * C;  // pairs in this chunk (the last may be short)
  const int local = r / cc;
  pair = (chunk * C + (r - local * cc)) * g + x;
  blk = last_first ? (nblk - 1 - local) : local;
}

// Item k of workgroup `bid` of a persistent grid of `grid` workgroups over npairs x nblk
// (pair, block) items; false when the workgroup has fewer than k + 1 items. When both the pair
// count and the grid are multiples of 8, the workgroups on XCD x (bid % 8 == x) serve the pairs
// p = x (mod 8), so all blocks of a pair share one L2; otherwise all workgroups form one group.
// A group's items are listed pair by pair, each pair's last (largest causal) block first, and
// dealt in snake order over its workgroups, so each workgroup gets about the same work.
__host__ __device__ inline bool fwd_item_of(int bid, int grid, int k, int npairs, int nblk, int& pair, int& blk) {
  const int G = ((npairs & 7) == 0 && (grid & 7) == 0) ? 8 : 1;
  const int x = bid % G, w = bid / G, W = grid / G;
  const int m = k * W + ((k & 1) ? W - 1 - w : w);
  if (m >= npairs / G * nblk) return false;
  const int j = m / nblk, local = m - j * nblk;
  pair = j * G + x;
  blk = nblk - 1 - local;
  return true;
}

constexpr int kFwdBlockM = 128;  // query rows per forward workgroup
// The forward runs persistent (each resident workgroup takes items in turn, the next item's first
// tiles loaded during the current item's last step) when there are at most this many (pair, query
// block) items per resident workgroup; with more, one workgroup per item in the chunked dispatch
// order balances better. Measured: persistent faster at two items per slot (config 1, and config
// 4's attention, 0.0855 against 0.090 ms), one workgroup per item faster at four (config 2,
// 0.110 against 0.1155 ms) and at sixteen (T = 4096, D = 128).
constexpr int kFwdPersistItems = 2;
constexpr int kBwdBlockN = 128;  // keys owned by one dK/dV workgroup
constexpr int kDqBlockM = 128;   // query rows owned by one dQ workgroup
constexpr int kTile = 64;        // the reference's TILE_M = TILE_N (attention.metal:14-15)

}  // namespace mla
