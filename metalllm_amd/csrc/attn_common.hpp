// attn_common.hpp -- gfx950 device helpers shared by the attention kernels.
//
// Matrix-core operand layouts (v_mfma_f32_32x32x16_bf16, one wave of 64 lanes, h = lane/32):
//   A (32 x 16): lane holds A[m = lane%32][k = 8h .. 8h+7]      (8 bf16 = 4 dwords)
//   B (16 x 32): lane holds B[k = 8h .. 8h+7][n = lane%32]
//   C (32 x 32): lane holds C[m = 8(r/4) + 4h + r%4][n = lane%32], r = 0..15 (16 fp32)
// The instruction adds its 16 products to C in two passes (k 0-7, then k 8-15); which logical k
// a lane slot carries is the caller's choice as long as A and B agree.
//
// ds_read_b64_tr_b16: within each group of 16 lanes, lane j receives column j of a 4 x 16 block
// of bf16 (4 rows), where source lane s of the group supplies the address of row s/4, columns
// 4(s%4)..4(s%4)+3.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mla {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

// Global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4): lane l reads sbase + voff
// and writes LDS byte address m0 + 16 l. Issued as inline asm, so the compiler does not track
// the copy: the caller waits for it (s_waitcnt vmcnt) before a barrier that precedes any read
// of the destination. The compiler-tracked builtin would make the first LDS read after it (of
// any buffer) wait for every copy in flight, which serialises double-buffered tile copies with
// the computation on the other buffer.
__device__ __forceinline__ void dma16(uint32_t voff, const void* sbase, uint32_t m0) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}
// Same with a per-lane 64-bit source address.
__device__ __forceinline__ void dma16_v(const void* src, uint32_t m0) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}
// s_waitcnt vmcnt(N) only (expcnt and lgkmcnt left at their maxima): waits until at most N of this
// wave's vector-memory operations are outstanding. They complete in issue order, so this waits
// for everything issued before the last N.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Waits for every vector-memory load of this wave (the untracked copies included) and every LDS
// access, then synchronises the workgroup.
__device__ __forceinline__ void wait_all_and_barrier() {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ float bf_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf_hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

// x rounded to bf16 (nearest even), as an fp32 value: the packed pair (0, x) read as one float.
// One instruction, where rounding a pair and unpacking both halves takes three.
__device__ __forceinline__ float round_bf16(float x) { return __uint_as_float(pack_bf16(0.0f, x)); }

// Rounds a pair in place to bf16-representable fp32 values.
__device__ __forceinline__ void round_pair(float& a, float& b) {
  const uint32_t p = pack_bf16(a, b);
  a = bf_lo(p);
  b = bf_hi(p);
}

// Rounds elements r, r+1 of an accumulator in place to bf16-representable fp32 values.
__device__ __forceinline__ void round_pair(f32x16& v, int r) {
  const uint32_t p = pack_bf16(v[r], v[r + 1]);
  v[r] = bf_lo(p);
  v[r + 1] = bf_hi(p);
}

__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// max(a, b, c) in one v_max3_f32 (fmaxf would first canonicalise operands that come from bit
// operations, one extra instruction each).
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Anchors: an empty asm that reads and rewrites a value pins its computation to this point of
// the program (code motion cannot move the work into another slot of a fenced schedule).
__device__ __forceinline__ void pin(float& a, float& b) { asm volatile("" : "+v"(a), "+v"(b)); }
__device__ __forceinline__ void pin(uint32_t& a) { asm volatile("" : "+v"(a)); }

// v_permlane32_swap(x, x) returns {lanes 0-31: own, 32-63: partner} and {lanes 0-31: partner,
// 32-63: own}, partner = lane ^ 32. Combining the two with a commutative op gives every lane
// op(own, partner), bit-identical in both halves.
__device__ __forceinline__ float max_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ u32x2 lds_tr(const uint16_t* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p));
}

__device__ __forceinline__ u32x4 lds_read16(const uint16_t* p) { return *(const u32x4*)p; }

}  // namespace mla
