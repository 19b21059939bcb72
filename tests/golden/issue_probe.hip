// issue_probe.hip -- test-only library: measures how many SIMD cycles a "slot" of
// {one v_mfma_f32_32x32x16_bf16 + V vector ALU instructions (+ one ds_read_b128)} takes on
// gfx950, with 1 or 2 waves per SIMD. The attention kernels are written as sequences of such
// slots, so this table turns their counted instructions into time floors.
// Built by __graft_entry__.build() into tests/golden/libissue_probe.so; run by
// tests/test_gpu_issue_probe.py.
//
// Each wave runs `iters` iterations of 16 slots. Slot s: (optionally) one ds_read_b128 into
// buffer s % 4 and an s_waitcnt that leaves at most two reads in flight, then one MFMA on two
// alternating accumulators whose B operand is the buffer read two slots earlier, then V vector
// instructions from a fixed rotation over eight independent registers:
//   fma v,v,v | add v,v | cvt_pk_bf16_f32 (0, x) | mul v,v | max v,v | fma v,v,v | add v,v |
//   fma v,s,v (or v_exp_f32 in the "exp" mix, one in eight)
// which is the mix of forms the attention kernels' softmax and rounding work uses.
// Every LDS read stays inside the 64 KB array (lane * 16 + slot * 1024 + 16 <= 16 KB + 1 KB).
// Result: cycles per SIMD slot = a wave's s_memtime span / (iters * 16) / waves per SIMD,
// the 90th percentile over the workgroups (one workgroup of 4 waves per CU and wave per SIMD).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kSlots = 16;

template <bool EXP>
__device__ __forceinline__ void vop(int k, float* x, const float* y, float s) {
  const int r = k & 7;
  if (EXP && r == 7) asm volatile("v_exp_f32 %0, %0" : "+v"(x[r]));
  else if (r == 0 || r == 5) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[r]) : "v"(y[0]), "v"(y[1]));
  else if (r == 1 || r == 6) asm volatile("v_add_f32 %0, %0, %1" : "+v"(x[r]) : "v"(y[2]));
  else if (r == 2) asm volatile("v_cvt_pk_bf16_f32 %0, 0, %1" : "+v"(x[r]) : "v"(y[3]));
  else if (r == 3) asm volatile("v_mul_f32 %0, %0, %1" : "+v"(x[r]) : "v"(y[4]));
  else if (r == 4) asm volatile("v_max_f32 %0, %0, %1" : "+v"(x[r]) : "v"(y[5]));
  else asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[r]) : "s"(s), "v"(y[6]));
}

template <int V, bool LDS, bool EXP>
__global__ void __launch_bounds__(256) slot_probe(float* out, long long* cyc, int iters, float sc) {
  __shared__ __attribute__((aligned(16))) float lds[64 * 1024 / 4];
  const int gid = blockIdx.x * blockDim.x + threadIdx.x;
  for (int i = threadIdx.x; i < 64 * 1024 / 4; i += 256) lds[i] = (float)(i & 1023) * 1e-3f;
  __syncthreads();
  f32x16 acc0, acc1;
  for (int i = 0; i < 16; ++i) acc0[i] = acc1[i] = 0.0f;
  const u32x4 a = {0x3f803f80u + threadIdx.x, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
  u32x4 b[4];
  for (int i = 0; i < 4; ++i) b[i] = u32x4{0x3f803f80u, 0x3f803f80u + threadIdx.x, 0x3f803f80u, 0x3f803f80u};
  float x[8], y[8];
  for (int i = 0; i < 8; ++i) {
    x[i] = lds[(threadIdx.x + i) & 255] * 1e-7f + i;
    y[i] = 0.5f + i * 1e-3f;
  }
  const uint32_t lbase =
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)lds + (threadIdx.x & 63) * 16;
  const long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      if (LDS) {
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "+v"(b[s & 3]) : "v"(lbase), "i"(s * 1024));
        asm volatile("s_waitcnt lgkmcnt(2)" ::: "memory");
      }
      if (s & 1)
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc1) : "v"(a), "v"(b[(s + 2) & 3]));
      else
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc0) : "v"(a), "v"(b[(s + 2) & 3]));
#pragma unroll
      for (int k = 0; k < V; ++k) vop<EXP>(k + s * V, x, y, sc);
    }
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n s_nop 15\n s_nop 15\n s_nop 15" ::: "memory");
  const long long t1 = __builtin_amdgcn_s_memtime();
  float sum = 0.0f;
  for (int i = 0; i < 16; ++i) sum += acc0[i] + acc1[i];
  for (int i = 0; i < 8; ++i) sum += x[i];
  for (int i = 0; i < 4; ++i) sum += __builtin_bit_cast(float, b[i][0] & 0x7fffffu);
  out[gid] = sum;
  if (threadIdx.x == 0) cyc[blockIdx.x] = t1 - t0;
}

typedef void (*ProbeFn)(float*, long long*, int, float);

template <int V>
ProbeFn pick(bool lds, bool ex) {
  if (lds) return ex ? slot_probe<V, true, true> : slot_probe<V, true, false>;
  return ex ? slot_probe<V, false, true> : slot_probe<V, false, false>;
}

ProbeFn probe_for(int v, bool lds, bool ex) {
  switch (v) {
    case 0: return pick<0>(lds, ex);
    case 2: return pick<2>(lds, ex);
    case 4: return pick<4>(lds, ex);
    case 6: return pick<6>(lds, ex);
    case 8: return pick<8>(lds, ex);
    case 10: return pick<10>(lds, ex);
    case 12: return pick<12>(lds, ex);
    case 14: return pick<14>(lds, ex);
    case 16: return pick<16>(lds, ex);
    case 20: return pick<20>(lds, ex);
    case 24: return pick<24>(lds, ex);
    default: return nullptr;
  }
}

}  // namespace

// cycles per SIMD slot for V in {0,2,...,16,20,24} vector instructions per slot; waves 1 or 2
// per SIMD; lds, ex: 0/1. Returns 0, or a negative code (bad arguments, HIP error).
extern "C" int issue_probe_run(int waves, int v, int lds, int ex, int iters, double* cycles_per_slot) {
  if (waves < 1 || waves > 2 || iters < 1 || iters > 100000 || !cycles_per_slot) return -1;
  const ProbeFn fn = probe_for(v, lds != 0, ex != 0);
  if (!fn) return -1;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || cus <= 0) return -2;
  const int blocks = waves * cus;
  float* out = nullptr;
  long long* cyc = nullptr;
  if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) != hipSuccess) return -2;
  if (hipMalloc(&cyc, (size_t)blocks * sizeof(long long)) != hipSuccess) {
    (void)hipFree(out);
    return -2;
  }
  int rc = 0;
  for (int rep = 0; rep < 2 && rc == 0; ++rep) {  // the first launch warms up clocks and caches
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), 0, 0, out, cyc, iters, 0.999f);
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) rc = -3;
  }
  std::vector<long long> h(blocks);
  if (rc == 0 && hipMemcpy(h.data(), cyc, blocks * sizeof(long long), hipMemcpyDeviceToHost) != hipSuccess) rc = -3;
  (void)hipFree(out);
  (void)hipFree(cyc);
  if (rc) return rc;
  std::sort(h.begin(), h.end());
  *cycles_per_slot = (double)h[(size_t)blocks * 9 / 10] / iters / kSlots / waves;
  return 0;
}
