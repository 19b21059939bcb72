// mfma_probe.hip -- test-only library: runs v_mfma_f32_32x32x16_bf16 on caller-provided tiles so
// the oracle's matrix-core accumulation model (oracle/attn_oracle.cpp, GEMM_MFMA) can be checked
// against the hardware. Built by __graft_entry__.build() into tests/golden/libmfma_probe.so.
//
// Tile layout (one wave per tile, operands as the instruction takes them):
//   a, b: [ntiles][64 lanes][8] bf16 bits; lane l holds A[m = l%32][k = 8(l/32)..+7] and
//         B[k = 8(l/32)..+7][n = l%32]
//   c:    [ntiles][64 lanes][16] fp32, accumulator in, result out; lane l, register r holds
//         C[m = 8(r/4) + 4(l/32) + r%4][n = l%32]
// The fixture tests/golden/mfma_rounding_cases.json holds the hand-made rounding cases that
// were recorded with this kernel (element C[0][0]); make_mfma_cases.py regenerates it.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(64) mfma_tiles(const uint16_t* a, const uint16_t* b, float* c, int ntiles) {
  const int t = blockIdx.x, l = threadIdx.x;
  if (t >= ntiles) return;
  const u32x4 av = *(const u32x4*)(a + ((size_t)t * 64 + l) * 8);
  const u32x4 bv = *(const u32x4*)(b + ((size_t)t * 64 + l) * 8);
  f32x16 acc;
  float* cp = c + ((size_t)t * 64 + l) * 16;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = cp[i];
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av), __builtin_bit_cast(bf16x8, bv), acc, 0,
                                                0, 0);
#pragma unroll
  for (int i = 0; i < 16; ++i) cp[i] = acc[i];
}

extern "C" int mfma_probe_run(const uint16_t* a, const uint16_t* b, float* c, int ntiles, void* stream) {
  if (ntiles <= 0 || !a || !b || !c) return -1;
  if (((uintptr_t)a | (uintptr_t)b) & 15) return -2;
  hipLaunchKernelGGL(mfma_tiles, dim3(ntiles), dim3(64), 0, (hipStream_t)stream, a, b, c, ntiles);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
