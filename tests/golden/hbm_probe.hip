// hbm_probe.hip -- test-only library: the rates HBM delivers on gfx950 to the access forms the
// attention kernels use, over a buffer far larger than the caches (4 MB of L2 per XCD, 256 MB of
// last-level cache), so that the streaming kernels' times can be set against a rate this chip
// reaches rather than only against the 8 TB/s quoted peak.
// Built by __graft_entry__.build() into tests/golden/libhbm_probe.so; run by
// tests/test_gpu_hbm_probe.py.
//
// Modes (every workgroup 256 threads, blocks_per_cu workgroups per CU):
//   0  reads: 16-byte vector loads into registers, four in flight per lane, XOR-folded into one
//      word per thread (written out so the loads are kept)
//   1  the same loads with the non-temporal hint
//   2  reads as the dQ-from-dS kernel makes them: 16-byte direct-to-LDS copies
//      (global_load_lds_dwordx4) with the non-temporal hint, one 1 KB row per wave instruction;
//      each wave keeps 8 to 16 rows in flight in a ring of 16 LDS slots of its own
//   3  writes: 16-byte vector stores
//   4  mode 2 over scattered chunks (hbm_probe_chunks): the buffer is cut into chunks of
//      chunk_kb 1 KB rows; a wave reads whole chunks, its s-th one being chunk (g * P) mod n for
//      g = wave + s * waves (P prime to n), so the chunks in flight lie far apart, as the dS tiles
//      that the dQ-from-dS kernel's workgroups read at the same time do
// Bounds: the buffer is `bytes` long, a multiple of 1024. Modes 0, 1, 3 touch 16-byte elements
// i < bytes / 16 only; modes 2 and 4 copy rows r < bytes / 1024 only (lane l reads bytes
// 16l..16l+15 of the row; mode 4: chunk c < n, row c * chunk_kb + i with i < chunk_kb) into LDS
// bytes [wave * 16 KB, wave * 16 KB + 16 KB) of a 64 KB array.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int MODE>
__global__ void __launch_bounds__(256) hbm_kernel(u32x4* __restrict__ buf, size_t n16, uint32_t* __restrict__ out) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (MODE == 3) {
    const u32x4 v = {(uint32_t)gid, 1u, 2u, 3u};
    for (size_t i = gid; i < n16; i += stride) buf[i] = v;
    return;
  }
  u32x4 acc = {0u, 0u, 0u, 0u};
  size_t i = gid;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    u32x4 a, b, c, d;
    if (MODE == 1) {
      a = __builtin_nontemporal_load(buf + i);
      b = __builtin_nontemporal_load(buf + i + stride);
      c = __builtin_nontemporal_load(buf + i + 2 * stride);
      d = __builtin_nontemporal_load(buf + i + 3 * stride);
    } else {
      a = buf[i];
      b = buf[i + stride];
      c = buf[i + 2 * stride];
      d = buf[i + 3 * stride];
    }
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += stride) acc ^= buf[i];
  out[gid] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

__device__ __forceinline__ void copy_row(const u32x4* buf, size_t row, uint32_t voff, uint32_t ring, int k) {
  const unsigned char* src = (const unsigned char*)buf + row * 1024;
  asm volatile("global_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(src), "{m0}"(ring + 1024u * (k & 15)) : "memory");
  if ((k & 7) == 7) __builtin_amdgcn_s_waitcnt((8 & 15) | (0 << 14) | (7 << 4) | (15 << 8));  // vmcnt(8)
}

// chunk_rows == 0: mode 2 (rows gw, gw + waves, ...); else mode 4 over n = nrows / chunk_rows chunks
__global__ void __launch_bounds__(256) hbm_lds_kernel(const u32x4* __restrict__ buf, size_t nrows, size_t chunk_rows,
                                                      size_t prime) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[4 * 16 * 1024];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const size_t nw = (size_t)gridDim.x * 4, gw = (size_t)blockIdx.x * 4 + wave;
  const uint32_t ring = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)lds + wave * 16 * 1024;
  const uint32_t voff = 16u * lane;
  int k = 0;
  if (chunk_rows == 0) {
    for (size_t row = gw; row < nrows; row += nw, ++k) copy_row(buf, row, voff, ring, k);
  } else {
    const size_t n = nrows / chunk_rows;
    for (size_t g = gw; g < n; g += nw) {
      const size_t c = (g * prime) % n;  // g < n < 2^32, prime < 2^21: no overflow
      for (size_t i = 0; i < chunk_rows; ++i, ++k) copy_row(buf, c * chunk_rows + i, voff, ring, k);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
}

}  // namespace

namespace {

size_t gcd(size_t a, size_t b) { return b ? gcd(b, a % b) : a; }

int run(int mode, size_t bytes, int blocks_per_cu, size_t chunk_rows, int reps, double* tbps) {
  if (mode < 0 || mode > 4 || bytes == 0 || bytes % 1024 || blocks_per_cu < 1 || blocks_per_cu > 16 ||
      (mode >= 2 && mode != 3 && blocks_per_cu > 2) || reps < 1 || reps > 1000 || !tbps)
    return -1;
  const size_t nrows = bytes / 1024;
  size_t prime = 1000003;
  if (mode == 4) {
    if (chunk_rows == 0 || chunk_rows > 64 || nrows % chunk_rows) return -1;
    while (gcd(prime, nrows / chunk_rows) != 1) prime += 2;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || cus <= 0) return -2;
  const unsigned blocks = (unsigned)(cus * blocks_per_cu);
  u32x4* buf = nullptr;
  uint32_t* out = nullptr;
  if (hipMalloc(&buf, bytes) != hipSuccess) return -2;
  if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(uint32_t)) != hipSuccess) {
    (void)hipFree(buf);
    return -2;
  }
  hipEvent_t e0 = nullptr, e1 = nullptr;
  bool ok = hipMemset(buf, 1, bytes) == hipSuccess && hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess;
  std::vector<float> ms;
  for (int r = 0; ok && r <= reps; ++r) {
    ok = hipEventRecord(e0, 0) == hipSuccess;
    if (mode == 0) hipLaunchKernelGGL(hbm_kernel<0>, dim3(blocks), dim3(256), 0, 0, buf, bytes / 16, out);
    if (mode == 1) hipLaunchKernelGGL(hbm_kernel<1>, dim3(blocks), dim3(256), 0, 0, buf, bytes / 16, out);
    if (mode == 2) hipLaunchKernelGGL(hbm_lds_kernel, dim3(blocks), dim3(256), 0, 0, buf, nrows, (size_t)0, prime);
    if (mode == 4) hipLaunchKernelGGL(hbm_lds_kernel, dim3(blocks), dim3(256), 0, 0, buf, nrows, chunk_rows, prime);
    if (mode == 3) hipLaunchKernelGGL(hbm_kernel<3>, dim3(blocks), dim3(256), 0, 0, buf, bytes / 16, out);
    ok = ok && hipGetLastError() == hipSuccess && hipEventRecord(e1, 0) == hipSuccess && hipEventSynchronize(e1) == hipSuccess;
    float t = 0.0f;
    ok = ok && hipEventElapsedTime(&t, e0, e1) == hipSuccess;
    if (ok && r > 0) ms.push_back(t);
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  (void)hipFree(out);
  (void)hipFree(buf);
  if (!ok || ms.empty()) return -2;
  std::sort(ms.begin(), ms.end());
  *tbps = (double)bytes / (ms[ms.size() / 2] * 1e-3) / 1e12;
  return 0;
}

}  // namespace

// Median rate in TB/s (1e12 bytes per second) of `reps` timed launches after one untimed one, of
// modes 0-3. Returns 0, or -1 for bad arguments, -2 for a HIP error.
extern "C" int hbm_probe_run(int mode, size_t bytes, int blocks_per_cu, int reps, double* tbps) {
  if (mode == 4) return -1;
  return run(mode, bytes, blocks_per_cu, 0, reps, tbps);
}

// The same for mode 4, chunks of chunk_kb KB (1-64; bytes a multiple of chunk_kb KB).
extern "C" int hbm_probe_chunks(size_t bytes, int blocks_per_cu, int chunk_kb, int reps, double* tbps) {
  if (chunk_kb < 1) return -1;
  return run(4, bytes, blocks_per_cu, (size_t)chunk_kb, reps, tbps);
}
