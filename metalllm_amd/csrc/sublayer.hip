// sublayer.hip -- the GEMMs of metalLLM's attention sublayer around the attention core, as extern "C"
// entry points with the reference kernels' names and buffer order (declared in
// include/metalllm_attn.h):
//   computeQKV      attention.metal:19-53   Q,K,V = X.Wq, X.Wk, X.Wv                       (bf16)
//   projForward     attention.metal:385-405 out = O.Wp                                    (bf16)
//   projBackwarddW  attention.metal:407-430 dWp += O^T.dZ                       (bf16, accumulated)
//   projBackwarddX  attention.metal:432-455 dO = dZ.Wp^T                                   (bf16)
//   computeGradDx   attention.metal:301-341 dX += dQ.Wq^T + dK.Wk^T + dV.Wv^T   (fp32, accumulated)
//   computeGradDw   attention.metal:343-383 dWq += X^T.dQ (fp32), dWk += X^T.dK, dWv += X^T.dV (bf16)
// Row-major matrices: X, O, dZ, Q, K, V, dK, dV bf16 [R, C] and dQ, dX fp32 [R, C] with R = B*M rows
// and C = N = NH*D features; weights bf16 [C, C] indexed [input feature][output feature].
//
// The bf16 GEMMs run on the platform library: rocBLAS gemm_ex with bf16 operands, fp32
// accumulation and a bf16 or fp32 destination (beta = 1 for the reference's multiply_accumulate
// kernels: the destination is read once and the sum rounded once). computeGradDx and computeGradDw
// read the fp32 dQ, which the library cannot take as is: for row and feature counts that are
// multiples of 128 they run hand-written matrix-core kernels (sublayer_gemm.hip) that load dQ as
// fp32 and split it in registers into two bf16 terms, dQ = hi + lo + O(2^-16 |dQ|), each product
// running on both; for other shapes a HIP kernel writes the same split to memory (split_dq) and
// the library runs each product twice. Either way the fp32 dQ never makes a bf16 round trip.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/metalllm_attn.h"

namespace mla {  // attn_fwd.hip
void forward_prepare();
}  // namespace mla

namespace mla {  // sublayer_gemm.hip
bool grad_dx_fused_ok(int R, int C);
hipError_t launch_grad_dx(float* dX, const float* dQ, const uint16_t* dK, const uint16_t* dV, const uint16_t* Wq,
                          const uint16_t* Wk, const uint16_t* Wv, int R, int C, bool accumulate, hipStream_t s);
bool grad_dw_fused_ok(int R, int C);
size_t grad_dw_partial_floats(int R, int C);
hipError_t launch_grad_dw(const uint16_t* X, const float* dQ, const uint16_t* dK, const uint16_t* dV, float* dQw,
                          uint16_t* dKw, uint16_t* dVw, float* partial, int R, int C, bool accumulate, hipStream_t s);
size_t grad_dw_one_partial_floats(int R, int C);
hipError_t launch_grad_dw_one(const uint16_t* X, const uint16_t* G, uint16_t* dW, float* partial, int R, int C,
                              bool accumulate, hipStream_t s);
size_t grad_dw4_partial_floats(int R, int C);
hipError_t launch_grad_dxdw4(float* dX, const uint16_t* X, const float* dQ, const uint16_t* dK, const uint16_t* dV,
                             const uint16_t* Wq, const uint16_t* Wk, const uint16_t* Wv, const uint16_t* Xp,
                             const uint16_t* Gp, float* dQw, uint16_t* dKw, uint16_t* dVw, uint16_t* dPw, float* partial,
                             int R, int C, hipStream_t s);
}  // namespace mla

namespace {

int validate_gemm(const AttentionParams* p) {
  if (!p) return METALLLM_ATTN_E_NULL;
  if (p->M == 0) return METALLLM_ATTN_E_SEQLEN;
  if (p->NH == 0 || p->B == 0 || p->D == 0 || (uint64_t)p->N != (uint64_t)p->NH * p->D || p->N % 8)
    return METALLLM_ATTN_E_LAYOUT;  // rows of 16-byte multiples
  if ((uint64_t)p->B * p->M * p->N >= (1ull << 31) || (uint64_t)p->N * p->N >= (1ull << 31)) return METALLLM_ATTN_E_SIZE;
  return METALLLM_ATTN_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

// Per-device library state: the rocBLAS handle (created on first use with that device current),
// the bf16 split of dQ and the fp32 partials of the weight gradients (grown on demand). A mutex
// per device serialises the host side of a call (stream binding and enqueue); the buffers are
// shared, so computeGradDx, computeGradDw and projBackwarddW calls on different streams of one
// device must not overlap.
struct DeviceState {
  std::mutex mu;
  rocblas_handle handle = nullptr;
  uint16_t* split = nullptr;  // hi [R*C] then lo [R*C]
  size_t split_elems = 0;
  float* partial = nullptr;   // fp32 partial products of the weight gradients [parts][C][C]
  size_t partial_elems = 0;
  uint8_t* attn_ws = nullptr;  // the attention backward's dS tiles (metalllmSublayerEncode)
  size_t attn_ws_bytes = 0;
};

// Grows a per-device buffer (never shrinks). Growing synchronises the device (the old buffer may
// still be in use by work enqueued on any stream) and allocates, so it is refused while `stream`
// is being captured into a graph: metalllmSublayerReserve sizes the buffers ahead of time.
template <typename T>
int ensure(T*& buf, size_t& have, size_t need, hipStream_t stream) {
  if (have >= need) return METALLLM_ATTN_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return METALLLM_ATTN_E_LIBRARY;
  if (cap != hipStreamCaptureStatusNone) return METALLLM_ATTN_E_CAPTURE;
  if (buf) {
    if (hipDeviceSynchronize() != hipSuccess || hipFree(buf) != hipSuccess) return METALLLM_ATTN_E_LIBRARY;
    buf = nullptr;
    have = 0;
  }
  if (hipMalloc((void**)&buf, need * sizeof(T)) != hipSuccess) {
    buf = nullptr;
    return METALLLM_ATTN_E_LIBRARY;
  }
  have = need;
  return METALLLM_ATTN_OK;
}

DeviceState& state(int dev) {
  static std::mutex table_mu;
  static std::vector<DeviceState*> table;
  std::lock_guard<std::mutex> g(table_mu);
  if ((int)table.size() <= dev) table.resize(dev + 1, nullptr);
  if (!table[dev]) table[dev] = new DeviceState();  // lives until the process ends
  return *table[dev];
}

// Locks the current device's state and binds its handle to `stream`; null handle on failure.
struct Session {
  std::unique_lock<std::mutex> lock;
  DeviceState* st = nullptr;
  int rc = METALLLM_ATTN_OK;

  explicit Session(hipStream_t stream) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
      rc = METALLLM_ATTN_E_LIBRARY;
      return;
    }
    st = &state(dev);
    lock = std::unique_lock<std::mutex>(st->mu);
    if (!st->handle && rocblas_create_handle(&st->handle) != rocblas_status_success) {
      st->handle = nullptr;
      rc = METALLLM_ATTN_E_LIBRARY;
      return;
    }
    if (rocblas_set_stream(st->handle, stream) != rocblas_status_success) rc = METALLLM_ATTN_E_LIBRARY;
  }
};

// Where a sequence of GEMMs and helper kernels goes: the rocBLAS handle (already bound to
// `stream`) and the stream. With `query` set, nothing is launched: rocBLAS calls only report the
// device workspace they need (rocblas_start_device_memory_size_query is active on the handle).
struct Ctx {
  rocblas_handle h = nullptr;
  hipStream_t stream = nullptr;
  bool query = false;
};

bool blas_ok(const Ctx& c, rocblas_status s) {
  return s == rocblas_status_success ||
         (c.query && (s == rocblas_status_size_increased || s == rocblas_status_size_unchanged));
}

// Row-major C[M][N] = op(A)[M][K] . op(B)[K][N] + beta * C. op(A) = A stored [M][K] (lda) or, with
// ta, A^T of A stored [K][M]; likewise op(B). rocBLAS is column-major: the row-major product is
// computed as C^T = op(B)^T . op(A)^T on the same memory.
int gemm_rm(const Ctx& c, bool ta, bool tb, int M, int N, int K, const void* A, rocblas_datatype at, int lda,
            const void* B, rocblas_datatype bt, int ldb, float beta, void* C, rocblas_datatype ct, int ldc) {
  const float alpha = 1.0f;
  const rocblas_status s = rocblas_gemm_ex(
      c.h, tb ? rocblas_operation_transpose : rocblas_operation_none, ta ? rocblas_operation_transpose : rocblas_operation_none,
      N, M, K, &alpha, B, bt, ldb, A, at, lda, &beta, C, ct, ldc, C, ct, ldc, rocblas_datatype_f32_r,
      rocblas_gemm_algo_standard, 0, 0);
  return blas_ok(c, s) ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LIBRARY;
}

constexpr rocblas_datatype BF = rocblas_datatype_bf16_r;
constexpr rocblas_datatype F32 = rocblas_datatype_f32_r;

__device__ __forceinline__ uint16_t rne_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);  // finite inputs
}

// hi = bf16(x), lo = bf16(x - hi): four elements per thread (16-byte loads).
__global__ void __launch_bounds__(256) split_kernel(const float4* __restrict__ x, uint2* __restrict__ hi,
                                                    uint2* __restrict__ lo, size_t n4) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += (size_t)gridDim.x * blockDim.x) {
    const float4 v = x[i];
    const float f[4] = {v.x, v.y, v.z, v.w};
    uint16_t h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h[j] = rne_bf16(f[j]);
      l[j] = rne_bf16(f[j] - __uint_as_float((uint32_t)h[j] << 16));
    }
    hi[i] = uint2{(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
    lo[i] = uint2{(uint32_t)l[0] | ((uint32_t)l[1] << 16), (uint32_t)l[2] | ((uint32_t)l[3] << 16)};
  }
}

// Writes hi = bf16(dQ), lo = bf16(dQ - hi) into split[0 .. elems) and split[elems .. 2 elems).
int split_dq(const Ctx& c, const float* dQ, size_t elems, uint16_t* split) {
  if (c.query) return METALLLM_ATTN_OK;
  const size_t n4 = elems / 4;  // C is a multiple of 8 (validate_gemm)
  const unsigned blocks = (unsigned)std::min<size_t>((n4 + 255) / 256, 65536);
  hipLaunchKernelGGL(split_kernel, dim3(blocks), dim3(256), 0, c.stream, (const float4*)dQ, (uint2*)split,
                     (uint2*)(split + elems), n4);
  return hipGetLastError() == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

// Weight gradients W[k][n] += sum_r X[r][k] G[r][n] reduce over all R rows into a small C x C
// output: one GEMM gives the library too few output tiles for the chip. The rows are split into
// `parts` chunks, computed as one strided-batched GEMM into fp32 partials [chunk][C][C], and
// reduce_kernel adds the partials (of one or more such products) and the destination's previous
// value once, then rounds to the destination type.
int row_chunks(int R) {
  for (int s : {16, 8, 4, 2})
    if (R % s == 0 && R / s >= 512) return s;
  return 1;
}

// Elements of the dQ split (hi, then lo) that the library paths of computeGradDx and
// computeGradDw read: none when the hand-written kernels take the shape (they split in registers).
size_t split_need(int R, int C) {
  return mla::grad_dx_fused_ok(R, C) && mla::grad_dw_fused_ok(R, C) ? 0 : 2 * (size_t)R * C;
}

// fp32 partial floats for projBackwarddW and computeGradDw: the hand-written kernel's chunks, or
// row_chunks(R) products of C x C (twice that for computeGradDw's dQw) on the library path.
size_t partial_need(int R, int C) {
  if (mla::grad_dw_fused_ok(R, C))
    return std::max({mla::grad_dw_one_partial_floats(R, C), mla::grad_dw_partial_floats(R, C),
                     mla::grad_dw4_partial_floats(R, C)});
  return 2 * (size_t)row_chunks(R) * C * C;
}

int xt_g_partials(const Ctx& c, const uint16_t* X, const uint16_t* G, int R, int C, int parts, float* out) {
  const float alpha = 1.0f, beta = 0.0f;
  const int Rs = R / parts;
  // row-major out_s[C][C] = X_s^T . G_s; column-major: out_s^T = G_s^T . X_s
  const rocblas_status st = rocblas_gemm_strided_batched_ex(
      c.h, rocblas_operation_none, rocblas_operation_transpose, C, C, Rs, &alpha, G, BF, C, (rocblas_stride)Rs * C, X,
      BF, C, (rocblas_stride)Rs * C, &beta, out, F32, C, (rocblas_stride)C * C, out, F32, C, (rocblas_stride)C * C,
      parts, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  return blas_ok(c, st) ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LIBRARY;
}

// dst[i] = round(dst[i] + sum_p part[p * n + i]) with the fp32 sum in p order; dst fp32 or bf16.
// Without acc_dst the destination is written as if it held zeros (bit for bit 0 + sum), unread.
template <bool BF16_DST>
__global__ void __launch_bounds__(256) reduce_kernel(const float* __restrict__ part, int nparts, size_t n, void* dst,
                                                     bool acc_dst) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    float acc = 0.0f;
    for (int p = 0; p < nparts; ++p) acc += part[(size_t)p * n + i];
    if (BF16_DST) {
      uint16_t* d = (uint16_t*)dst;
      d[i] = rne_bf16((acc_dst ? __uint_as_float((uint32_t)d[i] << 16) : 0.0f) + acc);
    } else {
      float* d = (float*)dst;
      d[i] = (acc_dst ? d[i] : 0.0f) + acc;
    }
  }
}

int reduce_into(const Ctx& c, const float* part, int nparts, size_t n, void* dst, bool bf16_dst, bool accumulate = true) {
  if (c.query) return METALLLM_ATTN_OK;
  const unsigned blocks = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  if (bf16_dst)
    hipLaunchKernelGGL(reduce_kernel<true>, dim3(blocks), dim3(256), 0, c.stream, part, nparts, n, dst, accumulate);
  else
    hipLaunchKernelGGL(reduce_kernel<false>, dim3(blocks), dim3(256), 0, c.stream, part, nparts, n, dst, accumulate);
  return hipGetLastError() == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

#define TRY(x)                  \
  do {                          \
    const int rc_ = (x);        \
    if (rc_) return rc_;        \
  } while (0)

#define CHECK_PTRS(...)                                           \
  do {                                                            \
    const void* ps_[] = {__VA_ARGS__};                            \
    for (const void* q_ : ps_) {                                  \
      if (!q_) return METALLLM_ATTN_E_NULL;                       \
      if (!aligned16(q_)) return METALLLM_ATTN_E_ALIGN;           \
    }                                                             \
  } while (0)

// ---- the reference kernels as sequences on a Ctx (R = B*M rows, C = N features) ----

// When q_w, k_w, v_w are equally spaced in memory (a fused [3][C][C] weight, or one weight used
// three times) and q, k, v are equally spaced without overlapping, the three products run as one
// strided-batched library call: 768 workgroups in flight at config 4 instead of three launches of
// 256, 66 against 75 us measured. Otherwise three calls.
int op_qkv(const Ctx& c, const uint16_t* X, uint16_t* q, uint16_t* k, uint16_t* v, const uint16_t* q_w,
           const uint16_t* k_w, const uint16_t* v_w, int R, int C) {
  // distances in bf16 elements, from the integer addresses (the buffers may be separate allocations)
  const auto at = [](const uint16_t* ptr) { return (intptr_t)(uintptr_t)ptr; };
  const intptr_t bw = at(k_w) - at(q_w), by = at(k) - at(q);
  const intptr_t dw = bw / 2, dy = by / 2;
  if (bw % 2 == 0 && by % 2 == 0 && dw >= 0 && at(v_w) - at(k_w) == bw && dy >= (intptr_t)R * C &&
      at(v) - at(k) == by) {
    const float alpha = 1.0f, beta = 0.0f;
    // row-major Y_i = X . W_i; column-major Y_i^T = W_i^T . X^T
    const rocblas_status st = rocblas_gemm_strided_batched_ex(
        c.h, rocblas_operation_none, rocblas_operation_none, C, R, C, &alpha, q_w, BF, C, (rocblas_stride)dw, X, BF, C, 0,
        &beta, q, BF, C, (rocblas_stride)dy, q, BF, C, (rocblas_stride)dy, 3, rocblas_datatype_f32_r,
        rocblas_gemm_algo_standard, 0, 0);
    return blas_ok(c, st) ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LIBRARY;
  }
  TRY(gemm_rm(c, false, false, R, C, C, X, BF, C, q_w, BF, C, 0.0f, q, BF, C));
  TRY(gemm_rm(c, false, false, R, C, C, X, BF, C, k_w, BF, C, 0.0f, k, BF, C));
  return gemm_rm(c, false, false, R, C, C, X, BF, C, v_w, BF, C, 0.0f, v, BF, C);
}

int op_proj_fwd(const Ctx& c, const uint16_t* attn_out, const uint16_t* proj_w, uint16_t* out, int R, int C) {
  return gemm_rm(c, false, false, R, C, C, attn_out, BF, C, proj_w, BF, C, 0.0f, out, BF, C);
}

// partial: at least partial_need(R, C) floats. accumulate = false: dProjw is written as if it
// held zeros (the phase encoder; every op_* below takes the same flag). Row counts that are
// multiples of 128 and feature counts that are multiples of 128 run computeGradDw's hand-written
// kernel (sublayer_gemm.hip) on the one bf16 gradient; other shapes use the library.
int op_proj_dw(const Ctx& c, const uint16_t* attn_out, const uint16_t* dZ, uint16_t* dProjw, int R, int C,
               float* partial, bool accumulate = true) {
  if (mla::grad_dw_fused_ok(R, C)) {
    if (c.query) return METALLLM_ATTN_OK;
    return mla::launch_grad_dw_one(attn_out, dZ, dProjw, partial, R, C, accumulate, c.stream) == hipSuccess
               ? METALLLM_ATTN_OK
               : METALLLM_ATTN_E_LAUNCH;
  }
  const int parts = row_chunks(R);
  TRY(xt_g_partials(c, attn_out, dZ, R, C, parts, partial));
  return reduce_into(c, partial, parts, (size_t)C * C, dProjw, true, accumulate);
}

int op_proj_dx(const Ctx& c, const uint16_t* dZ, const uint16_t* proj_w, uint16_t* dAttn, int R, int C) {
  return gemm_rm(c, false, true, R, C, C, dZ, BF, C, proj_w, BF, C, 0.0f, dAttn, BF, C);
}

// Row and feature counts that are multiples of 128 run the hand-written kernel (sublayer_gemm.hip),
// which reads the fp32 dQ itself; other shapes use the library on hi, lo, the two-term bf16 split
// of dQ (split_dq).
int op_grad_dx(const Ctx& c, float* dX, const uint16_t* qw, const uint16_t* kw, const uint16_t* vw, const float* dQ,
               const uint16_t* hi, const uint16_t* lo, const uint16_t* dK, const uint16_t* dV, int R, int C,
               bool accumulate = true) {
  if (mla::grad_dx_fused_ok(R, C)) {
    if (c.query) return METALLLM_ATTN_OK;
    return mla::launch_grad_dx(dX, dQ, dK, dV, qw, kw, vw, R, C, accumulate, c.stream) == hipSuccess
               ? METALLLM_ATTN_OK
               : METALLLM_ATTN_E_LAUNCH;
  }
  TRY(gemm_rm(c, false, true, R, C, C, hi, BF, C, qw, BF, C, accumulate ? 1.0f : 0.0f, dX, F32, C));
  TRY(gemm_rm(c, false, true, R, C, C, lo, BF, C, qw, BF, C, 1.0f, dX, F32, C));
  TRY(gemm_rm(c, false, true, R, C, C, dK, BF, C, kw, BF, C, 1.0f, dX, F32, C));
  return gemm_rm(c, false, true, R, C, C, dV, BF, C, vw, BF, C, 1.0f, dX, F32, C);
}

// partial: at least partial_need(R, C) floats. Row counts that are multiples of 128 and feature
// counts that are multiples of 128 run the hand-written kernel (sublayer_gemm.hip) on the fp32 dQ;
// other shapes use the library on hi, lo, the two-term bf16 split of dQ (split_dq).
int op_grad_dw(const Ctx& c, const uint16_t* x, const float* dQ, const uint16_t* hi, const uint16_t* lo,
               const uint16_t* dK, const uint16_t* dV, float* dQw, uint16_t* dKw, uint16_t* dVw, int R, int C,
               float* part, bool accumulate = true) {
  if (mla::grad_dw_fused_ok(R, C)) {
    if (c.query) return METALLLM_ATTN_OK;
    return mla::launch_grad_dw(x, dQ, dK, dV, dQw, dKw, dVw, part, R, C, accumulate, c.stream) == hipSuccess
               ? METALLLM_ATTN_OK
               : METALLLM_ATTN_E_LAUNCH;
  }
  const int parts = row_chunks(R);
  const size_t cc = (size_t)C * C;
  // dQw: the partials of X^T.hi and X^T.lo together, added into dQw once
  TRY(xt_g_partials(c, x, hi, R, C, parts, part));
  TRY(xt_g_partials(c, x, lo, R, C, parts, part + parts * cc));
  TRY(reduce_into(c, part, 2 * parts, cc, dQw, false, accumulate));
  TRY(xt_g_partials(c, x, dK, R, C, parts, part));
  TRY(reduce_into(c, part, parts, cc, dKw, true, accumulate));
  TRY(xt_g_partials(c, x, dV, R, C, parts, part));
  return reduce_into(c, part, parts, cc, dVw, true, accumulate);
}

// Zeroes up to 8 buffers in one launch (a fill kernel: no memset node when captured into a
// graph). Each segment is n16 16-byte words; grid-stride over each segment in turn.
struct ZeroSet {
  uint4* p[8];
  size_t n16[8];
  int n;
};

__global__ void __launch_bounds__(256) zero_kernel(ZeroSet z) {
  const size_t stride = (size_t)gridDim.x * blockDim.x, i0 = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  for (int k = 0; k < z.n; ++k)
    for (size_t i = i0; i < z.n16[k]; i += stride) z.p[k][i] = uint4{0u, 0u, 0u, 0u};
}

// (pointer, bytes) pairs, bytes a multiple of 16
int zero_buffers(const Ctx& c, std::initializer_list<std::pair<void*, size_t>> bufs) {
  if (c.query) return METALLLM_ATTN_OK;
  ZeroSet z{};
  size_t largest = 0;
  for (const auto& b : bufs) {
    if (z.n == 8) return METALLLM_ATTN_E_LAUNCH;
    z.p[z.n] = (uint4*)b.first;
    z.n16[z.n] = b.second / 16;
    largest = std::max(largest, z.n16[z.n]);
    ++z.n;
  }
  const unsigned blocks = (unsigned)std::max<size_t>(1, std::min<size_t>((largest + 255) / 256, 8192));
  hipLaunchKernelGGL(zero_kernel, dim3(blocks), dim3(256), 0, c.stream, z);
  return hipGetLastError() == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

// Public entry points: the device's handle and buffers, bound to the caller's stream.
struct Public {
  Session s;
  Ctx c;
  explicit Public(metalllm_stream_t stream) : s((hipStream_t)stream) {
    c.h = s.st ? s.st->handle : nullptr;
    c.stream = (hipStream_t)stream;
  }
};

}  // namespace

extern "C" {

int computeQKV(const uint16_t* X, uint16_t* q, uint16_t* k, uint16_t* v, const uint16_t* q_w, const uint16_t* k_w,
               const uint16_t* v_w, const AttentionParams* p, metalllm_stream_t stream) {
  TRY(validate_gemm(p));
  CHECK_PTRS(X, q, k, v, q_w, k_w, v_w);
  Public u(stream);
  TRY(u.s.rc);
  return op_qkv(u.c, X, q, k, v, q_w, k_w, v_w, (int)(p->B * p->M), (int)p->N);
}

int projForward(const uint16_t* attn_out, const uint16_t* proj_w, uint16_t* out, const AttentionParams* p,
                metalllm_stream_t stream) {
  TRY(validate_gemm(p));
  CHECK_PTRS(attn_out, proj_w, out);
  Public u(stream);
  TRY(u.s.rc);
  return op_proj_fwd(u.c, attn_out, proj_w, out, (int)(p->B * p->M), (int)p->N);
}

int projBackwarddW(const uint16_t* attn_out, const uint16_t* dZ, uint16_t* dProjw, const AttentionParams* p,
                   metalllm_stream_t stream) {
  TRY(validate_gemm(p));
  CHECK_PTRS(attn_out, dZ, dProjw);
  const int R = (int)(p->B * p->M), C = (int)p->N;
  Public u(stream);
  TRY(u.s.rc);
  TRY(ensure(u.s.st->partial, u.s.st->partial_elems, partial_need(R, C), u.c.stream));
  return op_proj_dw(u.c, attn_out, dZ, dProjw, R, C, u.s.st->partial);
}

int projBackwarddX(const uint16_t* dZ, const uint16_t* proj_w, uint16_t* dAttn, const AttentionParams* p,
                   metalllm_stream_t stream) {
  TRY(validate_gemm(p));
  CHECK_PTRS(dZ, proj_w, dAttn);
  Public u(stream);
  TRY(u.s.rc);
  return op_proj_dx(u.c, dZ, proj_w, dAttn, (int)(p->B * p->M), (int)p->N);
}

int computeGradDx(float* dX, const uint16_t* qw, const uint16_t* kw, const uint16_t* vw, const float* dQ,
                  const uint16_t* dK, const uint16_t* dV, const AttentionParams* p, metalllm_stream_t stream) {
  TRY(validate_gemm(p));
  CHECK_PTRS(dX, qw, kw, vw, dQ, dK, dV);
  const int R = (int)(p->B * p->M), C = (int)p->N;
  const size_t e = (size_t)R * C;
  Public u(stream);
  TRY(u.s.rc);
  if (mla::grad_dx_fused_ok(R, C)) return op_grad_dx(u.c, dX, qw, kw, vw, dQ, nullptr, nullptr, dK, dV, R, C);
  TRY(ensure(u.s.st->split, u.s.st->split_elems, 2 * e, u.c.stream));
  TRY(split_dq(u.c, dQ, e, u.s.st->split));
  return op_grad_dx(u.c, dX, qw, kw, vw, dQ, u.s.st->split, u.s.st->split + e, dK, dV, R, C);
}

int computeGradDw(const uint16_t* x, const float* dQ, const uint16_t* dK, const uint16_t* dV, float* dQw,
                  uint16_t* dKw, uint16_t* dVw, const AttentionParams* p, metalllm_stream_t stream) {
  TRY(validate_gemm(p));
  CHECK_PTRS(x, dQ, dK, dV, dQw, dKw, dVw);
  const int R = (int)(p->B * p->M), C = (int)p->N;
  const size_t e = (size_t)R * C;
  Public u(stream);
  TRY(u.s.rc);
  TRY(ensure(u.s.st->partial, u.s.st->partial_elems, partial_need(R, C), u.c.stream));
  if (mla::grad_dw_fused_ok(R, C))
    return op_grad_dw(u.c, x, dQ, nullptr, nullptr, dK, dV, dQw, dKw, dVw, R, C, u.s.st->partial);
  TRY(ensure(u.s.st->split, u.s.st->split_elems, 2 * e, u.c.stream));
  TRY(split_dq(u.c, dQ, e, u.s.st->split));
  return op_grad_dw(u.c, x, dQ, u.s.st->split, u.s.st->split + e, dK, dV, dQw, dKw, dVw, R, C, u.s.st->partial);
}

}  // extern "C"

// ---- Phase encoder ----
// model.h encodes each phase of a training step into one command buffer (forward :441-508,
// backward :587-708) and commits it once (commitWait, :358-366); the buffers are allocated once
// in the constructor (:236-277), so the same dispatches run on the same buffers every step. The
// MI355X form is a HIP graph per phase of the attention sublayer: the launches are recorded once
// on a private stream with the pointers and shapes baked in, and replayed with one launch. Each
// graph owns its rocBLAS handle, that handle's workspace (sized by a rocBLAS size query before
// capture) and its scratch (dQ split, weight-gradient partials, the attention backward's dS
// tiles), so nothing a replay touches is ever reallocated by other calls.
struct metalllmSublayerGraph {
  int phase = 0;
  rocblas_handle h = nullptr;
  void* workspace = nullptr;
  uint16_t* split = nullptr;
  float* partial = nullptr;
  void* attn_ws = nullptr;
  uint64_t attn_ws_bytes = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace {

int check_phase(int phase, const metalllmSublayerBuffers* b, const AttentionParams* p) {
  if (!b || !p) return METALLLM_ATTN_E_NULL;
  if (phase != 0 && phase != 1) return METALLLM_ATTN_E_LAYOUT;
  TRY(validate_gemm(p));
  if (p->M % 64) return METALLLM_ATTN_E_SEQLEN;
  if (p->D != 64 && p->D != 128) return METALLLM_ATTN_E_HEADDIM;
  if (phase == 0) {
    CHECK_PTRS(b->X, b->q_w, b->k_w, b->v_w, b->proj_w, b->q, b->k, b->v, b->attn_out, b->l, b->out);
  } else {
    CHECK_PTRS(b->X, b->q_w, b->k_w, b->v_w, b->proj_w, b->q, b->k, b->v, b->attn_out, b->l, b->dOut, b->dAttn,
               b->Dsum, b->dQ, b->dK, b->dV, b->dX, b->dQw, b->dKw, b->dVw, b->dProjw);
    if (b->dX_bf16 && !aligned16(b->dX_bf16)) return METALLLM_ATTN_E_ALIGN;
  }
  if (b->hidden) {  // the block's attention half
    CHECK_PTRS(b->hidden, b->ln_gamma, b->ln_beta, b->ln_xnorm, b->ln_stdev, b->ln_dgamma, b->ln_dbeta, b->residual,
               b->dStream);
    if (p->N > 4096 || !(b->ln_eps >= 0.0f)) return METALLLM_ATTN_E_LAYOUT;
  }
  return METALLLM_ATTN_OK;
}

// The launch sequence of one phase (model.h:444-483 forward, :549-555 and :620-693 backward).
int encode(const Ctx& c, int phase, const metalllmSublayerBuffers* b, const AttentionParams* p, uint16_t* split,
           float* partial, void* attn_ws, uint64_t attn_ws_bytes) {
  const int R = (int)(p->B * p->M), C = (int)p->N;
  const size_t e = (size_t)R * C;
  const metalllm_stream_t s = (metalllm_stream_t)c.stream;
  const bool block = b->hidden != nullptr;
  const LayernormParams lp{(uint32_t)R, (uint32_t)C, (uint32_t)std::min(C, 1024), b->ln_eps};
  if (phase == 0) {
    if (block && !c.query)  // model.h:445: X = ln1(hidden)
      TRY(layernormForward(b->hidden, b->ln_xnorm, (uint16_t*)b->X, b->ln_gamma, b->ln_beta, b->ln_stdev, &lp, s));
    TRY(op_qkv(c, b->X, b->q, b->k, b->v, b->q_w, b->k_w, b->v_w, R, C));
    if (!c.query) TRY(flashAttentionForward(b->q, b->k, b->v, b->attn_out, b->l, p, s));
    TRY(op_proj_fwd(c, b->attn_out, b->proj_w, b->out, R, C));
    if (block && !c.query) TRY(residualAdd(b->hidden, b->out, b->residual, (uint32_t)e, s));  // model.h:483
    return METALLLM_ATTN_OK;
  }
  // model.h:549-555 zeroes the accumulated gradients before the pass and the kernels add into
  // them. Each of dX, dQw, dKw, dVw and dProjw has a single producer in this phase, so the phase
  // runs them in write mode instead: the result is bit for bit 0 + the gradient (-0 becomes +0),
  // without the zeroing pass and without reading the destinations. The attention backward writes
  // dQ, dK and dV in full; the block's layernorm gradients (model.h:545-546), which its backward
  // adds into with atomics, are zeroed here.
  if (block) TRY(zero_buffers(c, {{b->ln_dgamma, (size_t)C * 4}, {b->ln_dbeta, (size_t)C * 4}}));
  // With the hand-written weight-gradient kernel, dProjw (which nothing in this phase reads) is
  // computed at the end, as a fourth weight of computeGradDw's launch and reduction: one launch of
  // balanced items instead of projBackwarddW's own short-item launch. Its sum then runs over
  // other row chunks than the entry point's, so it can differ from projBackwarddW's result by the
  // fp32 summation order (one bf16 rounding step at most).
  const bool fuse_pdw = mla::grad_dw_fused_ok(R, C) && mla::grad_dx_fused_ok(R, C);
  if (!fuse_pdw) TRY(op_proj_dw(c, b->attn_out, b->dOut, b->dProjw, R, C, partial, false));
  TRY(op_proj_dx(c, b->dOut, b->proj_w, b->dAttn, R, C));
  if (!c.query) {
    TRY(computeD(b->dAttn, b->attn_out, b->Dsum, p, s));
    TRY(flashAttentionBackwardWorkspace(b->dAttn, b->Dsum, b->l, b->q, b->k, b->v, b->dQ, b->dK, b->dV, attn_ws,
                                        attn_ws_bytes, p, s));
  }
  uint16_t* lo = nullptr;  // no split when both hand-written kernels take the shape
  if (split_need(R, C)) {
    TRY(split_dq(c, b->dQ, e, split));  // one split serves both consumers
    lo = split + e;
  } else {
    split = nullptr;
  }
  if (fuse_pdw) {
    // computeGradDx and the four weight gradients in one launch (dX tiles first, then the
    // weight-gradient items, which start as the dX tiles finish), then the reduction
    if (!c.query && mla::launch_grad_dxdw4(b->dX, b->X, b->dQ, b->dK, b->dV, b->q_w, b->k_w, b->v_w, b->attn_out,
                                           b->dOut, b->dQw, b->dKw, b->dVw, b->dProjw, partial, R, C,
                                           c.stream) != hipSuccess)
      return METALLLM_ATTN_E_LAUNCH;
  } else {
    TRY(op_grad_dx(c, b->dX, b->q_w, b->k_w, b->v_w, b->dQ, split, lo, b->dK, b->dV, R, C, false));
    TRY(op_grad_dw(c, b->X, b->dQ, split, lo, b->dK, b->dV, b->dQw, b->dKw, b->dVw, R, C, partial, false));
  }
  if (c.query) return METALLLM_ATTN_OK;
  if (block) {  // model.h:692-695
    TRY(castFloatToBfloat(b->dX, b->dStream, (uint32_t)e, s));
    TRY(layernormBackward(b->dStream, b->ln_xnorm, b->ln_gamma, b->ln_stdev, nullptr, b->ln_dgamma, b->ln_dbeta, &lp,
                          s));
    return residualAdd(b->dStream, b->dOut, b->dStream, (uint32_t)e, s);
  }
  if (b->dX_bf16) TRY(castFloatToBfloat(b->dX, b->dX_bf16, (uint32_t)e, s));
  return METALLLM_ATTN_OK;
}

int build_graph(metalllmSublayerGraph* g, const metalllmSublayerBuffers* b, const AttentionParams* p) {
  const int R = (int)(p->B * p->M), C = (int)p->N;
  if (rocblas_create_handle(&g->h) != rocblas_status_success) {
    g->h = nullptr;
    return METALLLM_ATTN_E_LIBRARY;
  }
  if (g->phase == 1) {
    const size_t split = split_need(R, C);
    if (split && hipMalloc((void**)&g->split, split * sizeof(uint16_t)) != hipSuccess) g->split = nullptr;
    if (hipMalloc((void**)&g->partial, partial_need(R, C) * sizeof(float)) != hipSuccess) g->partial = nullptr;
    TRY(metalllmAttnBackwardWorkspaceSize(p, &g->attn_ws_bytes));
    if (hipMalloc(&g->attn_ws, g->attn_ws_bytes) != hipSuccess) g->attn_ws = nullptr;
    if ((split && !g->split) || !g->partial || !g->attn_ws) return METALLLM_ATTN_E_LIBRARY;
  }
  // the workspace the phase's rocBLAS calls need, owned by the graph
  size_t ws = 0;
  if (rocblas_start_device_memory_size_query(g->h) != rocblas_status_success) return METALLLM_ATTN_E_LIBRARY;
  Ctx q;
  q.h = g->h;
  q.query = true;
  const int qrc = encode(q, g->phase, b, p, g->split, g->partial, g->attn_ws, g->attn_ws_bytes);
  if (rocblas_stop_device_memory_size_query(g->h, &ws) != rocblas_status_success || qrc) return METALLLM_ATTN_E_LIBRARY;
  if (ws && hipMalloc(&g->workspace, ws) != hipSuccess) {
    g->workspace = nullptr;
    return METALLLM_ATTN_E_LIBRARY;
  }
  if (rocblas_set_workspace(g->h, g->workspace, ws) != rocblas_status_success) return METALLLM_ATTN_E_LIBRARY;
  mla::forward_prepare();  // the forward's device queries, before the capture
  hipStream_t cap = nullptr;
  if (hipStreamCreateWithFlags(&cap, hipStreamNonBlocking) != hipSuccess) return METALLLM_ATTN_E_LIBRARY;
  int rc = rocblas_set_stream(g->h, cap) == rocblas_status_success ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LIBRARY;
  if (!rc && hipStreamBeginCapture(cap, hipStreamCaptureModeThreadLocal) != hipSuccess) rc = METALLLM_ATTN_E_LIBRARY;
  else if (!rc) {
    Ctx c;
    c.h = g->h;
    c.stream = cap;
    rc = encode(c, g->phase, b, p, g->split, g->partial, g->attn_ws, g->attn_ws_bytes);
    const hipError_t e = hipStreamEndCapture(cap, &g->graph);  // always ends the capture
    if (!rc && e != hipSuccess) rc = METALLLM_ATTN_E_LIBRARY;
  }
  if (!rc && hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0) != hipSuccess) rc = METALLLM_ATTN_E_LIBRARY;
  (void)hipStreamDestroy(cap);
  return rc;
}

}  // namespace

extern "C" {

int metalllmSublayerEncode(int phase, const metalllmSublayerBuffers* b, const AttentionParams* p,
                           metalllm_stream_t stream) {
  TRY(check_phase(phase, b, p));
  const int R = (int)(p->B * p->M), C = (int)p->N;
  Public u(stream);
  TRY(u.s.rc);
  uint64_t ws = 0;
  if (phase == 1) {
    TRY(ensure(u.s.st->split, u.s.st->split_elems, split_need(R, C), u.c.stream));
    TRY(ensure(u.s.st->partial, u.s.st->partial_elems, partial_need(R, C), u.c.stream));
    TRY(metalllmAttnBackwardWorkspaceSize(p, &ws));
    TRY(ensure(u.s.st->attn_ws, u.s.st->attn_ws_bytes, (size_t)ws, u.c.stream));
  }
  return encode(u.c, phase, b, p, u.s.st->split, u.s.st->partial, u.s.st->attn_ws, ws);
}

int metalllmSublayerReserve(const AttentionParams* p) {
  TRY(validate_gemm(p));
  if (p->D != 64 && p->D != 128) return METALLLM_ATTN_E_HEADDIM;
  if (p->M % 64) return METALLLM_ATTN_E_SEQLEN;
  const int R = (int)(p->B * p->M), C = (int)p->N;
  uint64_t ws = 0;
  TRY(metalllmAttnBackwardWorkspaceSize(p, &ws));
  Public u(nullptr);
  TRY(u.s.rc);
  TRY(ensure(u.s.st->split, u.s.st->split_elems, split_need(R, C), nullptr));
  TRY(ensure(u.s.st->partial, u.s.st->partial_elems, partial_need(R, C), nullptr));
  TRY(ensure(u.s.st->attn_ws, u.s.st->attn_ws_bytes, (size_t)ws, nullptr));
  return METALLLM_ATTN_OK;
}

int metalllmSublayerGraphCreate(int phase, const metalllmSublayerBuffers* b, const AttentionParams* p,
                                metalllmSublayerGraph** out) {
  if (!out) return METALLLM_ATTN_E_NULL;
  *out = nullptr;
  TRY(check_phase(phase, b, p));
  metalllmSublayerGraph* g = new metalllmSublayerGraph();
  g->phase = phase;
  const int rc = build_graph(g, b, p);
  if (rc) {
    metalllmSublayerGraphDestroy(g);
    return rc;
  }
  *out = g;
  return METALLLM_ATTN_OK;
}

int metalllmSublayerGraphLaunch(metalllmSublayerGraph* g, metalllm_stream_t stream) {
  if (!g || !g->exec) return METALLLM_ATTN_E_NULL;
  return hipGraphLaunch(g->exec, (hipStream_t)stream) == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

int metalllmSublayerGraphDestroy(metalllmSublayerGraph* g) {
  if (!g) return METALLLM_ATTN_OK;
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  if (g->h) (void)rocblas_destroy_handle(g->h);
  if (g->workspace) (void)hipFree(g->workspace);
  if (g->split) (void)hipFree(g->split);
  if (g->partial) (void)hipFree(g->partial);
  if (g->attn_ws) (void)hipFree(g->attn_ws);
  delete g;
  return METALLLM_ATTN_OK;
}

}  // extern "C"
