// gemm_oracle.cpp -- CPU oracle for the GEMMs of metalLLM's attention sublayer.
//
// TEST INFRASTRUCTURE ONLY (linked into liboracle_attn.so with attn_oracle.cpp): loaded by tests/
// and bench.py's cpu_baseline leg as the checker, never by the product.
//
// Restates the six sublayer kernels around the attention core, written from their source text:
//   computeQKV      /root/reference/attention.metal:19-53   Q,K,V = X.Wq, X.Wk, X.Wv        (bf16 out)
//   projForward     /root/reference/attention.metal:385-405 out = O.Wp                       (bf16 out)
//   projBackwarddW  /root/reference/attention.metal:407-430 dWp += O^T.dZ  (accumulate, bf16 dest)
//   projBackwarddX  /root/reference/attention.metal:432-455 dO = dZ.Wp^T                     (bf16 out)
//   computeGradDx   /root/reference/attention.metal:301-341 dX += dQ.Wq^T; += dK.Wk^T; += dV.Wv^T
//                                                           (accumulate, fp32 dest, dQ is fp32)
//   computeGradDw   /root/reference/attention.metal:343-383 dWq += X^T.dQ (fp32 dest, dQ fp32);
//                                                           dWk += X^T.dK, dWv += X^T.dV (bf16 dest)
// Matrices are row-major: X, O, dZ, Q, K, V, dK, dV bf16 [R, C] and dQ, dX fp32 [R, C] with R = B*T
// rows (the reference runs one sequence, R = T = params.M) and C = N = NH*D columns; W bf16 [C, C]
// indexed [input feature][output feature] (attention.metal:30-41: B = W.slice(cols), all K rows).
//
// Each matmul2d (attention.metal:38-52, 311-314, 351-355, 393-404, 414-429, 441-454) reduces over the
// full K extent into its destination; the oracle sums the exact products in fp32 in k order, then
// adds the destination's previous value once (multiply_accumulate mode) and rounds to the
// destination type (bf16 round-to-nearest-even). Apple's accumulation order is not published
// (parity unpinned at the fp32-rounding level); tests bound that difference.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));  // inf/nan
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

enum { T_BF16 = 0, T_F32 = 1 };

float load(const void* p, int type, size_t i) {
  return type == T_BF16 ? bf2f(((const uint16_t*)p)[i]) : ((const float*)p)[i];
}

template <typename F>
void parallel_rows(int rows, int threads, F fn) {
  if (threads <= 1 || rows < 2) {
    for (int r = 0; r < rows; ++r) fn(r);
    return;
  }
  std::vector<std::thread> pool;
  const int per = (rows + threads - 1) / threads;
  for (int t = 0; t < threads; ++t) {
    const int r0 = t * per, r1 = std::min(rows, r0 + per);
    if (r0 >= r1) break;
    pool.emplace_back([=] {
      for (int r = r0; r < r1; ++r) fn(r);
    });
  }
  for (auto& th : pool) th.join();
}

// C[M][N] (= or +=) op(A)[M][K] . op(B)[K][N], all row-major. op(A) = A [M][K] (lda) or, with
// ta, A^T where A is stored [K][M]; likewise op(B) = B [K][N] (ldb) or B^T with B stored [N][K].
// Products are exact in fp32 (bf16 x bf16; an fp32 operand makes them single-rounded); the sum runs
// in fp32 in k order; accumulate adds the previous destination once at the end.
void gemm(int ta, int tb, int M, int N, int K, const void* A, int at, int lda, const void* B, int bt, int ldb,
          void* C, int ct, int ldc, int accumulate, int threads) {
  parallel_rows(M, threads, [&](int m) {
    for (int n = 0; n < N; ++n) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) {
        const float a = load(A, at, ta ? (size_t)k * lda + m : (size_t)m * lda + k);
        const float b = load(B, bt, tb ? (size_t)n * ldb + k : (size_t)k * ldb + n);
        acc += a * b;
      }
      const size_t ci = (size_t)m * ldc + n;
      if (ct == T_BF16) {
        uint16_t* c = (uint16_t*)C;
        c[ci] = f2bf(accumulate ? bf2f(c[ci]) + acc : acc);
      } else {
        float* c = (float*)C;
        c[ci] = accumulate ? c[ci] + acc : acc;
      }
    }
  });
}

}  // namespace

extern "C" {

// Generic row-major GEMM of the oracle (types: 0 bf16 bits, 1 fp32). Returns 0.
int oracle_gemm(int ta, int tb, int M, int N, int K, const void* A, int at, int lda, const void* B, int bt, int ldb,
                void* C, int ct, int ldc, int accumulate, int threads) {
  if (M < 0 || N < 0 || K < 0 || !A || !B || !C) return -1;
  gemm(ta, tb, M, N, K, A, at, lda, B, bt, ldb, C, ct, ldc, accumulate, threads);
  return 0;
}

// attention.metal:19-53: Q = X.Wq, K = X.Wk, V = X.Wv over R rows of C = N features.
int oracle_computeQKV(const uint16_t* X, uint16_t* q, uint16_t* k, uint16_t* v, const uint16_t* qw,
                      const uint16_t* kw, const uint16_t* vw, int R, int C, int threads) {
  gemm(0, 0, R, C, C, X, T_BF16, C, qw, T_BF16, C, q, T_BF16, C, 0, threads);
  gemm(0, 0, R, C, C, X, T_BF16, C, kw, T_BF16, C, k, T_BF16, C, 0, threads);
  gemm(0, 0, R, C, C, X, T_BF16, C, vw, T_BF16, C, v, T_BF16, C, 0, threads);
  return 0;
}

// attention.metal:385-405: out = O.Wp.
int oracle_projForward(const uint16_t* attn_out, const uint16_t* proj_w, uint16_t* out, int R, int C, int threads) {
  gemm(0, 0, R, C, C, attn_out, T_BF16, C, proj_w, T_BF16, C, out, T_BF16, C, 0, threads);
  return 0;
}

// attention.metal:407-430: dWp[k][n] += sum_r O[r][k] dZ[r][n] (multiply_accumulate, bf16 dest).
int oracle_projBackwarddW(const uint16_t* attn_out, const uint16_t* dZ, uint16_t* dProjw, int R, int C, int threads) {
  gemm(1, 0, C, C, R, attn_out, T_BF16, C, dZ, T_BF16, C, dProjw, T_BF16, C, 1, threads);
  return 0;
}

// attention.metal:432-455: dAttn[r][k] = sum_n dZ[r][n] Wp[k][n].
int oracle_projBackwarddX(const uint16_t* dZ, const uint16_t* proj_w, uint16_t* dAttn, int R, int C, int threads) {
  gemm(0, 1, R, C, C, dZ, T_BF16, C, proj_w, T_BF16, C, dAttn, T_BF16, C, 0, threads);
  return 0;
}

// attention.metal:301-341: dX += dQ.Wq^T, then += dK.Wk^T, then += dV.Wv^T (three accumulate runs
// into the fp32 dX; dQ is read as fp32).
int oracle_computeGradDx(float* dX, const uint16_t* qw, const uint16_t* kw, const uint16_t* vw, const float* dQ,
                         const uint16_t* dK, const uint16_t* dV, int R, int C, int threads) {
  gemm(0, 1, R, C, C, dQ, T_F32, C, qw, T_BF16, C, dX, T_F32, C, 1, threads);
  gemm(0, 1, R, C, C, dK, T_BF16, C, kw, T_BF16, C, dX, T_F32, C, 1, threads);
  gemm(0, 1, R, C, C, dV, T_BF16, C, vw, T_BF16, C, dX, T_F32, C, 1, threads);
  return 0;
}

// attention.metal:343-383: dWq += X^T.dQ (fp32 dest, dQ fp32), dWk += X^T.dK, dWv += X^T.dV (bf16).
int oracle_computeGradDw(const uint16_t* x, const float* dQ, const uint16_t* dK, const uint16_t* dV, float* dQw,
                         uint16_t* dKw, uint16_t* dVw, int R, int C, int threads) {
  gemm(1, 0, C, C, R, x, T_BF16, C, dQ, T_F32, C, dQw, T_F32, C, 1, threads);
  gemm(1, 0, C, C, R, x, T_BF16, C, dK, T_BF16, C, dKw, T_BF16, C, 1, threads);
  gemm(1, 0, C, C, R, x, T_BF16, C, dV, T_BF16, C, dVw, T_BF16, C, 1, threads);
  return 0;
}

}  // extern "C"
