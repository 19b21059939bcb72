// glue.hip -- the kernels of metalLLM's pre-LN block that sit around the attention sublayer
// (declared in include/metalllm_attn.h):
//   castFloatToBfloat  elementwise.metal:19-28  out[i] = bf16(in[i])  (model.h:692: the fp32 dX of
//                      computeGradDx handed to the layernorm backward as bf16)
//   residualAdd        elementwise.metal:7-17   out[i] = bf16(a[i] + b[i])  (model.h:483,618,695)
//   layernormForward   layernorm.metal:10-70    per row: mean, variance, stdev = sqrt(var + eps),
//                      x_norm = bf16((x - mean)/stdev), out = bf16(gamma*xn + beta)  (model.h:385-396)
//   layernormBackward  layernorm.metal:73-127   dgamma += bf16(xn*dZ), dbeta += dZ (fp32, per column),
//                      dx_norm = bf16(dZ*gamma), dZ <- bf16(rstd*(dxn - mean(dxn) - xn*mean(bf16(dxn*xn))))
//                      (model.h:398-410, in place on dZ)
// All are HBM-bound. The elementwise kernels stream with 16-byte accesses in grid-stride loops.
// The layernorm kernels give each row to one wave: the row stays in registers as packed bf16
// (cols/512 16-byte chunks per lane), its sums are wave reductions, and it is read once and written
// once. The backward's column sums (dgamma, dbeta) are accumulated per workgroup over many rows in
// registers and LDS, then added with one fp32 atomic per column per workgroup. The reference adds
// one atomic per element from every row.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/metalllm_attn.h"

namespace {

// float -> bf16, round to nearest even (Metal's float -> bfloat conversion); NaN stays a quiet
// NaN of the same sign, infinities and overflow to infinity as in IEEE rounding.
__device__ __forceinline__ uint32_t to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__global__ void __launch_bounds__(256) cast_kernel(const float* __restrict__ in, uint16_t* __restrict__ out,
                                                   uint32_t count) {
  const size_t n4 = count / 4;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = ((const float4*)in)[i];
    ((uint2*)out)[i] = uint2{to_bf16(v.x) | (to_bf16(v.y) << 16), to_bf16(v.z) | (to_bf16(v.w) << 16)};
  }
  // the count % 4 tail
  const size_t t = 4 * n4 + blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (t < count) out[t] = (uint16_t)to_bf16(in[t]);
}

unsigned grid_for(size_t items) { return (unsigned)std::max<size_t>(1, std::min<size_t>((items + 255) / 256, 8192)); }

__device__ __forceinline__ float bf_f(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf_round(float f) { return bf_f(to_bf16(f)); }

// out = bf16(a + b), eight elements per thread and step
__global__ void __launch_bounds__(256) residual_kernel(const uint4* __restrict__ a, const uint4* __restrict__ b,
                                                       uint4* __restrict__ out, uint32_t count) {
  const size_t n8 = count / 8;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n8; i += stride) {
    const uint4 x = a[i], y = b[i];
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ys[4] = {y.x, y.y, y.z, y.w};
    uint32_t r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      r[j] = to_bf16(bf_f(xs[j] & 0xffffu) + bf_f(ys[j] & 0xffffu)) |
             (to_bf16(bf_f(xs[j] >> 16) + bf_f(ys[j] >> 16)) << 16);
    out[i] = uint4{r[0], r[1], r[2], r[3]};
  }
  const size_t t = 8 * n8 + blockIdx.x * (size_t)blockDim.x + threadIdx.x;  // the count % 8 tail
  if (t < count) {
    const uint16_t* a16 = (const uint16_t*)a;
    const uint16_t* b16 = (const uint16_t*)b;
    ((uint16_t*)out)[t] = (uint16_t)to_bf16(bf_f(a16[t]) + bf_f(b16[t]));
  }
}

// Sum over the 64 lanes of a wave, the same result in every lane.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Row layout in a wave: lane l holds the 16-byte chunks c = l + 64 j (j < NCH) of the row, i.e.
// columns 8c .. 8c + 7; chunks past cols/8 are absent (their lanes hold zeros and skip stores).
template <int NCH>
struct RowChunks {
  uint4 v[NCH];
};

template <int NCH>
__device__ __forceinline__ void load_row(const uint4* row, int nchunk, int lane, RowChunks<NCH>& r) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + 64 * j;
    r.v[j] = c < nchunk ? row[c] : uint4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void unpack8(const uint4& u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = bf_f(w[k] & 0xffffu);
    f[2 * k + 1] = bf_f(w[k] >> 16);
  }
}
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = to_bf16(f[2 * k]) | (to_bf16(f[2 * k + 1]) << 16);
  return uint4{w[0], w[1], w[2], w[3]};
}

// layernorm.metal:10-70, one row per wave, four waves per workgroup.
template <int NCH>
__global__ void __launch_bounds__(256) ln_fwd_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ xnorm,
                                                     uint16_t* __restrict__ out, const uint16_t* __restrict__ gamma,
                                                     const uint16_t* __restrict__ beta, float* __restrict__ stdev,
                                                     uint32_t rows, uint32_t cols, float eps) {
  const int lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nchunk = (int)(cols / 8);
  const size_t base = (size_t)row * cols;
  RowChunks<NCH> r;
  load_row<NCH>((const uint4*)(x + base), nchunk, lane, r);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    float f[8];
    unpack8(r.v[j], f);
#pragma unroll
    for (int k = 0; k < 8; ++k) s += f[k];
  }
  const float mean = wave_sum(s) / (float)cols;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    if (lane + 64 * j >= nchunk) continue;
    float f[8];
    unpack8(r.v[j], f);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float d = f[k] - mean;
      q += d * d;
    }
  }
  const float var = wave_sum(q) / (float)cols;
  const float sd = sqrtf(var + eps);
  const float rstd = 1.0f / sd;
  if (lane == 0) stdev[row] = sd;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane + 64 * j;
    if (c >= nchunk) continue;
    float f[8], g[8], b[8], xn[8], o[8];
    unpack8(r.v[j], f);
    unpack8(((const uint4*)gamma)[c], g);
    unpack8(((const uint4*)beta)[c], b);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      xn[k] = (f[k] - mean) * rstd;
      o[k] = g[k] * xn[k] + b[k];  // two roundings (no contraction: built with -ffp-contract=off)
    }
    ((uint4*)(xnorm + base))[c] = pack8(xn);
    ((uint4*)(out + base))[c] = pack8(o);
  }
}

// layernorm.metal:73-127. Wave w of workgroup g handles rows g*4 + w, then + 4*gridDim.x, ...;
// each lane keeps the dgamma/dbeta partial sums of its own columns across those rows; the four
// waves' partials meet in LDS and one fp32 atomic per column adds the workgroup's sum.
template <int NCH>
__global__ void __launch_bounds__(256) ln_bwd_kernel(uint16_t* __restrict__ dZ, const uint16_t* __restrict__ xnorm,
                                                     const uint16_t* __restrict__ gamma,
                                                     const float* __restrict__ stdev, uint16_t* __restrict__ dxnorm,
                                                     float* __restrict__ dgamma, float* __restrict__ dbeta,
                                                     uint32_t rows, uint32_t cols) {
  __shared__ float red[2][4][64 * NCH * 8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunk = (int)(cols / 8);
  float pg[NCH][8], pb[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) pg[j][k] = pb[j][k] = 0.0f;
  for (uint32_t row = blockIdx.x * 4 + wave; row < rows; row += 4 * gridDim.x) {
    const size_t base = (size_t)row * cols;
    RowChunks<NCH> dz, xn;
    load_row<NCH>((const uint4*)(dZ + base), nchunk, lane, dz);
    load_row<NCH>((const uint4*)(xnorm + base), nchunk, lane, xn);
    float dxn[NCH][8];
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + 64 * j;
      float z[8], x[8], g[8];
      unpack8(dz.v[j], z);
      unpack8(xn.v[j], x);
      if (c < nchunk) unpack8(((const uint4*)gamma)[c], g);
      else
#pragma unroll
        for (int k = 0; k < 8; ++k) g[k] = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        pg[j][k] += bf_round(x[k] * z[k]);  // bfloat * bfloat is a bfloat
        pb[j][k] += z[k];
        dxn[j][k] = bf_round(z[k] * g[k]);
        s1 += dxn[j][k];
        s2 += bf_round(dxn[j][k] * x[k]);
      }
      if (dxnorm && c < nchunk) ((uint4*)(dxnorm + base))[c] = pack8(dxn[j]);
    }
    const float rs1 = wave_sum(s1) / (float)cols;
    const float rs2 = wave_sum(s2) / (float)cols;
    const float rdev = 1.0f / stdev[row];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = lane + 64 * j;
      if (c >= nchunk) continue;
      float x[8], o[8];
      unpack8(xn.v[j], x);
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] = rdev * ((dxn[j][k] - rs1) - x[k] * rs2);
      ((uint4*)(dZ + base))[c] = pack8(o);
    }
  }
  // column partials of the four waves -> one atomic per column
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int col = 8 * (lane + 64 * j) + k;
      red[0][wave][col] = pg[j][k];
      red[1][wave][col] = pb[j][k];
    }
  __syncthreads();
  for (uint32_t col = threadIdx.x; col < cols; col += 256) {
    const float g = red[0][0][col] + red[0][1][col] + red[0][2][col] + red[0][3][col];
    const float b = red[1][0][col] + red[1][1][col] + red[1][2][col] + red[1][3][col];
    atomicAdd(dgamma + col, g);
    atomicAdd(dbeta + col, b);
  }
}

int validate_ln(const LayernormParams* p) {
  if (!p) return METALLLM_ATTN_E_NULL;
  if (p->rows == 0 || p->cols == 0 || p->cols % 8 || p->cols > 4096) return METALLLM_ATTN_E_LAYOUT;
  if ((uint64_t)p->rows * p->cols >= (1ull << 31)) return METALLLM_ATTN_E_SIZE;
  if (!(p->eps >= 0.0f)) return METALLLM_ATTN_E_LAYOUT;
  return METALLLM_ATTN_OK;
}

bool al16(const void* q) { return ((uintptr_t)q & 15u) == 0; }

}  // namespace

extern "C" {

int residualAdd(const uint16_t* a, const uint16_t* b, uint16_t* out, uint32_t count, metalllm_stream_t stream) {
  if (count == 0) return METALLLM_ATTN_OK;
  if (!a || !b || !out) return METALLLM_ATTN_E_NULL;
  if (!al16(a) || !al16(b) || !al16(out)) return METALLLM_ATTN_E_ALIGN;
  hipLaunchKernelGGL(residual_kernel, dim3(grid_for(count / 8 + 1)), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)a, (const uint4*)b, (uint4*)out, count);
  return hipGetLastError() == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

int layernormForward(const uint16_t* x, uint16_t* x_norm, uint16_t* out, const uint16_t* gamma, const uint16_t* beta,
                     float* stdev, const LayernormParams* p, metalllm_stream_t stream) {
  const int rc = validate_ln(p);
  if (rc) return rc;
  if (!x || !x_norm || !out || !gamma || !beta || !stdev) return METALLLM_ATTN_E_NULL;
  if (!al16(x) || !al16(x_norm) || !al16(out) || !al16(gamma) || !al16(beta) || !al16(stdev))
    return METALLLM_ATTN_E_ALIGN;
  const dim3 grid((p->rows + 3) / 4);
  const hipStream_t s = (hipStream_t)stream;
  const int nch = (int)((p->cols / 8 + 63) / 64);
#define LNF(N) hipLaunchKernelGGL(ln_fwd_kernel<N>, grid, dim3(256), 0, s, x, x_norm, out, gamma, beta, stdev, p->rows, p->cols, p->eps)
  switch (nch) {
    case 1: LNF(1); break;
    case 2: LNF(2); break;
    case 3: LNF(3); break;
    case 4: LNF(4); break;
    case 5: LNF(5); break;
    case 6: LNF(6); break;
    case 7: LNF(7); break;
    default: LNF(8); break;
  }
#undef LNF
  return hipGetLastError() == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

int layernormBackward(uint16_t* dZ, const uint16_t* x_norm_cache, const uint16_t* gamma, const float* stdev,
                      uint16_t* dx_norm, float* dgamma, float* dbeta, const LayernormParams* p,
                      metalllm_stream_t stream) {
  const int rc = validate_ln(p);
  if (rc) return rc;
  if (!dZ || !x_norm_cache || !gamma || !stdev || !dgamma || !dbeta) return METALLLM_ATTN_E_NULL;
  if (!al16(dZ) || !al16(x_norm_cache) || !al16(gamma) || !al16(stdev) || !al16(dgamma) || !al16(dbeta) ||
      (dx_norm && !al16(dx_norm)))
    return METALLLM_ATTN_E_ALIGN;
  // enough workgroups to fill the chip, each summing its columns over many rows
  const dim3 grid(std::min<uint32_t>((p->rows + 3) / 4, 1024));
  const hipStream_t s = (hipStream_t)stream;
  const int nch = (int)((p->cols / 8 + 63) / 64);
#define LNB(N) hipLaunchKernelGGL(ln_bwd_kernel<N>, grid, dim3(256), 0, s, dZ, x_norm_cache, gamma, stdev, dx_norm, dgamma, dbeta, p->rows, p->cols)
  switch (nch) {
    case 1: LNB(1); break;
    case 2: LNB(2); break;
    case 3: LNB(3); break;
    case 4: LNB(4); break;
    case 5: LNB(5); break;
    case 6: LNB(6); break;
    case 7: LNB(7); break;
    default: LNB(8); break;
  }
#undef LNB
  return hipGetLastError() == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

int castFloatToBfloat(const float* in, uint16_t* out, uint32_t count, metalllm_stream_t stream) {
  if (count == 0) return METALLLM_ATTN_OK;
  if (!in || !out) return METALLLM_ATTN_E_NULL;
  if (((uintptr_t)in & 15u) || ((uintptr_t)out & 15u)) return METALLLM_ATTN_E_ALIGN;
  hipLaunchKernelGGL(cast_kernel, dim3(grid_for(count / 4 + 1)), dim3(256), 0, (hipStream_t)stream, in, out, count);
  return hipGetLastError() == hipSuccess ? METALLLM_ATTN_OK : METALLLM_ATTN_E_LAUNCH;
}

}  // extern "C"
