/* metalllm_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Drop-in for the three Metal kernels of metalLLM's attention layer:
 *   flashAttentionForward  /root/reference/attention.metal:56-164, dispatched at
 *                          /root/reference/model.h:459-473
 *   computeD               /root/reference/attention.metal:166-195, model.h:639-647
 *   flashAttentionBackward /root/reference/attention.metal:198-299, model.h:648-665
 * Arguments keep the reference's buffer-index order (q0 k1 v2 out3 l4 params5; dO0 O1 D2 params3;
 * dZ0 d1 l2 q3 k4 v5 dQ6 dK7 dV8 params9) with a HIP stream appended.
 *
 * Layouts (all row-major, caller-owned device memory, 16-byte aligned):
 *   q, k, v, out, dO, dK, dV : bf16 bit patterns, [B, T, NH, D] (one token row = N = NH*D elements;
 *                              for B = 1 this is the reference's [T, N] buffer)
 *   l (logsumexp), D         : fp32 [B, NH, T] (the reference indexes them [t*NH + h], one sequence)
 *   dQ                       : fp32 [B, T, NH, D]
 * flashAttentionBackward keeps the reference's dQ contract: the gradient is ADDED to the fp32
 * dQ buffer (the reference adds per-tile parts with fp32 atomics, attention.metal:292-296, into
 * the buffer model.h:549 zeroes before every backward). Here each dQ element has one owner that
 * reads, adds and writes it once, so the sum is deterministic and needs no atomics. dK and dV are
 * written in full (model.h:550-551 zeroes them and each key tile has one owner, so the reference
 * leaves the same values). flashAttentionBackwardWorkspace writes dQ in full instead (no zeroing
 * pass, no read of the old values). D holds the bf16-rounded value of rowsum(dO*O), stored as
 * fp32.
 *
 * Semantics: asynchronous on `stream` (NULL = the default stream); no allocation and no host
 * synchronisation. Calls on distinct streams may run concurrently, with two exceptions: the
 * workspace variant's workspace belongs to one call at a time, and flashAttentionBackwardNoAlloc
 * calls on one GPU share that GPU's fixed dS array, so they must be serialised. Library state
 * that outlives a call: (1) two per-device caches in host memory, filled by device queries on the
 * first call on that device and read-only afterwards: the number of flashAttentionForward's
 * persistent workgroups resident at once (CU count times occupancy) and the CU count the dQ
 * kernel of the workspace backward sizes its grid by; (2) the
 * METALLLM_ATTN_NOALLOC_SCRATCH_BYTES (64 MiB) device array of flashAttentionBackwardNoAlloc,
 * which the HIP runtime creates on every GPU where it loads the library's code object (at the
 * first launch of any of its kernels there) and keeps until the process ends, whether or not that
 * entry point is ever called. Each
 * entry point validates its arguments before touching the device and returns METALLLM_ATTN_OK or
 * a negative error code; a failed kernel launch returns METALLLM_ATTN_E_LAUNCH.
 * Supported shapes: M (= T) a positive multiple of 64, D in {64, 128}, N == NH*D, B >= 1,
 * B*M*N < 2^31 elements per tensor.
 */
#ifndef METALLLM_ATTN_H
#define METALLLM_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* metalllm_stream_t; /* same type as hipStream_t */

/* attention.metal:7-12 / main.cpp:114-119: {M, N, D, NH}; B is appended (the reference runs
 * one sequence). */
typedef struct AttentionParams {
  uint32_t M;  /* sequence length T */
  uint32_t N;  /* NH * D */
  uint32_t D;  /* head size, 64 or 128 */
  uint32_t NH; /* number of heads */
  uint32_t B;  /* batch */
} AttentionParams;

enum {
  METALLLM_ATTN_OK = 0,
  METALLLM_ATTN_E_NULL = -1,     /* a required pointer is NULL */
  METALLLM_ATTN_E_SEQLEN = -2,   /* M == 0 or M % 64 != 0 */
  METALLLM_ATTN_E_HEADDIM = -3,  /* D not in {64, 128} */
  METALLLM_ATTN_E_LAYOUT = -4,   /* N != NH * D, NH == 0 or B == 0 */
  METALLLM_ATTN_E_SIZE = -5,     /* a tensor exceeds 2^31 elements */
  METALLLM_ATTN_E_ALIGN = -6,    /* a tensor pointer is not 16-byte aligned */
  METALLLM_ATTN_E_LAUNCH = -7,   /* the kernel launch failed */
  METALLLM_ATTN_E_LIBRARY = -8,  /* a platform library call (rocBLAS, device allocation) failed */
  METALLLM_ATTN_E_CAPTURE = -9   /* per-device scratch would have to grow while the stream is being
                                    captured into a graph: call metalllmSublayerReserve first */
};

/* Replaces the flashAttentionForward dispatch at model.h:459-473 (attention.metal:56-164).
 * out = softmax(q k^T / sqrt(D) + causal mask) v per (b, head); l = logsumexp per query row. */
int flashAttentionForward(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out, float* l,
                          const AttentionParams* p, metalllm_stream_t stream);

/* Replaces the computeD dispatch at model.h:639-647 (attention.metal:166-195).
 * D[b,h,t] = bf16( sum_d bf16(dO*O) ). */
int computeD(const uint16_t* dO, const uint16_t* O, float* D, const AttentionParams* p,
             metalllm_stream_t stream);

/* Replaces the flashAttentionBackward dispatch at model.h:648-665 (attention.metal:198-299).
 * dZ is dO; d and l are computeD's and the forward's outputs. dQ += gradient (fp32, accumulated
 * into as in the reference: zero it first for the plain gradient); dK, dV = gradients (bf16).
 * Two kernels: dK/dV by key-block owners, then dQ by query-block owners, each recomputing the
 * softmax tile it needs. For D = 64 and M <= 256 (the reference's own shape) one kernel does
 * both: a workgroup per (b, head) keeps the dS tiles in LDS (dK, dV bit-identical to the
 * two-kernel path). */
int flashAttentionBackward(const uint16_t* dZ, const float* d, const float* l, const uint16_t* q,
                           const uint16_t* k, const uint16_t* v, float* dQ, uint16_t* dK, uint16_t* dV,
                           const AttentionParams* p, metalllm_stream_t stream);

/* Bytes of device workspace flashAttentionBackwardWorkspace needs for shape p: one 64x64 bf16
 * dS tile per (query tile, key tile <= query tile) of every (b, head), i.e.
 * B*NH*(M/64)*(M/64+1)/2 * 8192 (4.4e9 at B = NH = 16, M = 4096). No counterpart in the
 * reference (its backward keeps dS in threadgroup memory). */
int metalllmAttnBackwardWorkspaceSize(const AttentionParams* p, uint64_t* bytes);

/* The same backward as flashAttentionBackward (model.h:648-665), faster at long sequences: the
 * dK/dV kernel also stores every bf16 dS tile it computes into `workspace` (device memory, 16-byte
 * aligned, at least metalllmAttnBackwardWorkspaceSize bytes), and dQ = dS.K then streams those
 * tiles instead of recomputing the softmax. dK and dV are bit-identical to flashAttentionBackward's.
 * dQ is overwritten with the gradient (it does not accumulate into dQ, unlike
 * flashAttentionBackward): the caller needs no zeroing pass and the dQ kernel no read of 4*B*M*N
 * bytes, 1.1 GB of HBM traffic less per step at B = NH = 16, M = 4096, D = 128. Its values equal
 * what flashAttentionBackward adds into a zeroed dQ up to fp32 summation order. The workspace
 * holds no state between calls, but one
 * workspace must not serve two calls at once. Returns METALLLM_ATTN_E_NULL / _E_ALIGN / _E_SIZE
 * for a NULL, misaligned or too small workspace. At D = 64 no dS is stored and the workspace is
 * validated but not used: for M <= 256 it runs the same single kernel as flashAttentionBackward
 * there (dS stays in LDS); for longer sequences flashAttentionBackward's two kernels, the dQ kernel
 * writing dQ instead of adding into it (at this head size the recomputation is faster than the dS
 * round trip), so dQ, dK and dV equal flashAttentionBackward's into a zeroed dQ bit for bit.
 * No counterpart in the reference. */
int flashAttentionBackwardWorkspace(const uint16_t* dZ, const float* d, const float* l, const uint16_t* q,
                                    const uint16_t* k, const uint16_t* v, float* dQ, uint16_t* dK, uint16_t* dV,
                                    void* workspace, uint64_t workspace_bytes, const AttentionParams* p,
                                    metalllm_stream_t stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The same computation as
 * flashAttentionBackwardWorkspace (same kernels, bit-identical dQ, dK, dV; dQ written in full),
 * with the dS tiles in a fixed per-device array of METALLLM_ATTN_NOALLOC_SCRATCH_BYTES (64 MiB,
 * held by every GPU the library runs on until the process ends) instead of a caller workspace.
 * Calls no hipMalloc/hipFree. D = 128 shapes whose metalllmAttnBackwardWorkspaceSize exceeds the
 * array return METALLLM_ATTN_E_SIZE (e.g. B = 4, NH = 12, M = 1024 needs 53.5 MB and fits; B = 8
 * does not). D = 64 stores no dS tiles (see flashAttentionBackwardWorkspace) and accepts every
 * shape. All calls on one GPU share the array: calls that overlap on one GPU race. The first call
 * on a device looks up the array's address there. */
#define METALLLM_ATTN_NOALLOC_SCRATCH_BYTES (64ull << 20)
int flashAttentionBackwardNoAlloc(const uint16_t* dZ, const float* d, const float* l, const uint16_t* q,
                                  const uint16_t* k, const uint16_t* v, float* dQ, uint16_t* dK, uint16_t* dV,
                                  const AttentionParams* p, metalllm_stream_t stream);

/* ---- The sublayer around the attention core (attention.metal:19-53, 301-455) ----
 * Plain GEMMs with the reference kernels' names and buffer order. Row-major: X, attn_out (O), dZ,
 * q, k, v, dK, dV, dAttn, out are bf16 [B*M, N]; dQ and dX are fp32 [B*M, N]; weights (q_w, k_w,
 * v_w, proj_w and their gradients) are bf16 [N, N] indexed [input feature][output feature], dQw
 * fp32 [N, N]. Products are computed with fp32 accumulation and rounded once to the destination
 * type: computeQKV, projForward and projBackwarddX on rocBLAS gemm_ex; computeGradDx,
 * computeGradDw and projBackwarddW on hand-written kernels when B*M and N are multiples of 128
 * (rocBLAS otherwise). The "accumulate" kernels read their destination once and add to it, as
 * the reference's multiply_accumulate matmuls do; the caller zeroes those destinations first
 * (model.h:549-555). Validation: M, B, NH, D >= 1, N == NH*D a multiple of 8, tensors below 2^31
 * elements, non-NULL 16-byte aligned pointers. The first call on a device creates that device's
 * rocBLAS handle; computeGradDx/Dw keep a per-device buffer for the two-term bf16 split of dQ, and
 * projBackwarddW/computeGradDw one for fp32 partial sums of the weight gradients (both kept until
 * the process ends), so those calls must not overlap on different streams of one device.
 * Asynchronous on `stream`, except that a call which needs a larger buffer than the device holds
 * grows it: hipDeviceSynchronize, then hipFree and hipMalloc (refused with
 * METALLLM_ATTN_E_CAPTURE while `stream` is being captured into a graph). metalllmSublayerReserve
 * sizes the buffers once, after which calls at that shape or smaller never allocate or
 * synchronise. */

/* Sizes the current device's sublayer scratch (dQ split, weight-gradient partials, the phase
 * encoder's attention workspace) for shape p, synchronising the device if a buffer grows; the
 * GEMM entry points and metalllmSublayerEncode at shapes up to p then run without allocating.
 * No counterpart in the reference (model.h allocates every buffer once, :236-277). */
int metalllmSublayerReserve(const AttentionParams* p);

/* attention.metal:19-53, dispatched at model.h:446-457: q = X.q_w, k = X.k_w, v = X.v_w. When
 * q_w, k_w, v_w are equally spaced in memory (e.g. slices of one [3][N][N] weight) and q, k, v
 * are equally spaced without overlapping (e.g. slices of one [3][B*M][N] buffer), the three
 * products run as one batched library call, which is faster; any other layout runs three. */
int computeQKV(const uint16_t* X, uint16_t* q, uint16_t* k, uint16_t* v, const uint16_t* q_w, const uint16_t* k_w,
               const uint16_t* v_w, const AttentionParams* p, metalllm_stream_t stream);

/* attention.metal:385-405, model.h:474-482: out = attn_out.proj_w. */
int projForward(const uint16_t* attn_out, const uint16_t* proj_w, uint16_t* out, const AttentionParams* p,
                metalllm_stream_t stream);

/* attention.metal:407-430, model.h:621-629: dProjw += attn_out^T.dZ (bf16, accumulated). */
int projBackwarddW(const uint16_t* attn_out, const uint16_t* dZ, uint16_t* dProjw, const AttentionParams* p,
                   metalllm_stream_t stream);

/* attention.metal:432-455, model.h:630-638: dAttn = dZ.proj_w^T (bf16). */
int projBackwarddX(const uint16_t* dZ, const uint16_t* proj_w, uint16_t* dAttn, const AttentionParams* p,
                   metalllm_stream_t stream);

/* attention.metal:301-341, model.h:666-677: dX += dQ.q_w^T + dK.k_w^T + dV.v_w^T (fp32, accumulated;
 * dQ is the fp32 gradient flashAttentionBackward produced). */
int computeGradDx(float* dX, const uint16_t* qw, const uint16_t* kw, const uint16_t* vw, const float* dQ,
                  const uint16_t* dK, const uint16_t* dV, const AttentionParams* p, metalllm_stream_t stream);

/* attention.metal:343-383, model.h:679-690: dQw += X^T.dQ (fp32), dKw += X^T.dK, dVw += X^T.dV (bf16);
 * all accumulated. */
int computeGradDw(const uint16_t* x, const float* dQ, const uint16_t* dK, const uint16_t* dV, float* dQw,
                  uint16_t* dKw, uint16_t* dVw, const AttentionParams* p, metalllm_stream_t stream);

/* elementwise.metal:19-28, model.h:692: out[i] = bf16(in[i]) for i < count (round to nearest
 * even; NaN stays NaN). The reference's buffer order (in0 out1 count2). Allocates nothing.
 * count == 0 is a no-op; otherwise both pointers non-NULL and 16-byte aligned. */
int castFloatToBfloat(const float* in, uint16_t* out, uint32_t count, metalllm_stream_t stream);

/* elementwise.metal:7-17, model.h:368-376 (used at :483,618,695): out[i] = bf16(a[i] + b[i]) for
 * i < count; out may alias a or b. The reference's buffer order (a0 b1 out2 count3). count == 0
 * is a no-op; otherwise non-NULL 16-byte aligned pointers. */
int residualAdd(const uint16_t* a, const uint16_t* b, uint16_t* out, uint32_t count, metalllm_stream_t stream);

/* layernorm.metal:3-8 / main.cpp:89-96: {rows, cols, group_size, eps}. group_size (the reference's
 * threads per row) is not used here: one wave handles a row. */
typedef struct LayernormParams {
  uint32_t rows;
  uint32_t cols;       /* a multiple of 8, at most 4096 */
  uint32_t group_size;
  float eps;           /* the reference's default is 1e-5 */
} LayernormParams;

/* layernorm.metal:10-70, dispatched by encodeLayernormForward (model.h:385-396). Per row of x
 * (bf16 [rows, cols]): mean and variance in fp32, stdev[row] = sqrt(var + eps) (fp32),
 * x_norm = bf16((x - mean) / stdev), out = bf16(gamma * x_norm_fp32 + beta) (gamma, beta bf16
 * [cols]). Buffer order x0 x_norm1 out2 gamma3 beta4 stdev5 params6. */
int layernormForward(const uint16_t* x, uint16_t* x_norm, uint16_t* out, const uint16_t* gamma, const uint16_t* beta,
                     float* stdev, const LayernormParams* p, metalllm_stream_t stream);

/* layernorm.metal:73-127, dispatched by encodeLayernormBackward (model.h:398-410). In place on dZ
 * (bf16 [rows, cols]): dgamma[c] += sum_rows bf16(x_norm*dZ), dbeta[c] += sum_rows dZ (fp32
 * [cols], accumulated: the caller zeroes them, model.h:543-548); dx_norm = bf16(dZ*gamma) is
 * written when dx_norm is non-NULL (the reference's scratch, model.h's dXnormBuffer); then
 * dZ = bf16((dx_norm - mean(dx_norm) - x_norm*mean(bf16(dx_norm*x_norm))) / stdev). Buffer order
 * dZ0 x_norm_cache1 gamma2 stdev3 dx_norm5 dgamma6 dbeta7 params8 (the reference binds nothing
 * at index 4). */
int layernormBackward(uint16_t* dZ, const uint16_t* x_norm_cache, const uint16_t* gamma, const float* stdev,
                      uint16_t* dx_norm, float* dgamma, float* dbeta, const LayernormParams* p,
                      metalllm_stream_t stream);

/* ---- Phase encoder (model.h:441-508 forward, :538-708 backward: one command buffer per phase) ----
 * The attention sublayer's buffers, as model.h's BlockBuffers hold them (model.h:236-277). All
 * device pointers, 16-byte aligned; shapes from AttentionParams as above (R = B*M rows, N = C
 * features): activations [R, N], weights [N, N] [input][output], l and Dsum fp32 [B, NH, M]. */
typedef struct metalllmSublayerBuffers {
  const uint16_t* X;      /* bf16: the sublayer input (ln1 output, model.h:447)             */
  const uint16_t* q_w;    /* bf16 weights                                                     */
  const uint16_t* k_w;
  const uint16_t* v_w;
  const uint16_t* proj_w;
  uint16_t* q;            /* bf16, written by the forward phase, read by the backward phase  */
  uint16_t* k;
  uint16_t* v;
  uint16_t* attn_out;     /* bf16 attention output O                                          */
  float* l;               /* fp32 logsumexp                                                    */
  uint16_t* out;          /* bf16 sublayer output (forward phase)                              */
  const uint16_t* dOut;   /* bf16 gradient at the sublayer output (model.h's dBranch, :622)    */
  uint16_t* dAttn;        /* bf16 gradient at O (model.h's dZAttn, :633)                       */
  float* Dsum;            /* fp32 computeD output                                               */
  float* dQ;              /* fp32                                                               */
  uint16_t* dK;           /* bf16                                                               */
  uint16_t* dV;
  float* dX;              /* fp32 gradient at X (model.h's dXAttn)                              */
  float* dQw;             /* fp32 [N, N]                                                        */
  uint16_t* dKw;          /* bf16 [N, N]                                                        */
  uint16_t* dVw;
  uint16_t* dProjw;
  uint16_t* dX_bf16;      /* optional (NULL: skipped): bf16(dX), model.h:692                   */
  /* Optional: the rest of the block's attention half (model.h:445 ln1, :483 and :695 residual
   * adds, :692-694 cast and ln1 backward). All NULL: the sublayer alone. When `hidden` is set,
   * every field below must be, X becomes an output (phase 0 writes ln1(hidden) into it) and
   * dX_bf16 is ignored (phase 1 casts dX into dStream). */
  const uint16_t* hidden;   /* bf16 [R, N]: the block input                                    */
  const uint16_t* ln_gamma; /* bf16 [N]                                                         */
  const uint16_t* ln_beta;  /* bf16 [N]                                                         */
  uint16_t* ln_xnorm;       /* bf16 [R, N]: ln1's x_norm cache                                  */
  float* ln_stdev;          /* fp32 [R]                                                         */
  float* ln_dgamma;         /* fp32 [N], zeroed by phase 1 (model.h:543-544)                    */
  float* ln_dbeta;          /* fp32 [N]                                                         */
  uint16_t* residual;       /* bf16 [R, N]: phase 0 output hidden + out (model.h's residual1)   */
  uint16_t* dStream;        /* bf16 [R, N]: phase 1 output, the gradient at hidden              */
  float ln_eps;             /* ln1's eps (the reference's default is 1e-5)                      */
} metalllmSublayerBuffers;

typedef struct metalllmSublayerGraph metalllmSublayerGraph;

/* Enqueues one phase of the sublayer on `stream`, in model.h's order.
 *   phase 0 (model.h:444-483): computeQKV, flashAttentionForward, projForward.
 *   phase 1 (model.h:549-555, 620-693): projBackwarddW, projBackwarddX, computeD,
 *            flashAttentionBackwardWorkspace, computeGradDx, computeGradDw, and
 *            castFloatToBfloat(dX) when dX_bf16 is set. dX, dQw, dKw, dVw and dProjw, which
 *            model.h zeroes before the pass and accumulates into, have one producer each here:
 *            they are written as 0 + the gradient, without being zeroed or read. When B*M and N
 *            are multiples of 128, dProjw is computed last, in computeGradDw's launch, so the
 *            four weight gradients are summed over other row chunks than the entry points use
 *            (equal up to fp32 summation order); every other output equals the entry points'
 *            chain bit for bit.
 * With the block fields set: phase 0 starts with layernormForward(hidden -> X) and ends with
 * residualAdd(hidden, out -> residual); phase 1 also zeroes ln_dgamma/ln_dbeta, casts dX into
 * dStream, then runs layernormBackward(dStream) and residualAdd(dStream, dOut -> dStream).
 * Validation: the GEMM rules and the attention rules above, every pointer the phase uses.
 * Uses the device's shared rocBLAS handle and scratch like the GEMM entry points above (plus a
 * per-device attention workspace, metalllmAttnBackwardWorkspaceSize bytes, grown on demand with
 * the same device synchronisation; metalllmSublayerReserve avoids it). */
int metalllmSublayerEncode(int phase, const metalllmSublayerBuffers* b, const AttentionParams* p,
                           metalllm_stream_t stream);

/* Records the same phase once as a HIP graph (pointers and shapes fixed at creation) and returns
 * it in *out; metalllmSublayerGraphLaunch replays it on `stream` with one launch, reading the
 * buffers' current contents. A graph owns its rocBLAS handle, workspaces and scratch (allocated
 * here, freed by Destroy), so it never depends on memory other calls may reallocate. Replays of
 * one graph must not overlap each other; Destroy only after the last replay completed. These
 * three have no single counterpart in the reference (it re-encodes the command buffer each step,
 * model.h:441,587). */
int metalllmSublayerGraphCreate(int phase, const metalllmSublayerBuffers* b, const AttentionParams* p,
                                metalllmSublayerGraph** out);
int metalllmSublayerGraphLaunch(metalllmSublayerGraph* g, metalllm_stream_t stream);
int metalllmSublayerGraphDestroy(metalllmSublayerGraph* g);

/* Bench hook (no counterpart in the reference): launches one of the kernels of the two backward
 * entry points on `stream`: part 0 = dK/dV and part 1 = dQ recomputing the softmax
 * (flashAttentionBackward is exactly part 0 then part 1); part 2 = dK/dV storing dS into the
 * workspace and part 3 = dQ from the stored dS (flashAttentionBackwardWorkspace is exactly part 2
 * then part 3). Timing the parts separately measures the same work. Same validation and return
 * codes as those entry points (parts 0 and 1 ignore the workspace arguments); a part outside
 * 0..3 returns METALLLM_ATTN_E_LAYOUT. For D = 64 and M <= 256 parts 0 and 2 launch the single
 * fused kernel (part 0 adds dQ, part 2 writes it) and parts 1 and 3 launch nothing. For D = 64 and
 * longer sequences parts 2 and 3 launch parts 0's and 1's kernels, part 3 writing dQ. */
int metalllmAttnBackwardPart(int part, const uint16_t* dZ, const float* d, const float* l, const uint16_t* q,
                             const uint16_t* k, const uint16_t* v, float* dQ, uint16_t* dK, uint16_t* dV,
                             void* workspace, uint64_t workspace_bytes, const AttentionParams* p,
                             metalllm_stream_t stream);

/* Static description of an error code (no counterpart in the reference, which has no error
 * path per kernel; model.h:333-336,361-365 only print). */
const char* metalllmAttnErrorString(int code);

/* Test hook (no counterpart in the reference): writes, for workgroup ids 0..count-1 of the
 * forward (kind 0), backward dK/dV (kind 1) or backward dQ (kind 2) grid of shape p, the
 * (pair, block) each one owns into
 * out[2*i], out[2*i+1]. Returns the grid size, or a negative error code. Host-only. */
int metalllmAttnWorkMap(int kind, const AttentionParams* p, int32_t* out, int32_t count);

/* Test hook (no counterpart in the reference): the item assignment of the persistent forward
 * that flashAttentionForward runs when B*NH*ceil(M/128) is at most twice the number of workgroups
 * resident at once (one workgroup per resident slot, each taking
 * (pair, query block) items in turn), for a grid of `grid` workgroups: writes, for workgroup
 * w = 0..grid-1 in turn and each of its items in the order it runs them, the triple
 * (w, pair, block) into out[3*i..3*i+2], at most `count` items. Returns the number of items of
 * the whole grid, or a negative error code. Host-only. */
int metalllmAttnForwardItems(const AttentionParams* p, int32_t grid, int32_t* out, int32_t count);

#ifdef __cplusplus
}
#endif

#endif /* METALLLM_ATTN_H */
