/*
 * nuvla_forge_hip.h -- C ABI of the MI355X (gfx950) kernels behind
 * nuvla_forge_amd.kernels.
 *
 * Every entry point
 *   - takes device pointers, int64_t sizes/strides (in elements) and a
 *     hipStream_t passed as `void *` (NULL = the null stream);
 *   - only enqueues work on that stream: it never allocates, frees or
 *     synchronises (callers own every buffer, including workspaces);
 *   - returns NF_OK (0) or a negative status; nf_last_error() then describes
 *     the failure (thread-local string, valid until the next call on the
 *     same thread).
 *
 * Element types are passed as NF_DTYPE_* codes.  Row strides ("ld_*") are in
 * elements; the last dimension is always unit-stride.  A row stride of 0 is
 * allowed for the [B, N] conditioning inputs (a broadcast `expand` view).
 *
 * The functions replace the launch sites of the reference's Triton kernels;
 * each declaration cites the reference code it stands in for (paths relative
 * to the nuvla-forge repository root).
 */
#ifndef NUVLA_FORGE_HIP_H
#define NUVLA_FORGE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NF_ABI_VERSION 3

/* element type codes */
#define NF_DTYPE_F32 0
#define NF_DTYPE_BF16 1
#define NF_DTYPE_F16 2

/* status codes */
#define NF_OK 0
#define NF_ERR_ARG (-1)       /* bad pointer / size / stride / alignment   */
#define NF_ERR_DTYPE (-2)     /* unsupported element type or combination  */
#define NF_ERR_WORKSPACE (-3) /* workspace too small                      */
#define NF_ERR_LAUNCH (-4)    /* hipLaunchKernel / hipGetLastError failed */

/* ABI version compiled into the library (NF_ABI_VERSION). */
int nf_abi_version(void);

/* Description of the last failure on the calling thread ("" if none). */
const char *nf_last_error(void);

/* ------------------------------------------------------------------------
 * SwiGLU: out = silu(a) * b, elementwise over n contiguous elements.
 * Replaces the `_swiglu_fwd` launch in nuvla_forge/kernels/swiglu.py:35-46
 * (called from _FusedSwiGLU.forward, swiglu.py:66-79).
 * fp32 math, one rounding at the store; a, b, out share `dtype`.
 * ---------------------------------------------------------------------- */
int nf_swiglu_fwd(const void *a, const void *b, void *out, int64_t n,
                  int dtype, void *stream);

/* SwiGLU backward, sigmoid recomputed from a:
 *   da = dout * b * s * (1 + a * (1 - s)),  db = dout * a * s,  s = sigmoid(a)
 * Replaces the `_swiglu_bwd` launch in nuvla_forge/kernels/swiglu.py:48-63
 * (called from _FusedSwiGLU.backward, swiglu.py:81-92). */
int nf_swiglu_bwd(const void *dout, const void *a, const void *b, void *da,
                  void *db, int64_t n, int dtype, void *stream);

/* ------------------------------------------------------------------------
 * Gate/up projection with the SwiGLU epilogue: one MFMA GEMM computing
 *   a = x W_gate^T,  b = x W_up^T,  act = silu(a) * b     (fp32 accumulate)
 * No kernel of the reference computes this: it replaces the two Linear calls
 * and the fused_swiglu call of SwiGLUMLP.forward
 * (nuvla_forge/model/dit.py:104-110), whose a and b round-trip HBM.
 * x [M, D] (row stride ldx), w_gate / w_up [H, D] (row strides ld_gate /
 * ld_up, the nn.Linear weight layout, used in place), a / b / act [M, H]
 * (row stride ldo).  a and b are written (rounded to bf16, for the
 * backward) only when both are non-null.  bf16 only (NF_ERR_DTYPE
 * otherwise); every operand and output under 2 GiB.
 * ---------------------------------------------------------------------- */
int nf_gemm_swiglu(const void *x, int64_t ldx, const void *w_gate,
                   int64_t ld_gate, const void *w_up, int64_t ld_up, void *a,
                   void *b, void *act, int64_t ldo, int64_t M, int64_t D,
                   int64_t H, int dtype, void *stream);

/* Bytes of workspace nf_gemm_swiglu_wgrad needs for this shape (the
 * token-contiguous copies of da, db and x plus the fp32 split-K slices). */
size_t nf_gemm_swiglu_wgrad_workspace(int64_t M, int64_t D, int64_t H);

/* Weight gradients of the gate/up projection, both in one launch:
 *   dw_gate = da^T x,   dw_up = db^T x          (fp32 accumulate, bf16 out)
 * No kernel of the reference computes this: it replaces the weight-gradient
 * GEMMs of the two Linears in SwiGLUMLP (nuvla_forge/model/dit.py:104-110)
 * that autograd runs in the backward.  da / db [M, H] (row stride ld_ab) are
 * the gradients at the gate and up outputs, x [M, D] (row stride ldx) the
 * projection input, dw_gate / dw_up [H, D] (row stride ldw) are overwritten.
 * The sum over the M tokens is split into slices added in a fixed order, so
 * the result is bit-identical run to run.  M == 0 zeroes the gradients.
 * bf16 only; every operand under 2 GiB; the workspace is 16-byte aligned. */
int nf_gemm_swiglu_wgrad(const void *da, const void *db, int64_t ld_ab,
                         const void *x, int64_t ldx, void *dw_gate,
                         void *dw_up, int64_t ldw, int64_t M, int64_t D,
                         int64_t H, int dtype, void *workspace,
                         size_t workspace_bytes, void *stream);

/* ------------------------------------------------------------------------
 * adaLN-Zero seam: gated residual add, RMSNorm, modulation.  Row m of the
 * [M, N] activations belongs to sample m / T (M = B * T).
 *   h   = x + gate[b] * y                                  (stored as dt_x)
 *   rstd= 1 / sqrt(mean(h*h) + eps)      (fp32, from the unrounded fp32 h)
 *   out = h * rstd * weight * (1 + scale[b]) + shift[b]   (stored as dt_x)
 * Replaces the `_adaln_rmsnorm_fwd` launch in
 * nuvla_forge/kernels/adaln_rmsnorm.py:61-95 (launched at :178-187).
 * h and out are contiguous [M, N]; rstd is fp32 [M].  x may differ in type
 * from y (dt_y); the conditioning tensors and weight carry their own types.
 * ---------------------------------------------------------------------- */
int nf_adaln_fwd(const void *x, int64_t ld_x, const void *y, int64_t ld_y,
                 const void *gate, int64_t ld_gate, const void *weight,
                 const void *scale, int64_t ld_scale, const void *shift,
                 int64_t ld_shift, void *h, void *out, float *rstd, int64_t M,
                 int64_t N, int64_t T, float eps, int dt_x, int dt_y,
                 int dt_gate, int dt_weight, int dt_scale, int dt_shift,
                 void *stream);

/* Bytes of fp32 workspace the backward pair below needs for this shape
 * (per-block partial rows of the M-axis reductions). */
size_t nf_adaln_bwd_workspace(int64_t M, int64_t N, int64_t T);

/* adaLN seam backward, row part.  h is recomputed in fp32 from x and y;
 * rstd is the forward's.  With dxhat = dout * weight * (1 + scale[b]) and
 * xhat = h * rstd:
 *   dh = dh_up + rstd * (dxhat - xhat * mean(dxhat * xhat))
 *   dx = dh                          (contiguous [M, N], dt_x)
 *   dy = dh * gate[b]                (contiguous [M, N], dt_y)
 * and, per block of rows of one sample, the partial column sums
 *   sum dout * xhat,  sum dout,  sum dh * y
 * written to `workspace` for nf_adaln_bwd_reduce.
 * Replaces the `_adaln_rmsnorm_bwd` kernel and its launch,
 * nuvla_forge/kernels/adaln_rmsnorm.py:97-162 and :207-229.
 * dh_up / dout are contiguous [M, N] of dt_x; either may be NULL (= zero). */
int nf_adaln_bwd(const void *dh_up, const void *dout, const void *x,
                 int64_t ld_x, const void *y, int64_t ld_y, const void *gate,
                 int64_t ld_gate, const void *weight, const void *scale,
                 int64_t ld_scale, const float *rstd, void *dx, void *dy,
                 void *workspace, size_t workspace_bytes, int64_t M, int64_t N,
                 int64_t T, int dt_x, int dt_y, int dt_gate, int dt_weight,
                 int dt_scale, void *stream);

/* adaLN seam backward, reductions over M of the partials nf_adaln_bwd left
 * in `workspace` (same shape arguments), in a fixed order with no atomics:
 *   dgate  = sum_t dh * y                ([B, N], dt_gate)
 *   dscale = weight * sum_t dout * xhat  ([B, N], dt_scale)
 *   dshift = sum_t dout                  ([B, N], dt_shift)
 *   dweight= sum_b (1 + scale[b]) * sum_t dout * xhat   ([N], dt_weight)
 * Replaces the partial `.sum` reductions and casts of
 * nuvla_forge/kernels/adaln_rmsnorm.py:231-234.  Outputs may each be NULL
 * (not computed).  Must follow nf_adaln_bwd on the same stream. */
int nf_adaln_bwd_reduce(void *workspace, size_t workspace_bytes,
                        const void *weight, const void *scale, int64_t ld_scale,
                        void *dgate, void *dweight, void *dscale, void *dshift,
                        int64_t M, int64_t N, int64_t T, int dt_gate,
                        int dt_weight, int dt_scale, int dt_shift,
                        void *stream);

/* Size of the static device buffer nf_adaln_bwd_noalloc keeps its partial
 * rows in (one per GPU, held until the process ends). */
#define NF_ADALN_SCRATCH_BYTES ((size_t)16 << 20)

/* The adaLN seam backward (nf_adaln_bwd, then nf_adaln_bwd_reduce, same
 * arguments and results) without a caller workspace and without allocating:
 * the partial rows live in a static device buffer of NF_ADALN_SCRATCH_BYTES
 * owned by the library, one per GPU.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Shapes
 * whose partial rows exceed the buffer (nf_adaln_bwd_workspace(M, N, T) >
 * NF_ADALN_SCRATCH_BYTES) return NF_ERR_WORKSPACE.  All calls on one GPU
 * share its buffer: calls that overlap in time on one GPU (other streams,
 * other threads) race and must be serialised by the caller.  Outputs may
 * each be NULL as in nf_adaln_bwd_reduce. */
int nf_adaln_bwd_noalloc(const void *dh_up, const void *dout, const void *x,
                         int64_t ld_x, const void *y, int64_t ld_y,
                         const void *gate, int64_t ld_gate, const void *weight,
                         const void *scale, int64_t ld_scale, const float *rstd,
                         void *dx, void *dy, void *dgate, void *dweight,
                         void *dscale, void *dshift, int64_t M, int64_t N,
                         int64_t T, int dt_x, int dt_y, int dt_gate,
                         int dt_weight, int dt_scale, int dt_shift,
                         void *stream);

/* ------------------------------------------------------------------------
 * Chunked cross entropy.
 *   logits = hidden @ weight^T          ([M, V]; a chunk of its rows at a
 *                                        time, all of it when one chunk
 *                                        covers every valid row)
 *   lse    = logsumexp_v logits         (fp32)
 *   n      = #(targets != ignore_index);  inv = 1 / max(n, 1)
 *   loss   = inv * sum_{valid m} (lse[m] - logits[m, t_m])   (fp32 scalar)
 *   dhidden= g * inv * (softmax - onehot) @ weight        ([M, D])
 *   dweight= g * inv * (softmax - onehot)^T @ hidden      ([V, D])
 * with g the loss's upstream gradient.  Ignored rows contribute no loss and
 * no gradient; an all-ignored batch gives loss 0 and zero gradients.
 * Targets outside [0, V) other than ignore_index are counted in
 * *bad_targets (device int32, may be NULL) and treated as ignored.
 * hidden [M, D] and weight [V, D] are contiguous and share `dtype`
 * (NF_DTYPE_BF16 uses bf16 MFMA with fp32 accumulation, NF_DTYPE_F32 uses
 * fp32 MFMA).  targets is int64 [M].
 *
 * Only valid rows do work: the forward compacts them on the device (the
 * count never reaches the host) and forms each row's logits once, so the
 * products execute 6 * n * V * D flops (logits, dhidden, dweight).
 *
 * nf_ce_fwd computes the loss and fills `state` (nf_ce_state_bytes, 16-byte
 * aligned), which the caller keeps for nf_ce_bwd; `workspace`
 * (nf_ce_fwd_workspace) is scratch for the call.  The valid rows are taken
 * a chunk at a time: a chunk's logits are held as exp(logit - the row's
 * target logit) in the input type, with the target entry carrying the
 * one-hot term and a per-row fp32 factor making them (softmax - onehot) *
 * inv; results do not depend on chunk_rows beyond fp rounding.  bf16 keeps
 * a chunk's logits and the fp32 dweight accumulator together within the
 * bytes the reference's row chunks hold for them (an fp32 [chunk_rows, V]
 * tile and an fp32 [V, D] accumulator, up to 256-row rounding): one chunk
 * over every row with no accumulator where that fits (logits held in both
 * layouts the products read for D >= 2048 when those fit, otherwise once,
 * row-major, the dweight product reading them transposed), else chunks of
 * 2 * chunk_rows rows held once beside the accumulator.  fp32 holds chunks
 * of chunk_rows rows (rounded up to 256) in both layouts.
 * The forward also runs the gradient products of every chunk but the last
 * (into fp32 accumulators in `state`).  Replaces _ChunkedCrossEntropy.forward
 * and the `_ce_fwd_bwd` kernel, nuvla_forge/kernels/chunked_ce.py:49-98 and
 * :120-172.
 *
 * nf_ce_bwd runs the last chunk's products and writes the gradients already
 * multiplied by grad_output (a device fp32 scalar, NULL: 1), in dt_hidden
 * and dt_weight (fp32, bf16 or fp16: the callers' types).  Replaces
 * _ChunkedCrossEntropy.backward's scaling and casts, chunked_ce.py:174-182.
 * The same M, D, V, chunk_rows and dtype as the forward.
 * ---------------------------------------------------------------------- */
size_t nf_ce_state_bytes(int64_t M, int64_t D, int64_t V, int64_t chunk_rows,
                         int dtype);
size_t nf_ce_fwd_workspace(int64_t M, int64_t D, int64_t V,
                           int64_t chunk_rows, int dtype);
int nf_ce_fwd(const void *hidden, const void *weight, const int64_t *targets,
              int64_t M, int64_t D, int64_t V, int64_t ignore_index,
              int64_t chunk_rows, int dtype, float *loss, int32_t *bad_targets,
              void *state, size_t state_bytes, void *workspace,
              size_t workspace_bytes, void *stream);
size_t nf_ce_bwd_workspace(int64_t M, int64_t D, int64_t V,
                           int64_t chunk_rows, int dtype);
int nf_ce_bwd(int64_t M, int64_t D, int64_t V, int64_t chunk_rows, int dtype,
              void *state, size_t state_bytes, const float *grad_output,
              void *dhidden, int dt_hidden, void *dweight, int dt_weight,
              void *workspace, size_t workspace_bytes, void *stream);

/* Both in one call, the reference's structure (_ce_fwd_bwd,
 * chunked_ce.py:49-98): loss and the unscaled fp32 gradients.  `workspace`
 * (nf_ce_workspace) holds the state and the scratch of both halves. */
size_t nf_ce_workspace(int64_t M, int64_t D, int64_t V, int64_t chunk_rows,
                       int dtype);
int nf_ce_fwd_bwd(const void *hidden, const void *weight,
                  const int64_t *targets, int64_t M, int64_t D, int64_t V,
                  int64_t ignore_index, int64_t chunk_rows, int dtype,
                  float *loss, float *dhidden, float *dweight,
                  int32_t *bad_targets, void *workspace,
                  size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NUVLA_FORGE_HIP_H */
