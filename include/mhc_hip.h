/*
 * mhc_hip.h — C ABI of libmhc_hip.so, the MI355X (gfx950) kernels for the
 * fused mHC (manifold-constrained hyper-connection) layer of
 * svdrecbd/mhc-mlx.
 *
 * Conventions (all entry points):
 *   - Plain pointers to device memory, row-major and contiguous.
 *     x / out / dout / dx are [T, n, C] (T tokens, n streams, C channels);
 *     M is [n, n] (or [T, n, n] with M_token_stride = n*n);
 *     h_pre / h_post are [n] (or [T, n] with h_token_stride = n).
 *   - Element dtypes are MHC_DTYPE_*; parameters and their gradients are fp32.
 *   - `stream` is a hipStream_t (NULL = default stream).  Every call only
 *     enqueues work on that stream; nothing synchronises the host.
 *   - The library never allocates device memory.  Scratch space is passed in
 *     as `workspace` with a size from the matching *_workspace_bytes().
 *   - Return value: MHC_OK (0); MHC_ERR_INVALID_ARG (<0) for a rejected
 *     argument; a positive hipError_t for a HIP runtime failure.  The text of
 *     the last error on the calling thread is mhc_last_error().
 *   - n must be in [1, MHC_MAX_N] (the reference caps n at 64:
 *     mhc_mlx/metal.py:71, 827-834).
 *
 * Citations are into the reference (svdrecbd/mhc-mlx, package mhc_mlx).
 */
#ifndef MHC_HIP_H_
#define MHC_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MHC_ABI_VERSION 1

#define MHC_DTYPE_F32 0
#define MHC_DTYPE_BF16 1
#define MHC_DTYPE_F16 2

#define MHC_OK 0
#define MHC_ERR_INVALID_ARG (-1)

#define MHC_MAX_N 64

/* Parameter activation modes for h_pre / h_post arguments. */
#define MHC_H_NONE 0      /* ignored: treated as all ones (plain stream mix) */
#define MHC_H_ACTIVATED 1 /* already activated: a = h_pre, p = h_post */
#define MHC_H_RAW 2       /* raw logits: a = sigmoid(h_pre), p = 2*sigmoid(h_post)
                             (reference.py:51-55) */

int mhc_abi_version(void);
const char* mhc_last_error(void);

/* --------------------------------------------------------------------- */
/* Launch-shape knobs                                                      */
/* --------------------------------------------------------------------- */

/* The library picks its launch shapes itself; a few integer choices
 * (workgroups per CU of a grid, slabs per wave, columns per lane, ...) can be
 * overridden by name ("MHC_RES_GRID", "MHC_BWD_GRID", ...).  Every knob
 * starts from the environment variable of the same name, read once when the
 * library is loaded; afterwards only these calls change it.  The table is
 * process-wide and its entries are atomics: a change made on one thread
 * applies to launches that start after it on any thread.  This is the
 * storage behind the reference's tuning file (metal.py:21-36: a JSON file of
 * per-kernel threadgroup sizes read at import); the Python package applies
 * such a file here.  Results never depend on a knob beyond fp32 rounding. */
int mhc_knob_count(void);
const char* mhc_knob_name(int index);                  /* NULL outside [0, count) */
int mhc_set_knob(const char* name, int value);         /* MHC_ERR_INVALID_ARG: unknown name */
int mhc_unset_knob(const char* name);                  /* back to the built-in choice */
int mhc_get_knob(const char* name, int* value);        /* 1: set (*value written), 0: unset */

/* --------------------------------------------------------------------- */
/* Sinkhorn-Knopp projection                                               */
/* --------------------------------------------------------------------- */

/* M[b] = sinkhorn_knopp(exp(logits[b] - rowmax(logits[b]))), b < batch.
 * logits, M: [batch, n, n] fp32.  Row step scale = (s > eps ? 1/s : 1),
 * column step scale = (s > eps ? 1/s : 0), `iters` row+column rounds.
 * Replaces sinkhorn_knopp_metal (metal.py:1525-1577) and the math of
 * mixing_matrix_from_logits / sinkhorn_knopp (reference.py:20-48, 58-69);
 * batch > 1 is the per-token extension. */
int mhc_sinkhorn_fwd(const float* logits, float* M, int64_t batch, int n, int iters,
                     float eps, void* stream);

/* Bytes of workspace mhc_sinkhorn_bwd needs (0 when the per-iteration state
 * fits in LDS). */
size_t mhc_sinkhorn_bwd_workspace_bytes(int64_t batch, int n, int iters);

/* dlogits = VJP of mhc_sinkhorn_fwd at logits for cotangent dM (all
 * [batch, n, n] fp32), through all `iters` iterations.
 * Replaces sinkhorn_knopp_backward_metal (metal.py:1978-2016) and the
 * Sinkhorn VJP of _sinkhorn_autograd_fn (metal.py:2724-2739). */
int mhc_sinkhorn_bwd(const float* logits, const float* dM, float* dlogits, int64_t batch,
                     int n, int iters, float eps, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Recorded state: the forward keeps what the VJP would otherwise recompute
 * (per iteration the cumulative row/column scales and the row/column sums
 * or scales: 256 bytes per matrix at n = 16, 6 * next_pow2(n) * 4 bytes for
 * 16 < n <= 64).  This splits _sinkhorn_autograd_fn's forward and VJP
 * (metal.py:2712-2758) the way an autograd function saves tensors for
 * backward; the results are those of mhc_sinkhorn_fwd / mhc_sinkhorn_bwd.
 *
 * Bytes of the state buffer for this shape; 0 when no recorded path exists
 * (n < 16, or the knob MHC_SK16 or MHC_SK16_RECORD is 0 at n = 16, or
 * MHC_SK_BLK_RECORD is 0 for 16 < n <= 64): then use mhc_sinkhorn_fwd /
 * mhc_sinkhorn_bwd. */
size_t mhc_sinkhorn_state_bytes(int64_t batch, int n, int iters);

/* mhc_sinkhorn_fwd that also writes the state to `state` (state_bytes >=
 * mhc_sinkhorn_state_bytes; at n = 16 logits and M 16-byte aligned). */
int mhc_sinkhorn_fwd_record(const float* logits, float* M, void* state, size_t state_bytes,
                            int64_t batch, int n, int iters, float eps, void* stream);

/* mhc_sinkhorn_bwd from the state mhc_sinkhorn_fwd_record wrote for the same
 * logits, iters and eps (no forward recompute, no workspace).  dM may alias
 * dlogits. */
int mhc_sinkhorn_bwd_recorded(const float* logits, const float* dM, float* dlogits,
                              const void* state, size_t state_bytes, int64_t batch, int n,
                              int iters, float eps, void* stream);

/* --------------------------------------------------------------------- */
/* Fused mHC forward: aggregate + RMSNorm + stream mix + H_post add         */
/* --------------------------------------------------------------------- */

/* out[t,i,c] = sum_j M[i,j] x[t,j,c] + p_i * (y[t,c] * inv[t]) * w[c]
 *   y[t,c] = sum_i a_i x[t,i,c],  inv[t] = 1/sqrt(mean_c y^2 + eps)
 * h_mode is MHC_H_ACTIVATED or MHC_H_RAW.  M_token_stride / h_token_stride
 * are 0 for layer-wide parameters or n*n / n for per-token parameters.
 * inv_rms ([T] fp32) is optional (NULL to skip).
 * Replaces mhc_forward_fused_metal (metal.py:1823-1975) — the agg / rms
 * reduce / mix+add launches (#4, #5, #6, #7, #3 of the reference). */
int mhc_fused_fwd(const void* x, int x_dtype, const float* M, int64_t M_token_stride,
                  const float* h_pre, const float* h_post, int64_t h_token_stride, int h_mode,
                  const float* rms_weight, void* out, int out_dtype, float* inv_rms, int64_t T,
                  int n, int C, float eps, void* stream);

/* Workspace for the fused backward (parameter-gradient partials). */
size_t mhc_fused_bwd_workspace_bytes(int64_t T, int n, int C, int per_token);

/* First stage of the fused backward: dx for every token and one row of
 * parameter-gradient partials per workgroup (deterministic, no atomics).
 * Per-token mode (M_token_stride != 0) also writes dM_tok [T,n,n],
 * dh_pre_tok [T,n], dh_post_tok [T,n] (gradients w.r.t. the raw logits when
 * h_mode == MHC_H_RAW, else w.r.t. the activated values).
 * *num_partials receives the number of partial rows written, to be passed
 * to mhc_reduce_param_grads.
 * Replaces the VJP of _mhc_fused_autograd_fn (metal.py:2787-2857): kernels
 * prep_tile, rms_reduce, dx_col, dM, dH_pre, dH_post, d_rms_weight
 * (#19-#25 of the reference). */
int mhc_fused_bwd_partials(const void* x, int x_dtype, const void* dout, int dout_dtype,
                           const float* M, int64_t M_token_stride, const float* h_pre,
                           const float* h_post, int64_t h_token_stride, int h_mode,
                           const float* rms_weight, void* dx, int dx_dtype, float* dM_tok,
                           float* dh_pre_tok, float* dh_post_tok, void* workspace,
                           size_t workspace_bytes, int64_t T, int n, int C, float eps,
                           int64_t* num_partials, void* stream);

/* Second stage: fixed-order sum of the partial rows.  Writes d_rms_weight [C]
 * and, for layer-wide parameters, dM [n,n], dh_pre [n], dh_post [n]
 * (w.r.t. raw logits when h_mode == MHC_H_RAW, else w.r.t. the activated
 * values as metal.py:2857 returns them).  Per-token mode writes only
 * d_rms_weight (pass NULL for the others). */
int mhc_reduce_param_grads(const void* workspace, size_t workspace_bytes, int64_t num_partials,
                           int n, int C, int per_token, const float* h_pre, const float* h_post,
                           int h_mode, float* dM, float* dh_pre, float* dh_post,
                           float* d_rms_weight, void* stream);

/* Both stages in one call. */
int mhc_fused_bwd(const void* x, int x_dtype, const void* dout, int dout_dtype, const float* M,
                  int64_t M_token_stride, const float* h_pre, const float* h_post,
                  int64_t h_token_stride, int h_mode, const float* rms_weight, void* dx,
                  int dx_dtype, float* dM, float* dh_pre, float* dh_post, float* d_rms_weight,
                  void* workspace, size_t workspace_bytes, int64_t T, int n, int C, float eps,
                  void* stream);

/* --------------------------------------------------------------------- */
/* Whole layer from raw parameters (MHCLayer.__call__ and its VJP)         */
/* --------------------------------------------------------------------- */

/* Forward of MHCLayer (layer.py:383-407 with the reference.py:164-184
 * math): M_out = sinkhorn_knopp(exp(h_res_raw)) then the fused forward with
 * a = sigmoid(h_pre_raw), p = 2*sigmoid(h_post_raw).  Layer-wide parameters
 * ([n], [n], [n,n]; M_out [n,n]) or, with per_token != 0, per-token ones
 * ([T,n], [T,n], [T,n,n]; M_out [T,n,n]).  M_out is kept for mhc_layer_bwd.
 * Replaces sinkhorn_knopp_metal_autograd + activate_pre_post +
 * mhc_forward_fused_metal_autograd as called from layer.py:387-407. */
int mhc_layer_fwd(const void* x, int x_dtype, const float* h_pre_raw, const float* h_post_raw,
                  const float* h_res_raw, const float* rms_weight, void* out, int out_dtype,
                  float* M_out, int64_t T, int n, int C, int per_token, int iters, float eps,
                  void* stream);

size_t mhc_layer_bwd_workspace_bytes(int64_t T, int n, int C, int per_token, int iters);

/* VJP of mhc_layer_fwd for cotangent dout: dx (x's dtype) and the gradients
 * w.r.t. the raw parameters (same shapes as the parameters) and rms_weight
 * [C].  M is the M_out of the forward.  Layer-wide: one partial-sums pass
 * over x and dout, then one launch that reduces the partial rows in a fixed
 * order, applies the sigmoid chain and runs the Sinkhorn VJP through all
 * `iters` iterations.  Per token: the same, plus a batched Sinkhorn VJP.
 * Replaces the MLX autograd chain through _mhc_fused_autograd_fn._f_vjp
 * (metal.py:2787-2857), activate_pre_post (reference.py:51-55) and the
 * Sinkhorn VJP (metal.py:2724-2739). */
int mhc_layer_bwd(const void* x, int x_dtype, const void* dout, int dout_dtype,
                  const float* h_pre_raw, const float* h_post_raw, const float* h_res_raw,
                  const float* M, const float* rms_weight, void* dx, float* d_h_pre_raw,
                  float* d_h_post_raw, float* d_h_res_raw, float* d_rms_weight, void* workspace,
                  size_t workspace_bytes, int64_t T, int n, int C, int per_token, int iters,
                  float eps, void* stream);

/* mhc_layer_bwd without a workspace argument: the workspace is a fixed
 * device array inside the library (64 MiB per GPU, reserved on a GPU by the
 * first call there and held until the process ends), so this call allocates
 * nothing.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Shapes whose mhc_layer_bwd_workspace_bytes
 * exceed 64 MiB are rejected with MHC_ERR_INVALID_ARG (e.g. layer-wide n = 4,
 * C = 4096 needs about 35 MB on a 256-CU GPU; per-token n = 16 needs its
 * Sinkhorn VJP state too).  All calls on one GPU share its array: calls that
 * overlap on one GPU (different streams, or threads on different streams)
 * race; calls on one stream are ordered by it. */
int mhc_layer_bwd_noalloc(const void* x, int x_dtype, const void* dout, int dout_dtype,
                          const float* h_pre_raw, const float* h_post_raw, const float* h_res_raw,
                          const float* M, const float* rms_weight, void* dx, float* d_h_pre_raw,
                          float* d_h_post_raw, float* d_h_res_raw, float* d_rms_weight, int64_t T, int n,
                          int C, int per_token, int iters, float eps, void* stream);

/* Second stage of mhc_layer_bwd on its own: after mhc_fused_bwd_partials
 * (h_mode MHC_H_RAW, the first mhc_fused_bwd_workspace_bytes() bytes of this
 * workspace, per-token dM / dh written into d_h_res_raw / d_h_pre_raw /
 * d_h_post_raw), reduce the `num_partials` rows and run the Sinkhorn VJP.
 * Lets a caller time the partial-sums kernel separately. */
int mhc_layer_bwd_reduce(void* workspace, size_t workspace_bytes, int64_t num_partials,
                         const float* h_pre_raw, const float* h_post_raw, const float* h_res_raw,
                         float* d_h_pre_raw, float* d_h_post_raw, float* d_h_res_raw,
                         float* d_rms_weight, int64_t T, int n, int C, int per_token, int iters,
                         float eps, void* stream);

/* --------------------------------------------------------------------- */
/* Stream mix + add (MHCRewire post-combine)                              */
/* --------------------------------------------------------------------- */

/* out[t,i,c] = p_i * (y[t,i,c] + sum_j M[i,j] a_j x[t,j,c])
 * h_mode MHC_H_NONE gives a = p = 1: out = M x + y, i.e.
 * stream_mix_add_metal (metal.py:954-1014, kernel #17).  MHC_H_RAW gives
 * MHCLayer.post_combine (layer.py:302-337).  y may be NULL (treated as 0). */
int mhc_stream_mix_add_fwd(const void* x, int x_dtype, const void* y, int y_dtype,
                           const float* M, const float* h_pre, const float* h_post, int h_mode,
                           void* out, int out_dtype, int64_t T, int n, int C, void* stream);

size_t mhc_stream_mix_add_bwd_workspace_bytes(int64_t T, int n, int C);

/* VJP of mhc_stream_mix_add_fwd for cotangent dout:
 *   dx_j = a_j sum_i M_ij p_i g_i       dy_i = p_i g_i   (dy may be NULL)
 *   S_ij = sum_{t,c} g_i x_j            Yd_i = sum g_i y_i
 *   h_mode NONE:      dM = S                                (metal.py:2672-2690)
 *   h_mode ACTIVATED: dM_ij = p_i S_ij a_j, dh_pre_j = sum_i p_i M_ij S_ij,
 *                     dh_post_i = sum_j M_ij a_j S_ij + Yd_i
 *   h_mode RAW:       the same chained through the activations. */
int mhc_stream_mix_add_bwd(const void* x, int x_dtype, const void* y, int y_dtype,
                           const void* dout, int dout_dtype, const float* M, const float* h_pre,
                           const float* h_post, int h_mode, void* dx, int dx_dtype, void* dy,
                           int dy_dtype, float* dM, float* dh_pre, float* dh_post,
                           void* workspace, size_t workspace_bytes, int64_t T, int n, int C,
                           void* stream);

/* MHCRewire pre-scale (layer.py:476-480): out[t,i,c] = a_i x[t,i,c]. */
int mhc_stream_scale_fwd(const void* x, int x_dtype, const float* h_pre, int h_mode, void* out,
                         int out_dtype, int64_t T, int n, int C, void* stream);

size_t mhc_stream_scale_bwd_workspace_bytes(int64_t T, int n, int C);

/* VJP of mhc_stream_scale_fwd: dx = a_i g (+ dx_accum if not NULL, same
 * dtype as dx, may alias dx) and dh_pre_i = sum g_i x_i (chained through the
 * sigmoid when h_mode == MHC_H_RAW). */
int mhc_stream_scale_bwd(const void* x, int x_dtype, const void* dout, int dout_dtype,
                         const float* h_pre, int h_mode, const void* dx_accum, void* dx,
                         int dx_dtype, float* dh_pre, void* workspace, size_t workspace_bytes,
                         int64_t T, int n, int C, void* stream);

/* --------------------------------------------------------------------- */
/* Residual add + stream aggregate                                         */
/* --------------------------------------------------------------------- */

/* out[t,i,c] = x[t,i,c] + res[t,i,c];  y_agg[t,c] = sum_i a_i (x + res)[t,i,c]
 * with the sum taken in fp32 before out is rounded to out_dtype.
 * x and res share `dtype`; y_agg is [T, C] fp32.  h_mode MHC_H_ACTIVATED
 * (a = h_pre, as the reference passes it) or MHC_H_RAW (a = sigmoid(h_pre)).
 * Replaces residual_add_agg_metal (metal.py:1673-1731; kernel
 * residual_add_agg.metal:39-66) behind residual_add_agg (utils.py:4-24). */
int mhc_residual_add_agg_fwd(const void* x, const void* res, int dtype, const float* h_pre,
                             int h_mode, void* out, int out_dtype, float* y_agg, int64_t T, int n,
                             int C, void* stream);

size_t mhc_residual_add_agg_bwd_workspace_bytes(int64_t T, int n, int C);

/* VJP of mhc_residual_add_agg_fwd for cotangents dout ([T,n,C], fp32 or
 * `dtype`; NULL = 0) and dy_agg ([T,C] fp32; NULL = 0):
 *   dx = dres = dout_i + a_i dy_agg     (each written if not NULL, in `dtype`)
 *   dh_pre_i = sum_{t,c} dy_agg (x + res)_i  (chained through the sigmoid for
 *   MHC_H_RAW; skipped if dh_pre is NULL, which needs no workspace).
 * The reference kernel has no VJP (an mx.fast.metal_kernel without a
 * custom_function); this is the gradient of the math it computes. */
int mhc_residual_add_agg_bwd(const void* x, const void* res, int dtype, const void* dout,
                             int dout_dtype, const float* dy_agg, const float* h_pre, int h_mode,
                             void* dx, void* dres, float* dh_pre, void* workspace,
                             size_t workspace_bytes, int64_t T, int n, int C, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MHC_HIP_H_ */
