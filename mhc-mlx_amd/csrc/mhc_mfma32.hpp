// Kernels for 16 < n <= 32 on MFMA (mfma32.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhc {

struct Mf32Args {
  const void* x;
  const void* g;     // backward: dout
  void* out;         // forward: out; backward: dx
  float* inv_rms;    // forward, optional
  const float* M;
  const float* hpre;
  const float* hpost;
  const float* w;
  float* part;       // backward: one partial row per workgroup
  int64_t T;
  int64_t M_ts;
  int64_t h_ts;
  int n;
  int C;
  int Cp;
  int P;
  int h_mode;
  float eps;
  // forward with the Sinkhorn projection in the kernel (layer-wide, at most one token per CU): the raw
  // logits, the iteration count and M written by workgroup 0 (null: M is read from M)
  const float* hres;
  float* M_out;
  int iters;
  // backward with per-token parameters: the token's dM [n, n] and dh_pre, dh_post [n] (with the
  // activation chain in raw-logit mode)
  float* dM_tok;
  float* dpre_tok;
  float* dpost_tok;
};

// Forward (out = M x + p * rms_norm(a^T x) w) for 16 < n <= 32, 16-bit x,
// out fp32 or x's dtype, C a multiple of 128 up to 16384, layer-wide or
// per-token parameters.  Returns 1 when the shape is not covered.
int mf32_fused_fwd(const Mf32Args& A, int x_dtype, int out_dtype, hipStream_t s);

// The layer forward from raw parameters in one launch (A.hres, A.M_out, A.iters set; raw h, layer-wide,
// 16 < n <= 32, at most one token per CU): every workgroup projects the logits in its wave 0 (the block
// Sinkhorn, so M is bitwise that of mhc_sinkhorn_fwd) and workgroup 0 writes M.  Returns 1 when the
// shape is not covered.
int mf32_layer_fwd_single_launch(const Mf32Args& A, int x_dtype, int out_dtype, hipStream_t s);

// Backward partial-sums pass for 16 < n <= 32 with layer-wide parameters,
// 16-bit x and dout of one dtype, C a multiple of 128 up to 1024: dx, and one
// partial row [dw C | pad | dM n*n | dA n | dP n | pad] per workgroup (at
// most gmax workgroups).  With per-token parameters (16 < n <= 32, C a
// multiple of 128 up to 1024): dx, the token's dM, dh_pre, dh_post (A.dM_tok,
// A.dpre_tok, A.dpost_tok) and one partial row [dw C | pad] per workgroup.
// Returns 1 when the shape is not covered.
int mf32_fused_bwd(const Mf32Args& A, int x_dtype, int g_dtype, int64_t gmax, hipStream_t s,
                   int64_t* num_partials);

}  // namespace mhc
