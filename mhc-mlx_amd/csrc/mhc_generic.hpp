// Runtime-n kernels for 16 < n <= 64 (generic.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhc {

struct GenArgs {
  const void* x;
  const void* y;
  const void* g;
  void* out;  // fused fwd: out; bwd: dx
  void* dy;
  const float* M;
  const float* hpre;
  const float* hpost;
  const float* w;
  float* inv_rms;
  float* part;
  float* scratch;  // bwd: 2*C floats per workgroup
  float* dM_tok;
  float* dpre_tok;
  float* dpost_tok;
  int64_t T;
  int64_t M_ts;
  int64_t h_ts;
  int n;
  int C;
  int Cp;
  int P;
  int h_mode;
  float eps;
};

int64_t gen_grid(int64_t T);
int gen_fused_fwd(const GenArgs& A, int x_dtype, int out_dtype, hipStream_t s);
int gen_fused_bwd(const GenArgs& A, int x_dtype, int g_dtype, hipStream_t s, int64_t* num_partials);
int gen_mix_fwd(const GenArgs& A, int x_dtype, int y_dtype, int out_dtype, hipStream_t s);
int gen_mix_bwd(const GenArgs& A, int x_dtype, int y_dtype, int g_dtype, hipStream_t s, int64_t blocks);

}  // namespace mhc
