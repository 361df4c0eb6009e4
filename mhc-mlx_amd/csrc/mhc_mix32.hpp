// Post-combine (stream_mix_add) kernels for 16 < n <= 64 on MFMA (mix32.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhc {

struct Mix32Args {
  const void* x;
  const void* y;      // optional
  const void* g;      // backward: dout
  void* out;          // forward: out; backward: dx
  void* dy;           // backward, optional
  const float* M;
  const float* hpre;
  const float* hpost;
  float* part;        // backward: one partial row [S n*n | Yd n | pad] per workgroup
  int64_t T;
  int n;
  int C;
  int h_mode;
  int P;              // floats per partial row
};

// out = Mf X + p Y for 16 < n <= 64, C a multiple of 64, 16-byte aligned
// tensors; y and out fp32 or x's dtype.  Returns 1 when not covered.
int mix32_fwd(const Mix32Args& A, int x_dtype, int y_dtype, int out_dtype, hipStream_t s);

// dx = Mf^T G, dy = p G and at most gmax partial rows of the sums; same
// coverage, dout fp32 or x's dtype.  Returns 1 when not covered.
int mix32_bwd(const Mix32Args& A, int x_dtype, int y_dtype, int g_dtype, int64_t gmax, hipStream_t s,
              int64_t* num_partials);

}  // namespace mhc
