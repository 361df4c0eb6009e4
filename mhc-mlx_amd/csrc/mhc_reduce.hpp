// Fixed-order reduction of per-workgroup partial rows (first stage).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mhc {

// part2[s][c] = sum over rows [s*rows, min(G, (s+1)*rows)) of part[row][c],
// four columns per thread; P is a multiple of 4 and rows are 16-byte aligned.
static __global__ __launch_bounds__(256) void reduce_rows_kernel(const float* __restrict__ part,
                                                                 float* __restrict__ part2,
                                                                 int64_t G, int P, int rows) {
  const int c4 = blockIdx.x * blockDim.x + threadIdx.x;
  if (c4 * 4 >= P) return;
  const int64_t g0 = (int64_t)blockIdx.y * rows;
  const int64_t g1 = g0 + rows < G ? g0 + rows : G;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t g = g0; g < g1; ++g) {
    const float4 v = *reinterpret_cast<const float4*>(part + g * P + c4 * 4);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  *reinterpret_cast<float4*>(part2 + (int64_t)blockIdx.y * P + c4 * 4) = acc;
}

}  // namespace mhc
