// Fixed-order reduction of per-workgroup partial rows (first stage).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MHC_REDUCE_INLINE static __device__ __forceinline__

namespace mhc {

// part2[s][c] = sum over rows [s*rows, min(G, (s+1)*rows)) of part[row][c],
// four columns per thread; P is a multiple of 4 and rows are 16-byte aligned.
// Sixteen rows are loaded per step (enough loads in flight to cover HBM
// latency) into four accumulators combined as (a0 + a1) + (a2 + a3): the
// association is fixed by (G, rows) alone.
MHC_REDUCE_INLINE float4 f4add(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

static __global__ __launch_bounds__(256) void reduce_rows_kernel(const float* __restrict__ part,
                                                                 float* __restrict__ part2,
                                                                 int64_t G, int P, int rows) {
  const int c4 = blockIdx.x * blockDim.x + threadIdx.x;
  if (c4 * 4 >= P) return;
  const int64_t g0 = (int64_t)blockIdx.y * rows;
  const int64_t g1 = g0 + rows < G ? g0 + rows : G;
  const float* src = part + c4 * 4;
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 a0 = z, a1 = z, a2 = z, a3 = z;
  int64_t g = g0;
  for (; g + 16 <= g1; g += 16) {
    float4 r[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) r[k] = *reinterpret_cast<const float4*>(src + (g + k) * P);
#pragma unroll
    for (int k = 0; k < 16; k += 4) {
      a0 = f4add(a0, r[k]); a1 = f4add(a1, r[k + 1]); a2 = f4add(a2, r[k + 2]); a3 = f4add(a3, r[k + 3]);
    }
  }
  for (; g < g1; ++g) a0 = f4add(a0, *reinterpret_cast<const float4*>(src + g * P));
  *reinterpret_cast<float4*>(part2 + (int64_t)blockIdx.y * P + c4 * 4) = f4add(f4add(a0, a1), f4add(a2, a3));
}

}  // namespace mhc
