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

// out[c] = sum over g < G of part[g][c] for c < C, in one launch (the per-token
// backward's d_w, where the parameter sums need no second stage).  A
// workgroup takes kColSumCols four-column groups and splits the rows over
// kColSumPhases phases (rows phase, phase + kColSumPhases, ...): a thread adds
// its rows eight loads at a time into four accumulators, and the phases are
// added in phase order through LDS.  The association depends on G alone.
constexpr int kColSumCols = 4;
constexpr int kColSumPhases = 64;

static __global__ __launch_bounds__(kColSumCols* kColSumPhases) void col_sum_kernel(const float* __restrict__ part,
                                                                                   int64_t G, int P, int C,
                                                                                   float* __restrict__ out) {
  __shared__ float4 s_part[kColSumPhases][kColSumCols];
  const int col4 = threadIdx.x % kColSumCols;
  const int phase = threadIdx.x / kColSumCols;
  const int c = (blockIdx.x * kColSumCols + col4) * 4;
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 a0 = z, a1 = z, a2 = z, a3 = z;
  if (c < P) {
    const float* src = part + c;
    constexpr int64_t ph = kColSumPhases;
    int64_t g = phase;
    for (; g + 7 * ph < G; g += 8 * ph) {
      float4 r[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) r[k] = *reinterpret_cast<const float4*>(src + (g + k * ph) * P);
      a0 = f4add(a0, f4add(r[0], r[4]));
      a1 = f4add(a1, f4add(r[1], r[5]));
      a2 = f4add(a2, f4add(r[2], r[6]));
      a3 = f4add(a3, f4add(r[3], r[7]));
    }
    for (; g < G; g += ph) a0 = f4add(a0, *reinterpret_cast<const float4*>(src + g * P));
  }
  s_part[phase][col4] = f4add(f4add(a0, a1), f4add(a2, a3));
  __syncthreads();
  if (phase == 0 && c < C) {
    float4 v = s_part[0][col4];
    for (int p = 1; p < kColSumPhases; ++p) v = f4add(v, s_part[p][col4]);
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c + e < C) out[c + e] = vv[e];
  }
}

}  // namespace mhc
