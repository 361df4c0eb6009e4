// Batched Sinkhorn-Knopp projection and its VJP (one wavefront per group of
// matrices; see mhc_sinkhorn.hpp for the lane layout and the semantics of
// mhc_mlx/reference.py:20-48, 58-69 that they follow).
#include "mhc_device.hpp"
#include "mhc_host.hpp"
#include "mhc_plan.hpp"
#include "mhc_sinkhorn.hpp"

namespace mhc {

constexpr int kSkThreads = 256;
constexpr int kSkLdsBudget = 64 * 1024;

template <int NP>
__global__ __launch_bounds__(kSkThreads) void sinkhorn_fwd_kernel(const float* __restrict__ logits,
                                                                  float* __restrict__ out,
                                                                  int64_t batch, int n, int iters,
                                                                  float eps) {
  using L = SkLayout<NP>;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wpb = blockDim.x >> 6;
  const int msub = (lane % 64) / L::G;
  const int64_t ngroups = (batch + L::MPW - 1) / L::MPW;
  const int64_t nn = (int64_t)n * n;
  for (int64_t grp = (int64_t)blockIdx.x * wpb + wave; grp < ngroups;
       grp += (int64_t)gridDim.x * wpb) {
    const int64_t mat = grp * L::MPW + msub;
    const bool mvalid = mat < batch;
    const int64_t m = mvalid ? mat : 0;
    sk_fwd_group<NP>(logits + m * nn, out + m * nn, mvalid, n, iters, eps, lane);
  }
}

template <int NP, bool GLOBAL_STATE>
__global__ __launch_bounds__(kSkThreads) void sinkhorn_bwd_kernel(
    const float* __restrict__ logits, const float* __restrict__ dM, float* __restrict__ dlogits,
    int64_t batch, int n, int iters, float eps, float* __restrict__ gstate) {
  using L = SkLayout<NP>;
  extern __shared__ float sk_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wpb = blockDim.x >> 6;
  const int msub = lane / L::G;
  const int64_t ngroups = (batch + L::MPW - 1) / L::MPW;
  const int64_t nn = (int64_t)n * n;
  const int64_t per_wave = (int64_t)4 * iters * L::W;
  float* st;
  if constexpr (GLOBAL_STATE) {
    st = gstate + ((int64_t)blockIdx.x * wpb + wave) * per_wave;
  } else {
    st = sk_smem + (int64_t)wave * per_wave;
  }
  for (int64_t grp = (int64_t)blockIdx.x * wpb + wave; grp < ngroups;
       grp += (int64_t)gridDim.x * wpb) {
    const int64_t mat = grp * L::MPW + msub;
    const bool mvalid = mat < batch;
    const int64_t m = mvalid ? mat : 0;
    if constexpr (SkLayout<NP>::E == 1) {
      if (iters <= kSkRegIters) {
        sk_bwd_group_reg<NP, kSkRegIters>(logits + m * nn, dM + m * nn, dlogits + m * nn, mvalid, n, iters, eps,
                                          lane);
        continue;
      }
    }
    sk_bwd_group<NP>(logits + m * nn, dM + m * nn, dlogits + m * nn, mvalid, n, iters, eps, st, lane);
  }
}

// One matrix per wavefront in the block layout (mhc_sinkhorn.hpp), for
// 16 < n <= 64: a single layer-wide matrix is latency-bound, and this layout
// needs a third of the cross-lane steps per iteration.  With REC the forward
// also writes each matrix's VJP state to `rec` (sk_blk_state_floats per
// matrix, 16-byte aligned).
template <int NP, bool REC>
__global__ __launch_bounds__(kSkThreads) void sinkhorn_blk_fwd_kernel(const float* __restrict__ logits,
                                                                      float* __restrict__ out, int64_t batch,
                                                                      int n, int iters, float eps,
                                                                      float* __restrict__ rec) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wpb = blockDim.x >> 6;
  const int64_t nn = (int64_t)n * n;
  const int64_t per_matrix = sk_blk_state_floats(NP, iters);
  for (int64_t m = (int64_t)blockIdx.x * wpb + wave; m < batch; m += (int64_t)gridDim.x * wpb)
    sk_fwd_blk<NP, REC>(logits + m * nn, out + m * nn, n, iters, eps, lane, REC ? rec + m * per_matrix : nullptr);
}

// ---------------------------------------------------------------------------
// One 32 < n <= 64 matrix per workgroup of 8 / R waves (R = 2: four waves
// for few matrices, whose projection is latency-bound; R = 4: two waves for
// many, where the instruction count per matrix matters): one wave per matrix
// runs every instruction of an iteration's dependent chain itself, W waves a
// W-th of them.  Wave w holds rows 8 R w .. 8 R w + 8 R - 1; lane (rq = lane
// / 8, cq = lane % 8) rows 8 R w + R rq .. + R - 1, columns 8 cq .. 8 cq + 7.  Row
// sums stay in the wave (the 8 lanes of a row, DPP); a column sum adds the
// wave's lanes of the column (stride 8), then the four waves' partials from
// LDS in wave order: one barrier per iteration, the partials double-buffered
// by the iteration's parity.  The VJP state has the block layout's format
// (sk_blk_state_floats(64, iters) floats per matrix: row vectors by the row's
// lane cq = 0, column vectors by wave 0's lanes rq = 0), so a record from
// this forward serves this VJP; the values differ from the one-wave kernel's
// in summation order, so forward and VJP choose the same kernel family.
// ---------------------------------------------------------------------------
constexpr int kSkWgMaxStateBytes = 48 * 1024;  // the recomputing VJP's state in LDS: up to 32 iterations

struct SkWgLane {
  int lane, w, rq, cq, r0, c0;
};

// R rows per lane: 8 / R waves of 8 R rows each.
template <int R>
MHC_DEV SkWgLane sk_wg_lane() {
  SkWgLane L;
  L.lane = threadIdx.x & 63;
  L.w = threadIdx.x >> 6;
  L.rq = L.lane >> 3;
  L.cq = L.lane & 7;
  L.r0 = 8 * R * L.w + R * L.rq;
  L.c0 = 8 * L.cq;
  return L;
}

// cs: the lane's partial sums of its 8 columns over its two rows -> the column sums over every row.
template <int W>
MHC_DEV void sk_wg_colsum(float (&cs)[8], float (*s_cs)[W][64], int par, const SkWgLane& L) {
#pragma unroll
  for (int b = 0; b < 8; ++b) cs[b] = strided_sum<8, 64>(cs[b]);
  if (L.rq == 0) {
    float4* d = reinterpret_cast<float4*>(&s_cs[par][L.w][L.c0]);
    d[0] = make_float4(cs[0], cs[1], cs[2], cs[3]);
    d[1] = make_float4(cs[4], cs[5], cs[6], cs[7]);
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < 8; ++b) cs[b] = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float4* src = reinterpret_cast<const float4*>(&s_cs[par][w][L.c0]);
    const float4 u = src[0], v = src[1];
    cs[0] += u.x; cs[1] += u.y; cs[2] += u.z; cs[3] += u.w;
    cs[4] += v.x; cs[5] += v.y; cs[6] += v.z; cs[7] += v.w;
  }
}

// exp(H - rowmax) of the lane's 2 x 8 block (0 outside the matrix) and the row-maximum ties (bit 8a + b).
template <int R>
MHC_DEV uint32_t sk_wg_load_exp(const float* __restrict__ H, int n, const SkWgLane& L, float (&K)[R][8]) {
  uint32_t tie = 0;
#pragma unroll
  for (int a = 0; a < R; ++a) {
    float hv[8];
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool v = L.r0 + a < n && L.c0 + b < n;
      const float h = H[v ? (L.r0 + a) * n + L.c0 + b : 0];
      hv[b] = v ? h : -INFINITY;
      mx = fmaxf(mx, hv[b]);
    }
    mx = group_max<8>(mx);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool v = L.r0 + a < n && L.c0 + b < n;
      K[a][b] = v ? expf(hv[b] - mx) : 0.0f;
      if (v && hv[b] == mx) tie |= 1u << (8 * a + b);
    }
  }
  return tie;
}

// `iters` iterations on the lane's block P (the block layout's arithmetic per element: row step, then
// column step, masks and state as sk_blk_iterate); par counts the workgroup's column-sum rounds.
template <int R, bool REC>
MHC_DEV void sk_wg_iterate(float (&P)[R][8], int n, int iters, float eps, const SkWgLane& L,
                           float (*s_cs)[8 / R][64], int& par, float* st) {
  float Rc[R], Cc[8];
#pragma unroll
  for (int a = 0; a < R; ++a) Rc[a] = 1.0f;
#pragma unroll
  for (int b = 0; b < 8; ++b) Cc[b] = 1.0f;
  for (int it = 0; it < iters; ++it) {
    float rsc[R], rf[R];
#pragma unroll
    for (int a = 0; a < R; ++a) {
      float s = P[a][0];
#pragma unroll
      for (int b = 1; b < 8; ++b) s += P[a][b];
      s = group_sum<8>(s);
      const bool ok = L.r0 + a < n && s > eps;
      rsc[a] = ok ? sk_rcp(s) : 1.0f;
#pragma unroll
      for (int b = 0; b < 8; ++b) P[a][b] *= rsc[a];
      if (REC) {
        rf[a] = ok ? Rc[a] * rsc[a] * rsc[a] : 0.0f;
        Rc[a] *= rsc[a];
      }
    }
    float cs[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      cs[b] = P[0][b];
#pragma unroll
      for (int a = 1; a < R; ++a) cs[b] += P[a][b];
    }
    sk_wg_colsum<8 / R>(cs, s_cs, par, L);
    par ^= 1;
    float csc[8], cf[8], Cp[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bool ok = L.c0 + b < n && cs[b] > eps;
      csc[b] = ok ? sk_rcp(cs[b]) : 0.0f;
#pragma unroll
      for (int a = 0; a < R; ++a) P[a][b] *= csc[b];
      if (REC) {
        Cp[b] = Cc[b];
        cf[b] = ok ? Cc[b] * csc[b] * csc[b] : 0.0f;
        Cc[b] *= csc[b];
      }
    }
    if (REC) {
      float* sti = st + (int64_t)it * kSkBlkStateVecs * 64;
      if (L.cq == 0) {
#pragma unroll
        for (int a = 0; a < R; ++a) {
          sti[L.r0 + a] = Rc[a];
          sti[2 * 64 + L.r0 + a] = rsc[a];
          sti[3 * 64 + L.r0 + a] = rf[a];
        }
      }
      if (L.w == 0 && L.rq == 0) {
        sk_blk_st_store<8>(sti + 64 + L.c0, Cp);
        sk_blk_st_store<8>(sti + 4 * 64 + L.c0, csc);
        sk_blk_st_store<8>(sti + 5 * 64 + L.c0, cf);
      }
    }
  }
}

template <int R, bool REC>
__global__ __launch_bounds__(512 / R) void sinkhorn_wg_fwd_kernel(const float* __restrict__ logits,
                                                                          float* __restrict__ out, int64_t batch,
                                                                          int n, int iters, float eps,
                                                                          float* __restrict__ rec) {
  __shared__ __align__(16) float s_cs[2][8 / R][64];
  const SkWgLane L = sk_wg_lane<R>();
  const int64_t nn = (int64_t)n * n;
  const int64_t per_matrix = sk_blk_state_floats(64, iters);
  int par = 0;
  for (int64_t m = blockIdx.x; m < batch; m += gridDim.x) {
    float P[R][8];
    sk_wg_load_exp<R>(logits + m * nn, n, L, P);
    sk_wg_iterate<R, REC>(P, n, iters, eps, L, s_cs, par, REC ? rec + m * per_matrix : nullptr);
    float* o = out + m * nn;
#pragma unroll
    for (int a = 0; a < R; ++a)
#pragma unroll
      for (int b = 0; b < 8; ++b)
        if (L.r0 + a < n && L.c0 + b < n) o[(L.r0 + a) * n + L.c0 + b] = P[a][b];
  }
}

// VJP: RECORDED reads the forward's record where it lies; otherwise the iterations are recomputed into
// LDS first (at most kSkWgMaxStateBytes).  Reverse step k (column step, then row step):
//   Gd = csc Gd - cf * sum_rows(Gd K R_k),  Gd = rsc Gd - rf * sum_cols(Gd K C_k-1).
template <int R, bool RECORDED>
__global__ __launch_bounds__(512 / R) void sinkhorn_wg_bwd_kernel(const float* __restrict__ logits,
                                                                          const float* __restrict__ dM,
                                                                          float* __restrict__ dlogits,
                                                                          int64_t batch, int n, int iters,
                                                                          float eps, const float* __restrict__ rec) {
  extern __shared__ float4 sk_wg_smem4[];
  float* const s_st = reinterpret_cast<float*>(sk_wg_smem4);
  __shared__ __align__(16) float s_cs[2][8 / R][64];
  const SkWgLane L = sk_wg_lane<R>();
  const int64_t nn = (int64_t)n * n;
  const int64_t per_matrix = sk_blk_state_floats(64, iters);
  int par = 0;
  for (int64_t m = blockIdx.x; m < batch; m += gridDim.x) {
    float K[R][8], Gd[R][8];
    const uint32_t tie = sk_wg_load_exp<R>(logits + m * nn, n, L, K);
    const float* st;
    if constexpr (RECORDED) {
      st = rec + m * per_matrix;
    } else {
#pragma unroll
      for (int a = 0; a < R; ++a)
#pragma unroll
        for (int b = 0; b < 8; ++b) Gd[a][b] = K[a][b];
      sk_wg_iterate<R, true>(Gd, n, iters, eps, L, s_cs, par, s_st);
      __syncthreads();  // every lane's state entries before any lane reads them
      st = s_st;
    }
#pragma unroll
    for (int a = 0; a < R; ++a)
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const bool v = L.r0 + a < n && L.c0 + b < n;
        const float g = dM[m * nn + (v ? (L.r0 + a) * n + L.c0 + b : 0)];
        Gd[a][b] = v ? g : 0.0f;
      }
    for (int it = iters - 1; it >= 0; --it) {
      const float* sti = st + (int64_t)it * kSkBlkStateVecs * 64;
      float Rk[R], rsc[R], rf[R], Cp[8], csc[8], cf[8];
#pragma unroll
      for (int a = 0; a < R; ++a) {
        Rk[a] = sti[L.r0 + a];
        rsc[a] = sti[2 * 64 + L.r0 + a];
        rf[a] = sti[3 * 64 + L.r0 + a];
      }
      sk_blk_st_load<8>(sti + 64 + L.c0, Cp);
      sk_blk_st_load<8>(sti + 4 * 64 + L.c0, csc);
      sk_blk_st_load<8>(sti + 5 * 64 + L.c0, cf);
      float cs[8];
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        cs[b] = Gd[0][b] * K[0][b] * Rk[0];
#pragma unroll
        for (int a = 1; a < R; ++a) cs[b] += Gd[a][b] * K[a][b] * Rk[a];
      }
      sk_wg_colsum<8 / R>(cs, s_cs, par, L);
      par ^= 1;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const float sub = cs[b] * cf[b];
#pragma unroll
        for (int a = 0; a < R; ++a) Gd[a][b] = csc[b] * Gd[a][b] - sub;
      }
#pragma unroll
      for (int a = 0; a < R; ++a) {
        float dot = Gd[a][0] * (K[a][0] * Cp[0]);
#pragma unroll
        for (int b = 1; b < 8; ++b) dot += Gd[a][b] * (K[a][b] * Cp[b]);
        const float sub = group_sum<8>(dot) * rf[a];
#pragma unroll
        for (int b = 0; b < 8; ++b) Gd[a][b] = rsc[a] * Gd[a][b] - sub;
      }
    }
    // through exp and the row-max shift (the gradient of the max split evenly among tied maxima)
#pragma unroll
    for (int a = 0; a < R; ++a) {
      float tot = 0.0f, cnt = 0.0f;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        Gd[a][b] *= K[a][b];
        tot += Gd[a][b];
        cnt += (tie >> (8 * a + b)) & 1 ? 1.0f : 0.0f;
      }
      tot = group_sum<8>(tot);
      cnt = group_sum<8>(cnt);
      const float corr = cnt > 0.0f ? tot / cnt : 0.0f;
#pragma unroll
      for (int b = 0; b < 8; ++b)
        if (L.r0 + a < n && L.c0 + b < n)
          dlogits[m * nn + (L.r0 + a) * n + L.c0 + b] = Gd[a][b] - ((tie >> (8 * a + b)) & 1 ? corr : 0.0f);
    }
    if constexpr (!RECORDED) __syncthreads();  // the state is read before the next matrix writes over it
  }
}

// Where the block-layout VJP finds its state.
enum SkBlkState : int {
  kSkBlkLds = 0,        // recomputed into the wave's LDS
  kSkBlkWs = 1,         // recomputed into the wave's slice of the workspace
  kSkBlkRecLds = 2,     // recorded by the forward, copied to the wave's LDS first
  kSkBlkRecGlobal = 3,  // recorded by the forward, read where it lies
};

template <int NP, int STATE>
__global__ __launch_bounds__(kSkThreads) void sinkhorn_blk_bwd_kernel(
    const float* __restrict__ logits, const float* __restrict__ dM, float* __restrict__ dlogits, int64_t batch,
    int n, int iters, float eps, float* __restrict__ gstate) {
  extern __shared__ float4 sk_smem4[];
  float* sk_smem = reinterpret_cast<float*>(sk_smem4);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wpb = blockDim.x >> 6;
  const int64_t nn = (int64_t)n * n;
  const int64_t per_wave = sk_blk_state_floats(NP, iters);
  float* const lds = sk_smem + wave * per_wave;
  for (int64_t m = (int64_t)blockIdx.x * wpb + wave; m < batch; m += (int64_t)gridDim.x * wpb) {
    float* st;
    if constexpr (STATE == kSkBlkLds) {
      st = lds;
    } else if constexpr (STATE == kSkBlkWs) {
      st = gstate + ((int64_t)blockIdx.x * wpb + wave) * per_wave;
    } else if constexpr (STATE == kSkBlkRecLds) {
      // the matrix's record, 16 bytes per lane and step, read out before any
      // of it is written (no lane reads what another lane has yet to copy)
      const float4* src = reinterpret_cast<const float4*>(gstate + m * per_wave);
      float4* dst = reinterpret_cast<float4*>(lds);
      const int64_t n4 = per_wave / 4;
      for (int64_t i = lane; i < n4; i += 64) dst[i] = src[i];
      // every lane's LDS writes complete before any lane reads the state
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      __builtin_amdgcn_wave_barrier();
      st = lds;
    } else {
      st = gstate + m * per_wave;
    }
    sk_bwd_blk<NP, STATE == kSkBlkLds || STATE == kSkBlkWs>(logits + m * nn, dM + m * nn, dlogits + m * nn, n,
                                                            iters, eps, st, lane);
  }
}

// ---------------------------------------------------------------------------
// n == 16, batched (per-token mappings, config 3): four lanes per matrix.
//
// With CPL columns per lane (4 by default), lane (g = lane / LPM,
// p = lane % LPM), LPM = 16 / CPL, holds columns CPL*p .. CPL*p + CPL-1 of
// all 16 rows of matrix g (64 / LPM matrices per wave, one float4 / float2
// per row).  Column sums are in-lane (15 adds per column); row sums add the
// lane's columns and finish across the LPM lanes of the matrix with DPP
// permutes, so no iteration touches LDS.  With CPL = 4: ~200 VALU per
// iteration and lane for the row step and ~140 for the column step, i.e.
// ~21 per matrix, against ~75 plus 8 ds_bpermute per matrix for the
// one-matrix-per-wave layout.
//
// exp(H - rowmax) uses the hardware exp2 after scaling by log2 e (relative
// error ~|H - max| * 2^-24, far inside the fp32 tolerance).
//
// The VJP recomputes the forward and writes, per iteration, the cumulative
// row / column scales R_k, C_k and the row / column sums to a workspace
// (64 floats per matrix and iteration, [iters][R | rs | C | cs][16]); the
// reverse sweep reads them back.  The workspace of a wave is private to it
// and read shortly after being written, so it stays in the caches.
// ---------------------------------------------------------------------------

constexpr int kSk16Threads = 256;

MHC_DEV float sk16_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// CPL columns per lane: LPM = 16 / CPL lanes per matrix, 64 / LPM matrices per wave.
template <int CPL>
struct Sk16 {
  static constexpr int LPM = 16 / CPL;
  static constexpr int MPW = 64 / LPM;
  static constexpr int RPL = 16 / LPM;  // rows of the row vectors recorded per lane
};

template <int CPL>
MHC_DEV void sk16_lds(const float* __restrict__ src, float (&v)[CPL]) {
  if constexpr (CPL == 4) {
    const float4 f = *reinterpret_cast<const float4*>(src);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    const float2 f = *reinterpret_cast<const float2*>(src);
    v[0] = f.x; v[1] = f.y;
  }
}

template <int CPL>
MHC_DEV void sk16_st(float* __restrict__ dst, const float (&v)[CPL]) {
  if constexpr (CPL == 4) *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
  else *reinterpret_cast<float2*>(dst) = make_float2(v[0], v[1]);
}

// K = exp(H - rowmax) of the lane's CPL columns x 16 rows.
template <int CPL>
MHC_DEV void sk16_load_k(const float* __restrict__ Hm, bool mvalid, int p, float (&K)[16][CPL]) {
  constexpr int LPM = Sk16<CPL>::LPM;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (mvalid) sk16_lds<CPL>(Hm + i * 16 + CPL * p, K[i]);
    else {
#pragma unroll
      for (int e = 0; e < CPL; ++e) K[i][e] = -INFINITY;
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float mx = K[i][0];
#pragma unroll
    for (int e = 1; e < CPL; ++e) mx = fmaxf(mx, K[i][e]);
    mx = group_max<LPM>(mx);
#pragma unroll
    for (int e = 0; e < CPL; ++e) K[i][e] = mvalid ? sk16_exp(K[i][e] - mx) : 0.0f;
  }
}

// One row step and one column step on P, recording sums and scales through
// the callbacks (inlined).
template <int CPL, typename RowRec, typename ColRec>
MHC_DEV void sk16_iter(float (&P)[16][CPL], float eps, RowRec&& row_rec, ColRec&& col_rec) {
  constexpr int LPM = Sk16<CPL>::LPM;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float s = P[i][0];
#pragma unroll
    for (int e = 1; e < CPL; ++e) s += P[i][e];
    s = group_sum<LPM>(s);
    const float rsc = s > eps ? sk_rcp(s) : 1.0f;
#pragma unroll
    for (int e = 0; e < CPL; ++e) P[i][e] *= rsc;
    row_rec(i, s, rsc);
  }
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    float cs = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) cs += P[i][e];
    const float csc = cs > eps ? sk_rcp(cs) : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) P[i][e] *= csc;
    col_rec(e, cs, csc);
  }
}

template <int CPL>
MHC_DEV int64_t sk16_matrix(int& p) {
  constexpr int LPM = Sk16<CPL>::LPM;
  const int lane = threadIdx.x & 63;
  p = lane % LPM;
  return ((int64_t)blockIdx.x * (kSk16Threads / 64) + (threadIdx.x >> 6)) * Sk16<CPL>::MPW + lane / LPM;
}

// The forward iterations on P, recording per iteration k the cumulative row
// scales R_k and row sums rs_k (rows RPL*p ..) and the cumulative column
// scales C_k and column sums cs_k (columns CPL*p ..) at sm + 64 k (when
// mvalid).  P ends as M, bitwise the same as without recording.
template <int CPL>
MHC_DEV void sk16_forward_record(float (&P)[16][CPL], int iters, float eps, int p, bool mvalid, float* sm) {
  constexpr int LPM = Sk16<CPL>::LPM;
  constexpr int RPL = Sk16<CPL>::RPL;
  float R[16], Cc[CPL];
#pragma unroll
  for (int i = 0; i < 16; ++i) R[i] = 1.0f;
#pragma unroll
  for (int e = 0; e < CPL; ++e) Cc[e] = 1.0f;
  for (int it = 0; it < iters; ++it) {
    float rs[16], cs[CPL];
    sk16_iter<CPL>(P, eps,
                   [&](int i, float sum, float rsc) {
                     rs[i] = sum;
                     R[i] *= rsc;
                   },
                   [&](int e, float sum, float csc) {
                     cs[e] = sum;
                     Cc[e] *= csc;
                   });
    if (mvalid) {
      float* sk = sm + (int64_t)it * 64;
      float r4[RPL], s4[RPL];
#pragma unroll
      for (int k = 0; k < RPL; ++k) {
        float rv = R[k], sv = rs[k];
#pragma unroll
        for (int q = 1; q < LPM; ++q)
          if (p == q) {
            rv = R[RPL * q + k];
            sv = rs[RPL * q + k];
          }
        r4[k] = rv;
        s4[k] = sv;
      }
      sk16_st<RPL>(sk + RPL * p, r4);
      sk16_st<RPL>(sk + 16 + RPL * p, s4);
      sk16_st<CPL>(sk + 32 + CPL * p, Cc);
      sk16_st<CPL>(sk + 48 + CPL * p, cs);
    }
  }
}

template <int CPL>
__global__ __launch_bounds__(kSk16Threads) void sinkhorn16_fwd_kernel(const float* __restrict__ logits,
                                                                      float* __restrict__ out, int64_t batch,
                                                                      int iters, float eps) {
  int p;
  const int64_t m = sk16_matrix<CPL>(p);
  const bool mvalid = m < batch;
  float P[16][CPL];
  sk16_load_k<CPL>(logits + (mvalid ? m : 0) * 256, mvalid, p, P);
  for (int it = 0; it < iters; ++it)
    sk16_iter<CPL>(P, eps, [](int, float, float) {}, [](int, float, float) {});
  if (mvalid) {
    float* O = out + m * 256;
#pragma unroll
    for (int i = 0; i < 16; ++i) sk16_st<CPL>(O + i * 16 + CPL * p, P[i]);
  }
}

// st: the workspace, [batch][iters][4][16] floats (R_k, rs_k, C_k, cs_k),
// written by the forward recomputed here and read back by the reverse sweep.
// dM may alias dlogits.
template <int CPL>
__global__ __launch_bounds__(kSk16Threads) void sinkhorn16_bwd_kernel(const float* __restrict__ logits,
                                                                      const float* dM, float* dlogits,
                                                                      int64_t batch, int iters, float eps,
                                                                      float* __restrict__ st) {
  constexpr int LPM = Sk16<CPL>::LPM;
  int p;
  const int64_t m = sk16_matrix<CPL>(p);
  const bool mvalid = m < batch;
  const int64_t mm = mvalid ? m : 0;
  float K[16][CPL];
  sk16_load_k<CPL>(logits + mm * 256, mvalid, p, K);
  float* sm = st + mm * (int64_t)iters * 64;
  {
    float P[16][CPL];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int e = 0; e < CPL; ++e) P[i][e] = K[i][e];
    sk16_forward_record<CPL>(P, iters, eps, p, mvalid, sm);
    // the state written by the other lanes of the matrix is read below
    __builtin_amdgcn_s_waitcnt(0);
    __threadfence_block();
  }

  float G[16][CPL];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (mvalid) sk16_lds<CPL>(dM + mm * 256 + i * 16 + CPL * p, G[i]);
    else {
#pragma unroll
      for (int e = 0; e < CPL; ++e) G[i][e] = 0.0f;
    }
  }
  auto ld16 = [&](const float* src, float (&v)[16]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 f = *reinterpret_cast<const float4*>(src + 4 * k);
      v[4 * k] = f.x; v[4 * k + 1] = f.y; v[4 * k + 2] = f.z; v[4 * k + 3] = f.w;
    }
  };
  // Reverse sweep: iteration `it` reads R_it, rs_it, cs_it (own columns),
  // R_{it-1} and C_{it-1} (own columns).  Invalid matrices (past the batch)
  // never read the workspace.  The eps masks are selects, not branches.
  for (int it = iters - 1; it >= 0; --it) {
    float Rk[16], rs[16], Rp[16], csv[CPL], Cp[CPL];
    if (mvalid) {
      const float* sk = sm + (int64_t)it * 64;
      ld16(sk, Rk);
      ld16(sk + 16, rs);
      sk16_lds<CPL>(sk + 48 + CPL * p, csv);
      if (it > 0) {
        ld16(sk - 64, Rp);
        sk16_lds<CPL>(sk - 64 + 32 + CPL * p, Cp);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) Rp[i] = 1.0f;
#pragma unroll
        for (int e = 0; e < CPL; ++e) Cp[e] = 1.0f;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) Rk[i] = rs[i] = Rp[i] = 0.0f;
#pragma unroll
      for (int e = 0; e < CPL; ++e) csv[e] = 0.0f, Cp[e] = 1.0f;
    }
    // K C_{k-1}: both steps' inputs are R K C_{k-1}, R = R_k (column step) or R_{k-1} (row step)
    float KC[16][CPL];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int e = 0; e < CPL; ++e) KC[i][e] = K[i][e] * Cp[e];
    // column step (masked column: zero gradient)
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      float dot = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) dot = fmaf(G[i][e] * KC[i][e], Rk[i], dot);
      const bool on = csv[e] > eps;
      const float sc = on ? sk_rcp(csv[e]) : 0.0f;
      const float sc2 = sc * sc * dot;
#pragma unroll
      for (int i = 0; i < 16; ++i) G[i][e] = fmaf(sc, G[i][e], -sc2);
    }
    // row step (masked row: gradient passes unchanged)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float prod = 0.0f;
#pragma unroll
      for (int e = 0; e < CPL; ++e) prod = fmaf(G[i][e], KC[i][e], prod);
      const float dot = group_sum<LPM>(prod * Rp[i]);
      const bool on = rs[i] > eps;
      const float sc = on ? sk_rcp(rs[i]) : 1.0f;
      const float sc2 = on ? sc * sc * dot : 0.0f;
#pragma unroll
      for (int e = 0; e < CPL; ++e) G[i][e] = fmaf(sc, G[i][e], -sc2);
    }
  }
  // through exp and the row-max shift (the max's gradient split evenly among
  // tied maxima; zero in exact arithmetic)
  if (mvalid) {
    float* O = dlogits + mm * 256;
    const float* Hm = logits + mm * 256;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float hv[CPL];
      sk16_lds<CPL>(Hm + i * 16 + CPL * p, hv);
      float mx = hv[0];
#pragma unroll
      for (int e = 1; e < CPL; ++e) mx = fmaxf(mx, hv[e]);
      mx = group_max<LPM>(mx);
      float dsh[CPL], tot = 0.0f, cnt = 0.0f;
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        dsh[e] = G[i][e] * K[i][e];
        tot += dsh[e];
        cnt += hv[e] == mx ? 1.0f : 0.0f;
      }
      tot = group_sum<LPM>(tot);
      cnt = group_sum<LPM>(cnt);
      const float corr = cnt > 0.0f ? tot / cnt : 0.0f;
      float o[CPL];
#pragma unroll
      for (int e = 0; e < CPL; ++e) o[e] = dsh[e] - (hv[e] == mx ? corr : 0.0f);
      sk16_st<CPL>(O + i * 16 + CPL * p, o);
    }
  }
}

// ---------------------------------------------------------------------------
// n == 16, batched, block layout (the default for n == 16): one 16-lane DPP
// row per matrix, four matrices per wave, so a batch of B matrices fills
// B / 4 waves (four per SIMD at config 3's 16384 matrices, against one for the
// four-lanes-per-matrix kernels above).
//
// Lane l = 4 rb + cb of the matrix's row holds a 4 x 4 block, rotated:
// register [s][t] is element (4 rb + ((cb + s) & 3), 4 cb + ((rb + t) & 3)).
// Slot 0 is the lane's own row 4 rb + cb and own column 4 cb + rb; every row
// and column has exactly one owner, and the rotation makes every cross-lane
// step a uniform DPP read:
//  * the owner of a row adds the partial sums of its quad (quad lane cb + u
//    holds the row in slot (-u) & 3; quad_perm rotations), the owner of a
//    column those of lanes l + 4u (slot (-u) & 3 again; row_ror rotations):
//    three DPP adds per sum, computed once, by the owner;
//  * per-row and per-column scalars (scales, cumulative R and C) live on the
//    owner and are read back by the same rotations.
//
// The iterate is P_k = diag(R_k) K diag(C_k) (reference.py:35-46 scales P
// itself; the same products, associated differently): the row sums of
// P_{k-1} are R_{k-1} (K C_{k-1}) and the column sums after the row step are
// C_{k-1} (R_k K), so an iteration costs two FMAs per element and the matrix
// is formed once at the end.
//
// The recorded state (mhc_sinkhorn_fwd_record, always this layout at n = 16)
// is what the VJP cannot get cheaply: per iteration the row sums rs_k and
// column sums cs_k (32 floats), and at the start of every VJP segment but the
// first the cumulative scales R and C (32 floats), [iters][rs | cs][16] then
// [nseg - 1][R | C][16] per matrix.  The VJP rebuilds R_k and C_k inside a
// segment from its starting scales with the forward's own products
// (R_k = R_{k-1} rcp(rs_k) unless masked, likewise C_k), so they are
// bitwise the forward's: 128 bytes per iteration instead of the 256 of R_k,
// rs_k, C_k, cs_k.
//
// Without a record (MHC_SK16_RECORD=0, or the plain mhc_sinkhorn_bwd) the
// VJP keeps its per-iteration state (R_k, rs_k, C_k, cs_k of the lane's own
// row and column) in registers, kSk16bSeg iterations at a time.  The
// segments are aligned to the end (the first one is the short one); the
// forward runs once to the last segment's start, keeping each segment's
// starting scales in LDS, then each segment, last first, is recomputed into
// registers and swept in reverse: 2 iters - kSk16bSeg forward iterations in
// all (31 at 20 iterations) and no memory traffic beyond the matrices.  At
// 16384 matrices of 20 iterations the recorded pair (forward 19.9 us, VJP
// 32.5 us) still beats it (14.5 + 41.5 us), so the layer records by default.
// ---------------------------------------------------------------------------

constexpr int kSk16bThreads = 256;
constexpr int kSk16bSeg = 9;  // with 4 waves per SIMD (128 VGPRs), no spills
constexpr int kSk16bMaxSeg = 32;  // VJP checkpoints: 512 bytes of LDS per wave and segment
// The VJP from a record holds two segments' sums (the one swept and the next
// one's, loaded meanwhile) and the rebuilt scales: 5 iterations a segment keep
// that within 128 VGPRs (9 spilled).  The record's checkpoints follow it.
constexpr int kSk16bRecSeg = 5;

// Floats of recorded state per matrix: 32 per iteration, 32 per VJP segment
// after the first (at least 32, so that iters = 0 still has a record).
__host__ __device__ inline int64_t sk16b_rec_floats(int iters) {
  const int nseg = (iters + kSk16bRecSeg - 1) / kSk16bRecSeg;
  const int64_t k = (int64_t)iters + (nseg > 0 ? nseg - 1 : 0);
  return 32 * (k > 0 ? k : 1);
}

// A DPP read of another lane's v.  Every read here stays inside the lane's
// quad or 16-lane row, so no source lane is ever out of range: bound_ctrl on,
// and no "old" value for the compiler to materialise.
template <int CTRL>
MHC_DEV float sk16b_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                               __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// v of quad lane (c + U) & 3, c this lane's position in its quad
template <int U>
MHC_DEV float sk16b_quad(float v) {
  if constexpr ((U & 3) == 0) return v;
  else return sk16b_dpp<(U & 3) | (((U + 1) & 3) << 2) | (((U + 2) & 3) << 4) | (((U + 3) & 3) << 6)>(v);
}

// v of lane (l + 4 U) mod 16 of this lane's DPP row (row_ror:k reads lane (l - k) mod 16)
template <int U>
MHC_DEV float sk16b_col(float v) {
  if constexpr ((U & 3) == 0) return v;
  else return sk16b_dpp<0x120 + ((16 - 4 * U) & 15)>(v);
}

template <typename Op>
MHC_DEV float sk16b_row_own(const float (&p)[4], Op op) {
  return op(op(op(p[0], sk16b_quad<1>(p[3])), sk16b_quad<2>(p[2])), sk16b_quad<3>(p[1]));
}
template <typename Op>
MHC_DEV float sk16b_col_own(const float (&p)[4], Op op) {
  return op(op(op(p[0], sk16b_col<1>(p[3])), sk16b_col<2>(p[2])), sk16b_col<3>(p[1]));
}
MHC_DEV void sk16b_row_bcast(float v, float (&o)[4]) {
  o[0] = v;
  o[1] = sk16b_quad<1>(v);
  o[2] = sk16b_quad<2>(v);
  o[3] = sk16b_quad<3>(v);
}
MHC_DEV void sk16b_col_bcast(float v, float (&o)[4]) {
  o[0] = v;
  o[1] = sk16b_col<1>(v);
  o[2] = sk16b_col<2>(v);
  o[3] = sk16b_col<3>(v);
}

// The lane's block of a row-major 16 x 16 matrix: row slot s is one float4 of
// columns 4 cb .. 4 cb + 3, rotated left by rb into the column slots.
MHC_DEV void sk16b_load(const float* __restrict__ A, int rb, int cb, float (&E)[4][4]) {
  const bool b1 = (rb & 1) != 0, b2 = (rb & 2) != 0;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float4 f = *reinterpret_cast<const float4*>(A + (4 * rb + ((cb + s) & 3)) * 16 + 4 * cb);
    const float v[4] = {f.x, f.y, f.z, f.w};
    float a[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) a[t] = b1 ? v[(t + 1) & 3] : v[t];
#pragma unroll
    for (int t = 0; t < 4; ++t) E[s][t] = b2 ? a[(t + 2) & 3] : a[t];
  }
}

MHC_DEV void sk16b_store(float* A, int rb, int cb, const float (&E)[4][4]) {
  const bool b1 = (rb & 1) != 0, b2 = (rb & 2) != 0;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float a[4], v[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) a[x] = b2 ? E[s][(x + 2) & 3] : E[s][x];
#pragma unroll
    for (int x = 0; x < 4; ++x) v[x] = b1 ? a[(x + 3) & 3] : a[x];
    *reinterpret_cast<float4*>(A + (4 * rb + ((cb + s) & 3)) * 16 + 4 * cb) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// E <- exp(E - rowmax) (reference.py:67); mx: the row maxima of the lane's row slots
MHC_DEV void sk16b_exp(float (&E)[4][4], float (&mx)[4]) {
  float pm[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) pm[s] = fmaxf(fmaxf(E[s][0], E[s][1]), fmaxf(E[s][2], E[s][3]));
  sk16b_row_bcast(sk16b_row_own(pm, MaxOp{}), mx);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int t = 0; t < 4; ++t) E[s][t] = sk16_exp(E[s][t] - mx[s]);
}

struct Sk16bScales {
  float R, C;          // cumulative scale of the lane's own row / own column
  float Rs[4], Cs[4];  // ... of its row slots / column slots
};

MHC_DEV void sk16b_scales(Sk16bScales& S, float R, float C) {
  S.R = R;
  S.C = C;
  sk16b_row_bcast(R, S.Rs);
  sk16b_col_bcast(C, S.Cs);
}

// One iteration (row step, then column step, with the reference's eps masks);
// rs / cs: the sums of the lane's own row / column that the steps divided by.
MHC_DEV void sk16b_iter(const float (&K)[4][4], Sk16bScales& S, float eps, float& rs, float& cs) {
  float p[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float a = K[s][0] * S.Cs[0];
    a = fmaf(K[s][1], S.Cs[1], a);
    a = fmaf(K[s][2], S.Cs[2], a);
    p[s] = fmaf(K[s][3], S.Cs[3], a);
  }
  rs = S.R * sk16b_row_own(p, SumOp{});
  S.R *= rs > eps ? sk_rcp(rs) : 1.0f;
  sk16b_row_bcast(S.R, S.Rs);
  float q[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float a = S.Rs[0] * K[0][t];
    a = fmaf(S.Rs[1], K[1][t], a);
    a = fmaf(S.Rs[2], K[2][t], a);
    q[t] = fmaf(S.Rs[3], K[3][t], a);
  }
  cs = S.C * sk16b_col_own(q, SumOp{});
  S.C *= cs > eps ? sk_rcp(cs) : 0.0f;
  sk16b_col_bcast(S.C, S.Cs);
}

// Reverse of iteration k: G holds dL/dP_k on entry and dL/dP_{k-1} on exit.
// Rk, rs, cs: the lane's own-row R_k and sums of iteration k; Rp, Cp: its
// own-row R_{k-1} and own-column C_{k-1}.  For a step x -> s x with s = 1/sum:
// d_in = s g - s^2 <g, in> (the reference's autograd of reference.py:37-46);
// a masked column passes no gradient, a masked row passes it unchanged.
MHC_DEV void sk16b_vjp_step(float (&G)[4][4], const float (&K)[4][4], float Rk, float rs, float cs, float Rp,
                            float Cp, float eps) {
  float Rkb[4];
  sk16b_row_bcast(Rk, Rkb);
  // column step: its input is diag(R_k) K diag(C_{k-1}); the column's scale C_{k-1} factors out of
  // its dot product and is applied once, by the column's owner
  float d[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float a = (G[0][t] * K[0][t]) * Rkb[0];
#pragma unroll
    for (int s = 1; s < 4; ++s) a = fmaf(G[s][t] * K[s][t], Rkb[s], a);
    d[t] = a;
  }
  const float dot = Cp * sk16b_col_own(d, SumOp{});
  const float csc = cs > eps ? sk_rcp(cs) : 0.0f;
  float scb[4], s2b[4];
  sk16b_col_bcast(csc, scb);
  sk16b_col_bcast(csc * csc * dot, s2b);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int t = 0; t < 4; ++t) G[s][t] = fmaf(scb[t], G[s][t], -s2b[t]);
  // row step: its input is diag(R_{k-1}) K diag(C_{k-1})
  float Cpb[4];
  sk16b_col_bcast(Cp, Cpb);
  float e[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float a = G[s][0] * (K[s][0] * Cpb[0]);
    a = fmaf(G[s][1], K[s][1] * Cpb[1], a);
    a = fmaf(G[s][2], K[s][2] * Cpb[2], a);
    e[s] = fmaf(G[s][3], K[s][3] * Cpb[3], a);
  }
  const float rdot = Rp * sk16b_row_own(e, SumOp{});
  const bool on = rs > eps;
  const float rsc = on ? sk_rcp(rs) : 1.0f;
  float rsb[4], r2b[4];
  sk16b_row_bcast(rsc, rsb);
  sk16b_row_bcast(on ? rsc * rsc * rdot : 0.0f, r2b);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int t = 0; t < 4; ++t) G[s][t] = fmaf(rsb[s], G[s][t], -r2b[s]);
}

struct Sk16bLane {
  int rb, cb, ro, co;  // block coordinates; own row and own column
  int64_t m;           // matrix
  bool valid;          // m < batch (lanes past the batch work on matrix 0 and store nothing)
};

MHC_DEV Sk16bLane sk16b_lane(int64_t batch) {
  const int lane = threadIdx.x & 63;
  Sk16bLane L;
  L.rb = (lane >> 2) & 3;
  L.cb = lane & 3;
  L.ro = 4 * L.rb + L.cb;
  L.co = 4 * L.cb + L.rb;
  L.m = ((int64_t)blockIdx.x * (kSk16bThreads / 64) + (threadIdx.x >> 6)) * 4 + (lane >> 4);
  L.valid = L.m < batch;
  return L;
}

// REC: also record the VJP state at st (sk16b_rec_floats(iters) floats per
// matrix: the sums of every iteration, then the scales at the start of every
// VJP segment but the first).
template <bool REC>
__global__ __launch_bounds__(kSk16bThreads) void sinkhorn16b_fwd_kernel(const float* __restrict__ logits,
                                                                        float* __restrict__ out, int64_t batch,
                                                                        int iters, float eps,
                                                                        float* __restrict__ st) {
  const Sk16bLane L = sk16b_lane(batch);
  const int64_t mm = L.valid ? L.m : 0;
  float K[4][4], mx[4];
  sk16b_load(logits + mm * 256, L.rb, L.cb, K);
  sk16b_exp(K, mx);
  Sk16bScales S;
  sk16b_scales(S, 1.0f, 1.0f);
  float* rec = REC ? st + mm * sk16b_rec_floats(iters) : nullptr;
  // the VJP's segment sg >= 1 starts after iteration first + (sg - 1) kSk16bRecSeg - 1
  const int nseg = (iters + kSk16bRecSeg - 1) / kSk16bRecSeg;
  const int first = iters - (nseg - 1) * kSk16bRecSeg;
  int next_ck = first;  // completed iterations at the next checkpoint
  float* ck = REC ? rec + (int64_t)iters * 32 : nullptr;
  for (int it = 0; it < iters; ++it) {
    float rs, cs;
    sk16b_iter(K, S, eps, rs, cs);
    if constexpr (REC) {
      if (L.valid) {
        float* r = rec + (int64_t)it * 32;
        r[L.ro] = rs;
        r[16 + L.co] = cs;
        if (it + 1 == next_ck && it + 1 < iters) {
          ck[L.ro] = S.R;
          ck[16 + L.co] = S.C;
        }
      }
      if (it + 1 == next_ck && it + 1 < iters) {
        ck += 32;
        next_ck += kSk16bRecSeg;
      }
    }
  }
  if (L.valid) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) K[s][t] = (S.Rs[s] * K[s][t]) * S.Cs[t];
    sk16b_store(out + mm * 256, L.rb, L.cb, K);
  }
}

// RECORDED: st holds the forward's record for these logits (each segment's
// sums and starting scales are loaded while the segment before it in the
// sweep is processed); otherwise the iterations are recomputed (LDS:
// kSk16bThreads / 64 * nseg * 512 bytes).  dM may alias dlogits: each lane
// reads and writes only its own block.
template <bool RECORDED>
__global__ __launch_bounds__(kSk16bThreads) __attribute__((amdgpu_waves_per_eu(4))) void sinkhorn16b_bwd_kernel(const float* __restrict__ logits,
                                                                        const float* dM, float* dlogits,
                                                                        int64_t batch, int iters, float eps,
                                                                        const float* __restrict__ st) {
  extern __shared__ float2 sk16b_ck[];
  constexpr int SEG = RECORDED ? kSk16bRecSeg : kSk16bSeg;
  const Sk16bLane L = sk16b_lane(batch);
  const int64_t mm = L.valid ? L.m : 0;
  float K[4][4], G[4][4];
  {
    float mx[4];
    sk16b_load(logits + mm * 256, L.rb, L.cb, K);
    sk16b_exp(K, mx);
  }
  sk16b_load(dM + mm * 256, L.rb, L.cb, G);
  // segment sg covers iterations [first + (sg - 1) S, first + sg S) (sg >= 1) and segment 0 [0, first)
  const int nseg = (iters + SEG - 1) / SEG;
  const int first = iters - (nseg - 1) * SEG;
  const float* rec = RECORDED ? st + mm * sk16b_rec_floats(iters) : nullptr;
  float2* ck = sk16b_ck + (int64_t)(threadIdx.x >> 6) * nseg * 64 + (threadIdx.x & 63);
  // RECORDED: segment sg's sums (own row, own column) and starting scales.
  // The loads are unconditional, at addresses inside the matrix's record
  // (iterations past the segment clamped to the last one, segment 0's
  // checkpoint read from the last iteration's sums and replaced by 1 where it
  // is used), so that no value merges with an older one and each load is
  // waited for only where it is used.
  auto load_seg = [&](int sg, float (&rs_)[SEG], float (&cs_)[SEG], float& R0_, float& C0_) {
    const int it0 = sg == 0 ? 0 : first + (sg - 1) * SEG;
    const float* c = rec + (int64_t)iters * 32 + (int64_t)(sg - 1) * 32;
    R0_ = c[L.ro];
    C0_ = c[16 + L.co];
#pragma unroll
    for (int j = 0; j < SEG; ++j) {
      const float* r = rec + (int64_t)min(it0 + j, iters - 1) * 32;
      rs_[j] = r[L.ro];
      cs_[j] = r[16 + L.co];
    }
  };
  float nrs[SEG], ncs[SEG], nR0 = 1.0f, nC0 = 1.0f;
  if constexpr (RECORDED) {
    if (nseg > 0) load_seg(nseg - 1, nrs, ncs, nR0, nC0);
  }
  if constexpr (!RECORDED) {
    // the scales at each segment's start, lane-private (no cross-lane LDS use)
    Sk16bScales S;
    sk16b_scales(S, 1.0f, 1.0f);
    for (int sg = 0; sg < nseg; ++sg) {
      ck[sg * 64] = make_float2(S.R, S.C);
      if (sg == nseg - 1) break;
      const int len = sg == 0 ? first : SEG;
      for (int j = 0; j < len; ++j) {
        float rs, cs;
        sk16b_iter(K, S, eps, rs, cs);
      }
    }
  }
  for (int sg = nseg - 1; sg >= 0; --sg) {
    const int len = sg == 0 ? first : SEG;
    float R0 = 1.0f, C0 = 1.0f;
    float sR[SEG], srs[SEG], sC[SEG], scs[SEG];
    if constexpr (RECORDED) {
      R0 = sg > 0 ? nR0 : 1.0f;
      C0 = sg > 0 ? nC0 : 1.0f;
#pragma unroll
      for (int j = 0; j < SEG; ++j) {
        srs[j] = nrs[j];
        scs[j] = ncs[j];
      }
      if (sg > 0) load_seg(sg - 1, nrs, ncs, nR0, nC0);
      // the forward's cumulative scales, rebuilt with its own products (sk16b_iter)
      float R = R0, Cc = C0;
#pragma unroll
      for (int j = 0; j < SEG; ++j) {
        if (j < len) {
          R *= srs[j] > eps ? sk_rcp(srs[j]) : 1.0f;
          Cc *= scs[j] > eps ? sk_rcp(scs[j]) : 0.0f;
          sR[j] = R;
          sC[j] = Cc;
        }
      }
    } else {
      const float2 c = ck[sg * 64];
      R0 = c.x;
      C0 = c.y;
      Sk16bScales S;
      sk16b_scales(S, R0, C0);
#pragma unroll
      for (int j = 0; j < SEG; ++j) {
        if (j < len) {
          sk16b_iter(K, S, eps, srs[j], scs[j]);
          sR[j] = S.R;
          sC[j] = S.C;
        }
      }
    }
#pragma unroll
    for (int j = SEG - 1; j >= 0; --j) {
      if (j < len) sk16b_vjp_step(G, K, sR[j], srs[j], scs[j], j > 0 ? sR[j - 1] : R0, j > 0 ? sC[j - 1] : C0, eps);
    }
  }
  // through exp and the row-max shift: the max's gradient split evenly among
  // tied maxima (zero in exact arithmetic)
  float Hr[4][4], mx[4];
  sk16b_load(logits + mm * 256, L.rb, L.cb, Hr);
  {
    float pm[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) pm[s] = fmaxf(fmaxf(Hr[s][0], Hr[s][1]), fmaxf(Hr[s][2], Hr[s][3]));
    sk16b_row_bcast(sk16b_row_own(pm, MaxOp{}), mx);
  }
  float tot[4], cnt[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float a = 0.0f, c = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      G[s][t] *= K[s][t];
      a += G[s][t];
      c += Hr[s][t] == mx[s] ? 1.0f : 0.0f;
    }
    tot[s] = a;
    cnt[s] = c;
  }
  float totb[4], cntb[4];
  sk16b_row_bcast(sk16b_row_own(tot, SumOp{}), totb);
  sk16b_row_bcast(sk16b_row_own(cnt, SumOp{}), cntb);
  if (L.valid) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float corr = cntb[s] > 0.0f ? totb[s] / cntb[s] : 0.0f;
#pragma unroll
      for (int t = 0; t < 4; ++t) G[s][t] -= Hr[s][t] == mx[s] ? corr : 0.0f;
    }
    sk16b_store(dlogits + mm * 256, L.rb, L.cb, G);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

namespace {

// The n == 16 kernels need 16-byte aligned matrices; MHC_SK16=0 turns them off.
bool use_sk16(int n, const void* a, const void* b, const void* c) {
  if (n != 16 || knob(kKnobSk16, 1) == 0) return false;
  return aligned(a, 16) && aligned(b, 16) && (c == nullptr || aligned(c, 16));
}

// MHC_SK16_CPL selects the n == 16 batched layout: 0 (default) the block
// layout (16 lanes per matrix), 4 or 2 the kernels with that many columns per
// lane (4 or 8 lanes per matrix).
int sk16_cpl() {
  const int v = knob(kKnobSk16Cpl, 0);
  return v == 2 ? 2 : v == 4 ? 4 : 0;
}

// The block layout's VJP keeps a checkpoint per kSk16bSeg iterations in LDS.
int sk16b_nseg(int iters) { return (int)ceil_div((int64_t)iters, (int64_t)kSk16bSeg); }
bool sk16b_vjp_ok(int iters) { return sk16b_nseg(iters) <= kSk16bMaxSeg; }
size_t sk16b_lds_bytes(int iters) { return (size_t)(kSk16bThreads / 64) * sk16b_nseg(iters) * 64 * sizeof(float2); }
int64_t sk16b_blocks(int64_t batch) { return ceil_div(batch, (int64_t)4 * (kSk16bThreads / 64)); }

int64_t sk16_blocks(int64_t batch, int cpl) {
  return ceil_div(batch, (int64_t)(cpl == 4 ? Sk16<4>::MPW : Sk16<2>::MPW) * (kSk16Threads / 64));
}

struct SkPlan {
  int np;
  int wpb;          // wavefronts per block
  int64_t blocks;
  bool global_state;
  size_t lds_bytes;
  size_t ws_bytes;
};

int layout_w(int np) {
  const int e = np * np >= 64 ? np * np / 64 : 1;
  const int lr = np / e;
  const int g = np * lr;
  return (64 / g) * np;
}

int layout_mpw(int np) {
  const int e = np * np >= 64 ? np * np / 64 : 1;
  const int lr = np / e;
  return 64 / (np * lr);
}

SkPlan plan_bwd(int64_t batch, int n, int iters, int cus) {
  SkPlan p{};
  p.np = next_pow2(n);
  const int64_t ngroups = ceil_div(batch, layout_mpw(p.np));
  const size_t per_wave = (size_t)16 * (size_t)(iters > 0 ? iters : 1) * (size_t)layout_w(p.np);
  int wpb = (int)(kSkLdsBudget / per_wave);
  if (wpb > kSkThreads / 64) wpb = kSkThreads / 64;
  if (wpb >= 1) {
    p.global_state = false;
    p.wpb = (int)std::min<int64_t>(wpb, ngroups);
    if (p.wpb < 1) p.wpb = 1;
    p.lds_bytes = per_wave * p.wpb;
  } else {
    p.global_state = true;
    p.wpb = 1;
    p.lds_bytes = 0;
  }
  p.blocks = std::min<int64_t>(ceil_div(ngroups, p.wpb), (int64_t)cus * 16);
  if (p.blocks < 1) p.blocks = 1;
  p.ws_bytes = p.global_state ? per_wave * (size_t)p.blocks * (size_t)p.wpb : 0;
  return p;
}

// Block-layout kernels (16 < n <= 64): one wave per matrix, VJP state in
// LDS when one wave's fits the budget (as many waves per block as fit, up to
// 4), else in the workspace (which then starts at its first 256-byte
// boundary, hence 256 bytes more).
SkPlan plan_blk(int64_t batch, int n, int iters, int cus) {
  SkPlan p{};
  p.np = next_pow2(n);
  const size_t per_wave = (size_t)sk_blk_state_floats(p.np, iters) * sizeof(float);
  const int64_t fit = (int64_t)(kSkLdsBudget / per_wave);
  p.global_state = fit < 1;
  p.wpb = (int)std::max<int64_t>(1, std::min<int64_t>({kSkThreads / 64, batch, p.global_state ? 4 : fit}));
  p.blocks = std::max<int64_t>(1, std::min<int64_t>(ceil_div(batch, p.wpb), (int64_t)cus * 16));
  p.lds_bytes = p.global_state ? 0 : per_wave * (size_t)p.wpb;
  p.ws_bytes = p.global_state ? per_wave * (size_t)p.wpb * (size_t)p.blocks + 256 : 0;
  return p;
}

bool use_blk(int n) { return n > 16; }

// 32 < n <= 64: one four-wave workgroup per matrix (sinkhorn_wg_*), when the recomputing VJP's state
// fits its LDS.  Forward and VJP decide alike, so the VJP recomputes the forward's own iterates.  A
// single matrix is latency-bound on one wave; batched, the one-wave kernels hold one wave per SIMD
// (their 64 elements per lane take every register) and the workgroups several.  MHC_SK_WG=0 keeps the
// one-wave block kernels.
bool use_wg(int64_t batch, int n, int iters) {
  (void)batch;
  return n > 32 && knob(kKnobSkWg, 1) != 0 &&
         (size_t)sk_blk_state_floats(64, iters) * sizeof(float) <= (size_t)kSkWgMaxStateBytes;
}

dim3 wg_grid(int64_t batch) { return dim3((unsigned)std::min<int64_t>(batch, (int64_t)device_cu_count() * 16)); }

// Four waves per matrix up to one matrix per CU, two above (MHC_SK_WG=2: four at every batch).
bool wg_two_waves(int64_t batch) { return batch > device_cu_count() && knob(kKnobSkWg, 1) != 2; }

void launch_wg_fwd(const float* logits, float* M, int64_t batch, int n, int iters, float eps, float* rec,
                   hipStream_t s) {
  const dim3 g = wg_grid(batch);
  auto go = [&](auto rc) {
    constexpr int R = decltype(rc)::value;
    if (rec != nullptr)
      hipLaunchKernelGGL((sinkhorn_wg_fwd_kernel<R, true>), g, dim3(512 / R), 0, s, logits, M, batch, n, iters, eps, rec);
    else
      hipLaunchKernelGGL((sinkhorn_wg_fwd_kernel<R, false>), g, dim3(512 / R), 0, s, logits, M, batch, n, iters, eps,
                         nullptr);
  };
  if (wg_two_waves(batch)) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, 2>{});
}

void launch_wg_bwd(const float* logits, const float* dM, float* dlogits, int64_t batch, int n, int iters,
                   float eps, const float* rec, hipStream_t s) {
  const dim3 g = wg_grid(batch);
  const size_t smem = (size_t)sk_blk_state_floats(64, iters) * sizeof(float);
  auto go = [&](auto rc) {
    constexpr int R = decltype(rc)::value;
    if (rec != nullptr)
      hipLaunchKernelGGL((sinkhorn_wg_bwd_kernel<R, true>), g, dim3(512 / R), 0, s, logits, dM, dlogits, batch, n, iters,
                         eps, rec);
    else
      hipLaunchKernelGGL((sinkhorn_wg_bwd_kernel<R, false>), g, dim3(512 / R), smem, s, logits, dM, dlogits, batch, n,
                         iters, eps, nullptr);
  };
  if (wg_two_waves(batch)) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, 2>{});
}

// The first 256-byte boundary at or after p.
template <typename T>
T* align256(void* p) {
  const uintptr_t b = reinterpret_cast<uintptr_t>(p);
  return reinterpret_cast<T*>(b + (256 - b % 256) % 256);
}

template <int NP>
void launch_blk_fwd(const SkPlan& p, const float* logits, float* M, int64_t batch, int n, int iters, float eps,
                    float* rec, hipStream_t s) {
  if (rec != nullptr)
    hipLaunchKernelGGL((sinkhorn_blk_fwd_kernel<NP, true>), dim3((unsigned)p.blocks), dim3(p.wpb * 64), 0, s,
                       logits, M, batch, n, iters, eps, rec);
  else
    hipLaunchKernelGGL((sinkhorn_blk_fwd_kernel<NP, false>), dim3((unsigned)p.blocks), dim3(p.wpb * 64), 0, s,
                       logits, M, batch, n, iters, eps, nullptr);
}

// rec: the forward's recorded state (16-byte aligned), or nullptr to
// recompute it (in LDS, or in ws when the plan says so).
template <int NP>
void launch_blk_bwd(const SkPlan& p, const float* logits, const float* dM, float* dlogits, int64_t batch, int n,
                    int iters, float eps, float* ws, float* rec, hipStream_t s) {
  const dim3 g((unsigned)p.blocks), b(p.wpb * 64);
  if (rec != nullptr && !p.global_state)
    hipLaunchKernelGGL((sinkhorn_blk_bwd_kernel<NP, kSkBlkRecLds>), g, b, p.lds_bytes, s, logits, dM, dlogits,
                       batch, n, iters, eps, rec);
  else if (rec != nullptr)
    hipLaunchKernelGGL((sinkhorn_blk_bwd_kernel<NP, kSkBlkRecGlobal>), g, b, 0, s, logits, dM, dlogits, batch, n,
                       iters, eps, rec);
  else if (p.global_state)
    hipLaunchKernelGGL((sinkhorn_blk_bwd_kernel<NP, kSkBlkWs>), g, b, 0, s, logits, dM, dlogits, batch, n, iters,
                       eps, align256<float>(ws));
  else
    hipLaunchKernelGGL((sinkhorn_blk_bwd_kernel<NP, kSkBlkLds>), g, b, p.lds_bytes, s, logits, dM, dlogits, batch,
                       n, iters, eps, nullptr);
}

template <int NP>
void launch_fwd(const float* logits, float* M, int64_t batch, int n, int iters, float eps,
                hipStream_t stream, int cus) {
  using L = SkLayout<NP>;
  const int64_t ngroups = ceil_div(batch, L::MPW);
  const int wpb = (int)std::min<int64_t>(kSkThreads / 64, ngroups);
  const int64_t blocks = std::min<int64_t>(ceil_div(ngroups, wpb), (int64_t)cus * 16);
  hipLaunchKernelGGL(sinkhorn_fwd_kernel<NP>, dim3((unsigned)blocks), dim3(wpb * 64), 0, stream,
                     logits, M, batch, n, iters, eps);
}

template <int NP>
void launch_bwd(const SkPlan& p, const float* logits, const float* dM, float* dlogits,
                int64_t batch, int n, int iters, float eps, float* ws, hipStream_t stream) {
  if (p.global_state) {
    hipLaunchKernelGGL((sinkhorn_bwd_kernel<NP, true>), dim3((unsigned)p.blocks), dim3(p.wpb * 64),
                       0, stream, logits, dM, dlogits, batch, n, iters, eps, ws);
  } else {
    hipLaunchKernelGGL((sinkhorn_bwd_kernel<NP, false>), dim3((unsigned)p.blocks), dim3(p.wpb * 64),
                       p.lds_bytes, stream, logits, dM, dlogits, batch, n, iters, eps, ws);
  }
}

}  // namespace
}  // namespace mhc

using namespace mhc;

extern "C" int mhc_sinkhorn_fwd(const float* logits, float* M, int64_t batch, int n, int iters,
                                float eps, void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(batch >= 0, "batch=%lld must be >= 0", (long long)batch);
  MHC_CHECK_ARG(iters >= 0, "iters=%d must be >= 0", iters);
  if (batch == 0) return MHC_OK;
  MHC_CHECK_ARG(logits != nullptr && M != nullptr, "null pointer argument");
  const int cus = device_cu_count();
  hipStream_t s = (hipStream_t)stream;
  if (use_sk16(n, logits, M, nullptr)) {
    const int cpl = sk16_cpl();
    if (cpl == 0) {
      hipLaunchKernelGGL((sinkhorn16b_fwd_kernel<false>), dim3((unsigned)sk16b_blocks(batch)), dim3(kSk16bThreads),
                         0, s, logits, M, batch, iters, eps, nullptr);
      MHC_CHECK_LAUNCH("sinkhorn16b_fwd_kernel");
      return MHC_OK;
    }
    const dim3 g((unsigned)sk16_blocks(batch, cpl)), b(kSk16Threads);
    if (cpl == 4)
      hipLaunchKernelGGL((sinkhorn16_fwd_kernel<4>), g, b, 0, s, logits, M, batch, iters, eps);
    else
      hipLaunchKernelGGL((sinkhorn16_fwd_kernel<2>), g, b, 0, s, logits, M, batch, iters, eps);
    MHC_CHECK_LAUNCH("sinkhorn16_fwd_kernel");
    return MHC_OK;
  }
  if (use_wg(batch, n, iters)) {
    launch_wg_fwd(logits, M, batch, n, iters, eps, nullptr, s);
    MHC_CHECK_LAUNCH("sinkhorn_wg_fwd_kernel");
    return MHC_OK;
  }
  if (use_blk(n)) {
    const SkPlan p = plan_blk(batch, n, iters, cus);
    if (p.np == 32) launch_blk_fwd<32>(p, logits, M, batch, n, iters, eps, nullptr, s);
    else launch_blk_fwd<64>(p, logits, M, batch, n, iters, eps, nullptr, s);
    MHC_CHECK_LAUNCH("sinkhorn_blk_fwd_kernel");
    return MHC_OK;
  }
  switch (next_pow2(n)) {
    case 1: launch_fwd<1>(logits, M, batch, n, iters, eps, s, cus); break;
    case 2: launch_fwd<2>(logits, M, batch, n, iters, eps, s, cus); break;
    case 4: launch_fwd<4>(logits, M, batch, n, iters, eps, s, cus); break;
    case 8: launch_fwd<8>(logits, M, batch, n, iters, eps, s, cus); break;
    case 16: launch_fwd<16>(logits, M, batch, n, iters, eps, s, cus); break;
    case 32: launch_fwd<32>(logits, M, batch, n, iters, eps, s, cus); break;
    default: launch_fwd<64>(logits, M, batch, n, iters, eps, s, cus); break;
  }
  MHC_CHECK_LAUNCH("sinkhorn_fwd_kernel");
  return MHC_OK;
}

namespace {
// n == 16, lanes-per-matrix VJP: 64 floats of workspace per matrix and iteration.
size_t sk16_ws_bytes(int64_t batch, int iters) {
  return (size_t)batch * (size_t)(iters > 0 ? iters : 1) * 64 * sizeof(float);
}
}  // namespace

extern "C" size_t mhc_sinkhorn_bwd_workspace_bytes(int64_t batch, int n, int iters) {
  if (n < 1 || n > MHC_MAX_N || batch <= 0 || iters < 0) return 0;
  if (use_blk(n)) return plan_blk(batch, n, iters, device_cu_count()).ws_bytes;
  const size_t gen = plan_bwd(batch, n, iters, device_cu_count()).ws_bytes;
  // n == 16: the block layout needs none; the other layouts keep their state there
  if (n == 16 && !(sk16_cpl() == 0 && sk16b_vjp_ok(iters))) return std::max(gen, sk16_ws_bytes(batch, iters) + 256);
  return gen;
}

extern "C" int mhc_sinkhorn_bwd(const float* logits, const float* dM, float* dlogits,
                                int64_t batch, int n, int iters, float eps, void* workspace,
                                size_t workspace_bytes, void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(batch >= 0, "batch=%lld must be >= 0", (long long)batch);
  MHC_CHECK_ARG(iters >= 0, "iters=%d must be >= 0", iters);
  if (batch == 0) return MHC_OK;
  MHC_CHECK_ARG(logits != nullptr && dM != nullptr && dlogits != nullptr, "null pointer argument");
  hipStream_t s = (hipStream_t)stream;
  if (use_sk16(n, logits, dM, dlogits) && sk16_cpl() == 0 && sk16b_vjp_ok(iters)) {
    hipLaunchKernelGGL((sinkhorn16b_bwd_kernel<false>), dim3((unsigned)sk16b_blocks(batch)), dim3(kSk16bThreads),
                       sk16b_lds_bytes(iters), s, logits, dM, dlogits, batch, iters, eps, nullptr);
    MHC_CHECK_LAUNCH("sinkhorn16b_bwd_kernel");
    return MHC_OK;
  }
  if (use_sk16(n, logits, dM, dlogits) && workspace != nullptr) {
    // The recomputed state starts at the first 256-byte boundary of the workspace:
    // each matrix's state (256 bytes per iteration) then fills whole cache
    // lines, none shared with a matrix that another wave or CU processes.
    const uintptr_t base = reinterpret_cast<uintptr_t>(workspace);
    const size_t pad = (size_t)((256 - base % 256) % 256);
    const size_t need = sk16_ws_bytes(batch, iters);
    if (workspace_bytes >= need + pad) {
      float* st = reinterpret_cast<float*>(base + pad);
      const int cpl = sk16_cpl() == 2 ? 2 : 4;
      const dim3 g((unsigned)sk16_blocks(batch, cpl)), b(kSk16Threads);
      if (cpl == 4)
        hipLaunchKernelGGL((sinkhorn16_bwd_kernel<4>), g, b, 0, s, logits, dM, dlogits, batch, iters, eps,
                           st);
      else
        hipLaunchKernelGGL((sinkhorn16_bwd_kernel<2>), g, b, 0, s, logits, dM, dlogits, batch, iters, eps,
                           st);
      MHC_CHECK_LAUNCH("sinkhorn16_bwd_kernel");
      return MHC_OK;
    }
  }
  if (use_wg(batch, n, iters)) {
    launch_wg_bwd(logits, dM, dlogits, batch, n, iters, eps, nullptr, s);
    MHC_CHECK_LAUNCH("sinkhorn_wg_bwd_kernel");
    return MHC_OK;
  }
  if (use_blk(n)) {
    const SkPlan p = plan_blk(batch, n, iters, device_cu_count());
    MHC_CHECK_ARG(workspace_bytes >= p.ws_bytes && (p.ws_bytes == 0 || workspace != nullptr),
                  "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, p.ws_bytes);
    if (p.np == 32) launch_blk_bwd<32>(p, logits, dM, dlogits, batch, n, iters, eps, (float*)workspace, nullptr, s);
    else launch_blk_bwd<64>(p, logits, dM, dlogits, batch, n, iters, eps, (float*)workspace, nullptr, s);
    MHC_CHECK_LAUNCH("sinkhorn_blk_bwd_kernel");
    return MHC_OK;
  }
  const SkPlan p = plan_bwd(batch, n, iters, device_cu_count());
  MHC_CHECK_ARG(workspace_bytes >= p.ws_bytes && (p.ws_bytes == 0 || workspace != nullptr),
                "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes,
                p.ws_bytes);
  float* ws = (float*)workspace;
  switch (p.np) {
    case 1: launch_bwd<1>(p, logits, dM, dlogits, batch, n, iters, eps, ws, s); break;
    case 2: launch_bwd<2>(p, logits, dM, dlogits, batch, n, iters, eps, ws, s); break;
    case 4: launch_bwd<4>(p, logits, dM, dlogits, batch, n, iters, eps, ws, s); break;
    case 8: launch_bwd<8>(p, logits, dM, dlogits, batch, n, iters, eps, ws, s); break;
    case 16: launch_bwd<16>(p, logits, dM, dlogits, batch, n, iters, eps, ws, s); break;
    case 32: launch_bwd<32>(p, logits, dM, dlogits, batch, n, iters, eps, ws, s); break;
    default: launch_bwd<64>(p, logits, dM, dlogits, batch, n, iters, eps, ws, s); break;
  }
  MHC_CHECK_LAUNCH("sinkhorn_bwd_kernel");
  return MHC_OK;
}

// ---------------------------------------------------------------------------
// Recorded state: the forward keeps what the VJP would otherwise recompute.
// ---------------------------------------------------------------------------

namespace {
// Bytes of recorded state per layout: n == 16 (the block layout's compact
// record, whatever MHC_SK16_CPL selects for the unrecorded calls) and
// 16 < n <= 64 (block layout, MHC_SK_BLK_RECORD=0 turns its recording off).
size_t sk_record_bytes(int64_t batch, int n, int iters) {
  if (n == 16) return (size_t)batch * (size_t)sk16b_rec_floats(iters) * sizeof(float);
  return (size_t)batch * (size_t)sk_blk_state_floats(next_pow2(n), iters) * sizeof(float);
}

// The state starts at the first 256-byte boundary of the caller's buffer
// (the same offset for the forward that writes it and the VJP that reads it).
float* sk_state_ptr(const void* state, size_t state_bytes, int64_t batch, int n, int iters) {
  const uintptr_t base = reinterpret_cast<uintptr_t>(state);
  const size_t pad = (size_t)((256 - base % 256) % 256);
  if (state == nullptr || state_bytes < sk_record_bytes(batch, n, iters) + pad) return nullptr;
  return reinterpret_cast<float*>(base + pad);
}
}  // namespace

extern "C" size_t mhc_sinkhorn_state_bytes(int64_t batch, int n, int iters) {
  if (batch <= 0 || iters < 0) return 0;
  if (n == 16 && (knob(kKnobSk16, 1) == 0 || knob(kKnobSk16Record, 1) == 0)) return 0;
  if (n > 16 && n <= MHC_MAX_N && knob(kKnobSkBlkRecord, 1) == 0) return 0;
  if (n < 16 || n > MHC_MAX_N) return 0;
  return sk_record_bytes(batch, n, iters) + 256;
}

extern "C" int mhc_sinkhorn_fwd_record(const float* logits, float* M, void* state, size_t state_bytes,
                                       int64_t batch, int n, int iters, float eps, void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 16 && n <= MHC_MAX_N, "a recorded Sinkhorn state exists for 16 <= n <= %d only (n=%d)",
                MHC_MAX_N, n);
  MHC_CHECK_ARG(batch >= 0, "batch=%lld must be >= 0", (long long)batch);
  MHC_CHECK_ARG(iters >= 0, "iters=%d must be >= 0", iters);
  if (batch == 0) return MHC_OK;
  MHC_CHECK_ARG(logits != nullptr && M != nullptr, "null pointer argument");
  MHC_CHECK_ARG(n != 16 || (aligned(logits, 16) && aligned(M, 16)), "logits and M must be 16-byte aligned");
  float* st = sk_state_ptr(state, state_bytes, batch, n, iters);
  MHC_CHECK_ARG(st != nullptr, "state of %zu bytes is smaller than the %zu bytes required", state_bytes,
                sk_record_bytes(batch, n, iters) + 256);
  hipStream_t s = (hipStream_t)stream;
  if (use_wg(batch, n, iters)) {
    launch_wg_fwd(logits, M, batch, n, iters, eps, st, s);
    MHC_CHECK_LAUNCH("sinkhorn_wg_fwd_kernel");
    return MHC_OK;
  }
  if (n > 16) {
    const SkPlan p = plan_blk(batch, n, iters, device_cu_count());
    if (p.np == 32) launch_blk_fwd<32>(p, logits, M, batch, n, iters, eps, st, s);
    else launch_blk_fwd<64>(p, logits, M, batch, n, iters, eps, st, s);
    MHC_CHECK_LAUNCH("sinkhorn_blk_fwd_kernel");
    return MHC_OK;
  }
  hipLaunchKernelGGL((sinkhorn16b_fwd_kernel<true>), dim3((unsigned)sk16b_blocks(batch)), dim3(kSk16bThreads), 0, s,
                     logits, M, batch, iters, eps, st);
  MHC_CHECK_LAUNCH("sinkhorn16b_fwd_kernel");
  return MHC_OK;
}

extern "C" int mhc_sinkhorn_bwd_recorded(const float* logits, const float* dM, float* dlogits, const void* state,
                                         size_t state_bytes, int64_t batch, int n, int iters, float eps,
                                         void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 16 && n <= MHC_MAX_N, "a recorded Sinkhorn state exists for 16 <= n <= %d only (n=%d)",
                MHC_MAX_N, n);
  MHC_CHECK_ARG(batch >= 0, "batch=%lld must be >= 0", (long long)batch);
  MHC_CHECK_ARG(iters >= 0, "iters=%d must be >= 0", iters);
  if (batch == 0) return MHC_OK;
  MHC_CHECK_ARG(logits != nullptr && dM != nullptr && dlogits != nullptr, "null pointer argument");
  MHC_CHECK_ARG(n != 16 || (aligned(logits, 16) && aligned(dM, 16) && aligned(dlogits, 16)),
                "logits, dM and dlogits must be 16-byte aligned");
  float* st = sk_state_ptr(state, state_bytes, batch, n, iters);
  MHC_CHECK_ARG(st != nullptr, "state of %zu bytes is smaller than the %zu bytes required", state_bytes,
                sk_record_bytes(batch, n, iters) + 256);
  hipStream_t s = (hipStream_t)stream;
  if (use_wg(batch, n, iters)) {
    launch_wg_bwd(logits, dM, dlogits, batch, n, iters, eps, st, s);
    MHC_CHECK_LAUNCH("sinkhorn_wg_bwd_kernel");
    return MHC_OK;
  }
  if (n > 16) {
    const SkPlan p = plan_blk(batch, n, iters, device_cu_count());
    if (p.np == 32) launch_blk_bwd<32>(p, logits, dM, dlogits, batch, n, iters, eps, nullptr, st, s);
    else launch_blk_bwd<64>(p, logits, dM, dlogits, batch, n, iters, eps, nullptr, st, s);
    MHC_CHECK_LAUNCH("sinkhorn_blk_bwd_kernel");
    return MHC_OK;
  }
  hipLaunchKernelGGL((sinkhorn16b_bwd_kernel<true>), dim3((unsigned)sk16b_blocks(batch)), dim3(kSk16bThreads), 0, s,
                     logits, dM, dlogits, batch, iters, eps, st);
  MHC_CHECK_LAUNCH("sinkhorn16b_bwd_kernel");
  return MHC_OK;
}
