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

// REC: also record the VJP state ([batch][iters][4][16] floats at st) for
// sinkhorn16_bwd_kernel<CPL', true>.
template <int CPL, bool REC>
__global__ __launch_bounds__(kSk16Threads) void sinkhorn16_fwd_kernel(const float* __restrict__ logits,
                                                                      float* __restrict__ out, int64_t batch,
                                                                      int iters, float eps, float* __restrict__ st) {
  int p;
  const int64_t m = sk16_matrix<CPL>(p);
  const bool mvalid = m < batch;
  float P[16][CPL];
  sk16_load_k<CPL>(logits + (mvalid ? m : 0) * 256, mvalid, p, P);
  if constexpr (REC) {
    sk16_forward_record<CPL>(P, iters, eps, p, mvalid, st + (mvalid ? m : 0) * (int64_t)iters * 64);
  } else {
    for (int it = 0; it < iters; ++it)
      sk16_iter<CPL>(P, eps, [](int, float, float) {}, [](int, float, float) {});
  }
  if (mvalid) {
    float* O = out + m * 256;
#pragma unroll
    for (int i = 0; i < 16; ++i) sk16_st<CPL>(O + i * 16 + CPL * p, P[i]);
  }
}

// st: [batch][iters][4][16] floats (R_k, rs_k, C_k, cs_k).  dM may alias dlogits.
// RECORDED: st was written by sinkhorn16_fwd_kernel<CPL', true> for the same
// logits; otherwise the forward is recomputed here and recorded first.
template <int CPL, bool RECORDED>
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

  if constexpr (!RECORDED) {
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
// host side
// ---------------------------------------------------------------------------

namespace {

// The n == 16 kernels need 16-byte aligned matrices; MHC_SK16=0 turns them off.
bool use_sk16(int n, const void* a, const void* b, const void* c) {
  if (n != 16 || knob(kKnobSk16, 1) == 0) return false;
  return aligned(a, 16) && aligned(b, 16) && (c == nullptr || aligned(c, 16));
}

// MHC_SK16_CPL (2 or 4) selects the columns per lane (tuning override).
int sk16_cpl() { return knob(kKnobSk16Cpl, 4) == 2 ? 2 : 4; }

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
    const dim3 g((unsigned)sk16_blocks(batch, cpl)), b(kSk16Threads);
    if (cpl == 4)
      hipLaunchKernelGGL((sinkhorn16_fwd_kernel<4, false>), g, b, 0, s, logits, M, batch, iters, eps, nullptr);
    else
      hipLaunchKernelGGL((sinkhorn16_fwd_kernel<2, false>), g, b, 0, s, logits, M, batch, iters, eps, nullptr);
    MHC_CHECK_LAUNCH("sinkhorn16_fwd_kernel");
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
// n == 16: 64 floats of recorded state per matrix and iteration.
size_t sk16_state_bytes(int64_t batch, int iters) {
  return (size_t)batch * (size_t)(iters > 0 ? iters : 1) * 64 * sizeof(float);
}
}  // namespace

extern "C" size_t mhc_sinkhorn_bwd_workspace_bytes(int64_t batch, int n, int iters) {
  if (n < 1 || n > MHC_MAX_N || batch <= 0 || iters < 0) return 0;
  if (use_blk(n)) return plan_blk(batch, n, iters, device_cu_count()).ws_bytes;
  const size_t gen = plan_bwd(batch, n, iters, device_cu_count()).ws_bytes;
  if (n == 16) return std::max(gen, sk16_state_bytes(batch, iters) + 256);
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
  if (use_sk16(n, logits, dM, dlogits) && workspace != nullptr) {
    // The recorded state starts at the first 256-byte boundary of the workspace:
    // each matrix's records (256 bytes per iteration) then fill whole cache
    // lines, none shared with a matrix that another wave or CU processes.
    const uintptr_t base = reinterpret_cast<uintptr_t>(workspace);
    const size_t pad = (size_t)((256 - base % 256) % 256);
    const size_t need = sk16_state_bytes(batch, iters);
    if (workspace_bytes >= need + pad) {
      float* st = reinterpret_cast<float*>(base + pad);
      const int cpl = sk16_cpl();
      const dim3 g((unsigned)sk16_blocks(batch, cpl)), b(kSk16Threads);
      if (cpl == 4)
        hipLaunchKernelGGL((sinkhorn16_bwd_kernel<4, false>), g, b, 0, s, logits, dM, dlogits, batch, iters, eps,
                           st);
      else
        hipLaunchKernelGGL((sinkhorn16_bwd_kernel<2, false>), g, b, 0, s, logits, dM, dlogits, batch, iters, eps,
                           st);
      MHC_CHECK_LAUNCH("sinkhorn16_bwd_kernel");
      return MHC_OK;
    }
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
// Bytes of recorded state per layout: n == 16 (batched kernels) and
// 16 < n <= 64 (block layout, MHC_SK_BLK_RECORD=0 turns its recording off).
size_t sk_record_bytes(int64_t batch, int n, int iters) {
  if (n == 16) return sk16_state_bytes(batch, iters);
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
  if (n > 16) {
    const SkPlan p = plan_blk(batch, n, iters, device_cu_count());
    if (p.np == 32) launch_blk_fwd<32>(p, logits, M, batch, n, iters, eps, st, s);
    else launch_blk_fwd<64>(p, logits, M, batch, n, iters, eps, st, s);
    MHC_CHECK_LAUNCH("sinkhorn_blk_fwd_kernel");
    return MHC_OK;
  }
  const int cpl = sk16_cpl();
  const dim3 g((unsigned)sk16_blocks(batch, cpl)), b(kSk16Threads);
  if (cpl == 4)
    hipLaunchKernelGGL((sinkhorn16_fwd_kernel<4, true>), g, b, 0, s, logits, M, batch, iters, eps, st);
  else
    hipLaunchKernelGGL((sinkhorn16_fwd_kernel<2, true>), g, b, 0, s, logits, M, batch, iters, eps, st);
  MHC_CHECK_LAUNCH("sinkhorn16_fwd_kernel");
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
  if (n > 16) {
    const SkPlan p = plan_blk(batch, n, iters, device_cu_count());
    if (p.np == 32) launch_blk_bwd<32>(p, logits, dM, dlogits, batch, n, iters, eps, nullptr, st, s);
    else launch_blk_bwd<64>(p, logits, dM, dlogits, batch, n, iters, eps, nullptr, st, s);
    MHC_CHECK_LAUNCH("sinkhorn_blk_bwd_kernel");
    return MHC_OK;
  }
  const int cpl = sk16_cpl();
  const dim3 g((unsigned)sk16_blocks(batch, cpl)), b(kSk16Threads);
  if (cpl == 4)
    hipLaunchKernelGGL((sinkhorn16_bwd_kernel<4, true>), g, b, 0, s, logits, dM, dlogits, batch, iters, eps, st);
  else
    hipLaunchKernelGGL((sinkhorn16_bwd_kernel<2, true>), g, b, 0, s, logits, dM, dlogits, batch, iters, eps, st);
  MHC_CHECK_LAUNCH("sinkhorn16_bwd_kernel");
  return MHC_OK;
}
