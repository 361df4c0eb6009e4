// Sinkhorn-Knopp projection and its VJP for the matrices of one wavefront
// (device functions shared by the batched kernels and the fused reduction).
//
// Semantics follow mhc_mlx/reference.py:20-48, 58-69:
//   K = exp(H - rowmax(H));  repeat `iters` times:
//     row step:    s_i = sum_j P_ij;  P_ij *= (s_i > eps ? 1/s_i : 1)
//     column step: s_j = sum_i P_ij;  P_ij *= (s_j > eps ? 1/s_j : 0)
//
// Lane layout for an NP x NP matrix (NP = n rounded up to a power of two,
// padding entries are exact zeros and never change a sum):
//   E   elements per lane (NP*NP/64, at least 1),
//   LR  lanes per row (a row is LR consecutive lanes, E columns each),
//   G   lanes per matrix (NP*LR), MPW = 64/G matrices per wavefront.
// Row sums reduce over LR adjacent lanes, column sums over lanes LR apart;
// all `iters` rounds stay in registers.
//
// The VJP recomputes the forward and records, per iteration, the row and
// column sums and the cumulative row/column scale vectors R_k, C_k
// (4 * iters * W floats per wavefront).  The pre-step matrices are rebuilt
// as R K C, which stays exact for masked (zeroed) columns, unlike dividing
// the scaled matrix by its scale.
#pragma once

#include "mhc_device.hpp"

namespace mhc {

// Row / column scale 1/s: the hardware reciprocal (v_rcp_f32, within 1 ulp;
// s > eps > 0 is never denormal).  The reference divides by s; the results
// agree to a few ulp, far inside the fp32 tolerance.
MHC_DEV float sk_rcp(float s) { return __builtin_amdgcn_rcpf(s); }

// Iteration counts up to this keep the VJP state in registers (n <= 8).
constexpr int kSkRegIters = 32;

template <int NP>
struct SkLayout {
  static constexpr int E = NP * NP >= 64 ? NP * NP / 64 : 1;
  static constexpr int LR = NP / E;
  static constexpr int G = NP * LR;
  static constexpr int MPW = 64 / G;
  static constexpr int W = MPW * NP;  // row (or column) slots per wavefront
};

// Floats of VJP state per wavefront.
__host__ __device__ inline int64_t sk_state_floats(int np, int iters) {
  const int e = np * np >= 64 ? np * np / 64 : 1;
  const int lr = np / e;
  const int g = np * lr;
  return (int64_t)4 * (iters > 0 ? iters : 1) * (64 / g) * np;
}

// Forward for the matrix of this lane's group: H / out point at that
// matrix ([n, n] row-major); mvalid false for groups past the batch.
template <int NP>
MHC_DEV void sk_fwd_group(const float* __restrict__ H, float* __restrict__ out, bool mvalid, int n,
                          int iters, float eps, int lane) {
  using L = SkLayout<NP>;
  const int lm = lane % L::G;
  const int r = lm / L::LR;
  const int c0 = (lm % L::LR) * L::E;
  const bool rvalid = mvalid && r < n;
  const float* Hr = H + (int64_t)r * n;
  float P[L::E];
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < L::E; ++e) {
    const bool v = rvalid && (c0 + e) < n;
    P[e] = v ? Hr[c0 + e] : -INFINITY;
    mx = fmaxf(mx, P[e]);
  }
  mx = group_max<L::LR>(mx);
#pragma unroll
  for (int e = 0; e < L::E; ++e) {
    const bool v = rvalid && (c0 + e) < n;
    P[e] = v ? expf(P[e] - mx) : 0.0f;
  }
  for (int it = 0; it < iters; ++it) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < L::E; ++e) s += P[e];
    s = group_sum<L::LR>(s);
    const float rsc = (rvalid && s > eps) ? sk_rcp(s) : 1.0f;
#pragma unroll
    for (int e = 0; e < L::E; ++e) P[e] *= rsc;
#pragma unroll
    for (int e = 0; e < L::E; ++e) {
      const float cs = strided_sum<L::LR, L::G>(P[e]);
      const bool cv = mvalid && (c0 + e) < n;
      const float csc = (cv && cs > eps) ? sk_rcp(cs) : 0.0f;
      P[e] *= csc;
    }
  }
  if (rvalid) {
    float* O = out + (int64_t)r * n;
#pragma unroll
    for (int e = 0; e < L::E; ++e)
      if ((c0 + e) < n) O[c0 + e] = P[e];
  }
}

// The same projection of one n x n matrix, n == NP <= 8, computed by a whole
// wave (its 64 / G lane groups all process the matrix) with the lane layout
// and arithmetic of sk_fwd_group, so the results are bitwise those of the
// batched kernel.  Returns the matrix as wave-uniform values M[i * NP + j]
// and, in `mine`, the element of lanes < NP * NP (row lane / NP, column
// lane % NP).
template <int NP>
MHC_DEV void sk_fwd_wave(const float* __restrict__ H, int iters, float eps, int lane, float (&M)[NP * NP],
                         float& mine) {
  using L = SkLayout<NP>;
  static_assert(L::E == 1 && L::LR == NP, "one element per lane, one row per NP lanes");
  const int lm = lane % L::G;
  const int r = lm / L::LR;
  const int c = lm % L::LR;
  float P = H[r * NP + c];
  const float mx = group_max<L::LR>(P);
  P = expf(P - mx);
  for (int it = 0; it < iters; ++it) {
    const float s = group_sum<L::LR>(P);
    P *= s > eps ? sk_rcp(s) : 1.0f;
    const float cs = strided_sum<L::LR, L::G>(P);
    P *= cs > eps ? sk_rcp(cs) : 0.0f;
  }
  mine = P;
#pragma unroll
  for (int k = 0; k < NP * NP; ++k)
    M[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, P), k));
}

// VJP for the matrix of this lane's group: dlogits = d/dH <dM, SK(H)>.
// st: this wavefront's state, layout [4][iters][W] (row sums, cumulative row
// scale R_k, column sums, cumulative column scale C_k).
template <int NP>
MHC_DEV void sk_bwd_group(const float* __restrict__ H, const float* __restrict__ dM,
                          float* __restrict__ dlogits, bool mvalid, int n, int iters, float eps,
                          float* st, int lane) {
  using L = SkLayout<NP>;
  const int lm = lane % L::G;
  const int msub = lane / L::G;
  const int r = lm / L::LR;
  const int c0 = (lm % L::LR) * L::E;
  const bool rvalid = mvalid && r < n;
  float* st_rs = st;
  float* st_R = st + (int64_t)iters * L::W;
  float* st_cs = st + (int64_t)2 * iters * L::W;
  float* st_C = st + (int64_t)3 * iters * L::W;
  const int rslot = msub * NP + r;
  const int cslot = msub * NP + c0;

  const float* Hrow = H + (int64_t)r * n;
  float Hr[L::E], K[L::E], P[L::E];
  float mx = -INFINITY;
#pragma unroll
  for (int e = 0; e < L::E; ++e) {
    const bool v = rvalid && (c0 + e) < n;
    Hr[e] = v ? Hrow[c0 + e] : -INFINITY;
    mx = fmaxf(mx, Hr[e]);
  }
  mx = group_max<L::LR>(mx);
#pragma unroll
  for (int e = 0; e < L::E; ++e) {
    const bool v = rvalid && (c0 + e) < n;
    K[e] = v ? expf(Hr[e] - mx) : 0.0f;
    P[e] = K[e];
  }
  // forward recompute, recording sums and cumulative scales
  float Rc = 1.0f;
  float Cc[L::E];
#pragma unroll
  for (int e = 0; e < L::E; ++e) Cc[e] = 1.0f;
  for (int it = 0; it < iters; ++it) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < L::E; ++e) s += P[e];
    s = group_sum<L::LR>(s);
    const float rsc = (rvalid && s > eps) ? sk_rcp(s) : 1.0f;
#pragma unroll
    for (int e = 0; e < L::E; ++e) P[e] *= rsc;
    Rc *= rsc;
    st_rs[(int64_t)it * L::W + rslot] = s;
    st_R[(int64_t)it * L::W + rslot] = Rc;
#pragma unroll
    for (int e = 0; e < L::E; ++e) {
      const float cs = strided_sum<L::LR, L::G>(P[e]);
      const bool cv = mvalid && (c0 + e) < n;
      const float csc = (cv && cs > eps) ? sk_rcp(cs) : 0.0f;
      P[e] *= csc;
      Cc[e] *= csc;
      st_cs[(int64_t)it * L::W + cslot + e] = cs;
      st_C[(int64_t)it * L::W + cslot + e] = Cc[e];
    }
  }
  // reverse sweep
  float Gd[L::E];
  {
    const float* D = dM + (int64_t)r * n;
#pragma unroll
    for (int e = 0; e < L::E; ++e) {
      const bool v = rvalid && (c0 + e) < n;
      Gd[e] = v ? D[c0 + e] : 0.0f;
    }
  }
  for (int it = iters - 1; it >= 0; --it) {
    const float Rk = st_R[(int64_t)it * L::W + rslot];
    const float Rp = it > 0 ? st_R[(int64_t)(it - 1) * L::W + rslot] : 1.0f;
    float Cp[L::E];
#pragma unroll
    for (int e = 0; e < L::E; ++e) Cp[e] = it > 0 ? st_C[(int64_t)(it - 1) * L::W + cslot + e] : 1.0f;
    // column step: input R_k K C_{k-1}
#pragma unroll
    for (int e = 0; e < L::E; ++e) {
      const float pin = Rk * K[e] * Cp[e];
      const float dot = strided_sum<L::LR, L::G>(Gd[e] * pin);
      const float cs = st_cs[(int64_t)it * L::W + cslot + e];
      const bool cv = mvalid && (c0 + e) < n;
      if (cv && cs > eps) {
        const float sc = sk_rcp(cs);
        Gd[e] = sc * Gd[e] - sc * sc * dot;
      } else {
        Gd[e] = 0.0f;
      }
    }
    // row step: input R_{k-1} K C_{k-1}
    float prod = 0.0f;
#pragma unroll
    for (int e = 0; e < L::E; ++e) prod += Gd[e] * (Rp * K[e] * Cp[e]);
    const float dot = group_sum<L::LR>(prod);
    const float rs = st_rs[(int64_t)it * L::W + rslot];
    if (rvalid && rs > eps) {
      const float sc = sk_rcp(rs);
#pragma unroll
      for (int e = 0; e < L::E; ++e) Gd[e] = sc * Gd[e] - sc * sc * dot;
    }
  }
  // through exp and the row-max shift (gradient of the max split evenly
  // among tied maxima; it is zero in exact arithmetic)
  float cnt = 0.0f, tot = 0.0f;
  float dsh[L::E];
#pragma unroll
  for (int e = 0; e < L::E; ++e) {
    const bool v = rvalid && (c0 + e) < n;
    dsh[e] = v ? Gd[e] * K[e] : 0.0f;
    tot += dsh[e];
    cnt += (v && Hr[e] == mx) ? 1.0f : 0.0f;
  }
  tot = group_sum<L::LR>(tot);
  cnt = group_sum<L::LR>(cnt);
  if (rvalid) {
    float* O = dlogits + (int64_t)r * n;
    const float corr = cnt > 0.0f ? tot / cnt : 0.0f;
#pragma unroll
    for (int e = 0; e < L::E; ++e)
      if ((c0 + e) < n) O[c0 + e] = dsh[e] - (Hr[e] == mx ? corr : 0.0f);
  }
}

// sk_bwd_group with the per-iteration state in registers: one element per
// lane (NP <= 8) and iters <= ITMAX, loops fully unrolled and predicated on
// the uniform iteration count.  Same arithmetic, same results.
template <int NP, int ITMAX>
MHC_DEV void sk_bwd_group_reg(const float* __restrict__ H, const float* __restrict__ dM,
                              float* __restrict__ dlogits, bool mvalid, int n, int iters, float eps, int lane) {
  using L = SkLayout<NP>;
  static_assert(L::E == 1, "register state holds one element per lane");
  const int lm = lane % L::G;
  const int r = lm / L::LR;
  const int c0 = lm % L::LR;
  const bool rvalid = mvalid && r < n;
  const bool v = rvalid && c0 < n;
  const bool cv = mvalid && c0 < n;
  const float Hr = v ? H[(int64_t)r * n + c0] : -INFINITY;
  const float mx = group_max<L::LR>(Hr);
  const float K = v ? expf(Hr - mx) : 0.0f;
  float rs_[ITMAX], R_[ITMAX], cs_[ITMAX], C_[ITMAX];
  float P = K, Rc = 1.0f, Cc = 1.0f;
#pragma unroll
  for (int it = 0; it < ITMAX; ++it) {
    if (it < iters) {
      const float s = group_sum<L::LR>(P);
      const float rsc = (rvalid && s > eps) ? sk_rcp(s) : 1.0f;
      P *= rsc;
      Rc *= rsc;
      rs_[it] = s;
      R_[it] = Rc;
      const float cs = strided_sum<L::LR, L::G>(P);
      const float csc = (cv && cs > eps) ? sk_rcp(cs) : 0.0f;
      P *= csc;
      Cc *= csc;
      cs_[it] = cs;
      C_[it] = Cc;
    }
  }
  float Gd = v ? dM[(int64_t)r * n + c0] : 0.0f;
#pragma unroll
  for (int it = ITMAX - 1; it >= 0; --it) {
    if (it < iters) {
      const float Rk = R_[it];
      const float Rp = it > 0 ? R_[it > 0 ? it - 1 : 0] : 1.0f;
      const float Cp = it > 0 ? C_[it > 0 ? it - 1 : 0] : 1.0f;
      const float dotc = strided_sum<L::LR, L::G>(Gd * (Rk * K * Cp));
      if (cv && cs_[it] > eps) {
        const float sc = sk_rcp(cs_[it]);
        Gd = sc * Gd - sc * sc * dotc;
      } else {
        Gd = 0.0f;
      }
      const float dotr = group_sum<L::LR>(Gd * (Rp * K * Cp));
      if (rvalid && rs_[it] > eps) {
        const float sc = sk_rcp(rs_[it]);
        Gd = sc * Gd - sc * sc * dotr;
      }
    }
  }
  const float dsh = v ? Gd * K : 0.0f;
  const float tot = group_sum<L::LR>(dsh);
  const float cnt = group_sum<L::LR>((v && Hr == mx) ? 1.0f : 0.0f);
  if (v) {
    const float corr = cnt > 0.0f ? tot / cnt : 0.0f;
    dlogits[(int64_t)r * n + c0] = dsh - (Hr == mx ? corr : 0.0f);
  }
}

// ---------------------------------------------------------------------------
// Block layout: one NP x NP matrix per wavefront, NP in {32, 64}.  Lane
// (R = lane >> 3, Q = lane & 7) holds the B x B block (B = NP / 8) at rows
// R*B .. R*B+B-1 and columns Q*B .. Q*B+B-1.  A row sum adds B values in the
// lane and then the 8 lanes of R (lane ^ 1, 2, 4: DPP); a column sum adds B
// values in the lane and then the 8 lanes of Q (lane ^ 8: DPP, lane ^ 16 and
// ^ 32: permlane swaps).  Per iteration that is 3B + 3B cross-lane steps,
// against 5 per element for the one-row-per-lane-pair layout of SkLayout
// (NP = 32: 24 against 80), which bounds a single matrix's latency.
// Same semantics and arithmetic per element as sk_fwd_group; only the
// association of each row or column sum differs.
//
// VJP state, per iteration k (6 * NP floats, each entry a multiple of 16
// bytes from the start of the matrix's state):
//   [0]   R_k     cumulative row scale after the row step
//   [1]   C_k-1   cumulative column scale before the column step
//   [2]   rsc_k   row scale applied (1 for a masked row)
//   [3]   rf_k    R_k-1 * rsc_k^2 (0 for a masked row)
//   [4]   csc_k   column scale applied (0 for a masked column)
//   [5]   cf_k    C_k-1 * csc_k^2 (0 for a masked column)
// A masked row or column is one past n or whose sum is <= eps.  With these
// the VJP of iteration k needs no reciprocal and no mask test.
// ---------------------------------------------------------------------------

constexpr int kSkBlkStateVecs = 6;

__host__ __device__ inline int64_t sk_blk_state_floats(int np, int iters) {
  return (int64_t)kSkBlkStateVecs * np * (iters > 0 ? iters : 1);
}

// B contiguous floats of a 16-byte aligned state row.
template <int B>
MHC_DEV void sk_blk_st_store(float* p, const float (&v)[B]) {
#pragma unroll
  for (int i = 0; i < B; i += 4)
    *reinterpret_cast<float4*>(p + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
}

template <int B>
MHC_DEV void sk_blk_st_load(const float* p, float (&v)[B]) {
#pragma unroll
  for (int i = 0; i < B; i += 4) {
    const float4 t = *reinterpret_cast<const float4*>(p + i);
    v[i] = t.x;
    v[i + 1] = t.y;
    v[i + 2] = t.z;
    v[i + 3] = t.w;
  }
}

// exp(H - rowmax) of the lane's block (0 outside the matrix); with TIE, also
// the mask of elements at their row's maximum (bit a*B+b).  Reads are
// in-bounds for every lane (index 0 for padding elements), then selected.
template <int NP, bool TIE>
MHC_DEV uint64_t sk_blk_load_exp(const float* __restrict__ H, int n, int lane, float (&K)[NP / 8][NP / 8]) {
  constexpr int B = NP / 8;
  const int r0 = (lane >> 3) * B, c0 = (lane & 7) * B;
  uint64_t tie = 0;
#pragma unroll
  for (int a = 0; a < B; ++a) {
    float hv[B];
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const bool v = r0 + a < n && c0 + b < n;
      const float h = H[v ? (r0 + a) * n + c0 + b : 0];
      hv[b] = v ? h : -INFINITY;
      mx = fmaxf(mx, hv[b]);
    }
    mx = group_max<8>(mx);
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const bool v = r0 + a < n && c0 + b < n;
      K[a][b] = v ? expf(hv[b] - mx) : 0.0f;
      if (TIE && v && hv[b] == mx) tie |= (uint64_t)1 << (a * B + b);
    }
  }
  return tie;
}

// `iters` Sinkhorn iterations on the lane's block P.  With REC, iteration k's
// state goes to st + k * 6 * NP (16-byte aligned).  Every lane writes the
// entries of its own rows and columns (the lanes sharing a row or column
// write the same values), so a lane that reads the state back reads only
// what it wrote itself.
template <int NP, bool REC>
MHC_DEV void sk_blk_iterate(float (&P)[NP / 8][NP / 8], int n, int iters, float eps, int lane, float* st) {
  constexpr int B = NP / 8;
  const int r0 = (lane >> 3) * B, c0 = (lane & 7) * B;
  float Rc[B], Cc[B];
#pragma unroll
  for (int a = 0; a < B; ++a) Rc[a] = Cc[a] = 1.0f;
  for (int it = 0; it < iters; ++it) {
    float rsc[B], rf[B], csc[B], cf[B], Cp[B];
#pragma unroll
    for (int a = 0; a < B; ++a) {
      float s = P[a][0];
#pragma unroll
      for (int b = 1; b < B; ++b) s += P[a][b];
      s = group_sum<8>(s);
      const bool ok = r0 + a < n && s > eps;
      rsc[a] = ok ? sk_rcp(s) : 1.0f;
#pragma unroll
      for (int b = 0; b < B; ++b) P[a][b] *= rsc[a];
      if (REC) {
        rf[a] = ok ? Rc[a] * rsc[a] * rsc[a] : 0.0f;
        Rc[a] *= rsc[a];
      }
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
      float cs = P[0][b];
#pragma unroll
      for (int a = 1; a < B; ++a) cs += P[a][b];
      cs = strided_sum<8, 64>(cs);
      const bool ok = c0 + b < n && cs > eps;
      csc[b] = ok ? sk_rcp(cs) : 0.0f;
#pragma unroll
      for (int a = 0; a < B; ++a) P[a][b] *= csc[b];
      if (REC) {
        Cp[b] = Cc[b];
        cf[b] = ok ? Cc[b] * csc[b] * csc[b] : 0.0f;
        Cc[b] *= csc[b];
      }
    }
    if (REC) {
      float* sti = st + (int64_t)it * kSkBlkStateVecs * NP;
      sk_blk_st_store<B>(sti + r0, Rc);
      sk_blk_st_store<B>(sti + NP + c0, Cp);
      sk_blk_st_store<B>(sti + 2 * NP + r0, rsc);
      sk_blk_st_store<B>(sti + 3 * NP + r0, rf);
      sk_blk_st_store<B>(sti + 4 * NP + c0, csc);
      sk_blk_st_store<B>(sti + 5 * NP + c0, cf);
    }
  }
}

// Forward of one matrix; with REC the VJP state also goes to st.
template <int NP, bool REC>
MHC_DEV void sk_fwd_blk(const float* __restrict__ H, float* __restrict__ out, int n, int iters, float eps,
                        int lane, float* st) {
  constexpr int B = NP / 8;
  const int r0 = (lane >> 3) * B, c0 = (lane & 7) * B;
  float P[B][B];
  sk_blk_load_exp<NP, false>(H, n, lane, P);
  sk_blk_iterate<NP, REC>(P, n, iters, eps, lane, st);
#pragma unroll
  for (int a = 0; a < B; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (r0 + a < n && c0 + b < n) out[(r0 + a) * n + c0 + b] = P[a][b];
}

// One reverse-sweep iteration's state for this lane's rows and columns.
template <int B>
struct SkBlkRev {
  float Rk[B], Cp[B], rsc[B], rf[B], csc[B], cf[B];
};

template <int NP, int B>
MHC_DEV void sk_blk_rev_load(const float* st, int it, int r0, int c0, SkBlkRev<B>& s) {
  const float* sti = st + (int64_t)it * kSkBlkStateVecs * NP;
  sk_blk_st_load<B>(sti + r0, s.Rk);
  sk_blk_st_load<B>(sti + NP + c0, s.Cp);
  sk_blk_st_load<B>(sti + 2 * NP + r0, s.rsc);
  sk_blk_st_load<B>(sti + 3 * NP + r0, s.rf);
  sk_blk_st_load<B>(sti + 4 * NP + c0, s.csc);
  sk_blk_st_load<B>(sti + 5 * NP + c0, s.cf);
}

// VJP of one Sinkhorn iteration (column step, then row step) on the lane's
// block Gd.  Column step, input R_k K C_k-1:
//   Gd = csc Gd - cf * sum_rows(Gd K R_k);
// row step, input R_k-1 K C_k-1:
//   Gd = rsc Gd - rf * sum_cols(Gd K C_k-1).
template <int B>
MHC_DEV void sk_blk_rev_step(float (&Gd)[B][B], const float (&K)[B][B], const SkBlkRev<B>& s) {
  float GK[B][B];
#pragma unroll
  for (int a = 0; a < B; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) GK[a][b] = Gd[a][b] * K[a][b];
#pragma unroll
  for (int b = 0; b < B; ++b) {
    float dot = GK[0][b] * s.Rk[0];
#pragma unroll
    for (int a = 1; a < B; ++a) dot += GK[a][b] * s.Rk[a];
    const float sub = strided_sum<8, 64>(dot) * s.cf[b];
#pragma unroll
    for (int a = 0; a < B; ++a) Gd[a][b] = s.csc[b] * Gd[a][b] - sub;
  }
#pragma unroll
  for (int a = 0; a < B; ++a) {
    float KC[B];
#pragma unroll
    for (int b = 0; b < B; ++b) KC[b] = K[a][b] * s.Cp[b];
    float dot = Gd[a][0] * KC[0];
#pragma unroll
    for (int b = 1; b < B; ++b) dot += Gd[a][b] * KC[b];
    const float sub = group_sum<8>(dot) * s.rf[a];
#pragma unroll
    for (int b = 0; b < B; ++b) Gd[a][b] = s.rsc[a] * Gd[a][b] - sub;
  }
}

// VJP of sk_fwd_blk: dH = d/dH <dM, SK(H)>.  st holds the matrix's state
// (recorded by the forward, or written here first when RECOMPUTE).  The
// reverse sweep reads each iteration's state one iteration ahead, into two
// alternating sets, so the reads are in flight during the previous
// iteration's arithmetic.
template <int NP, bool RECOMPUTE>
MHC_DEV void sk_bwd_blk(const float* __restrict__ H, const float* __restrict__ dM, float* __restrict__ dH, int n,
                        int iters, float eps, float* st, int lane) {
  constexpr int B = NP / 8;
  static_assert(B * B <= 64, "tie mask holds one bit per element");
  const int r0 = (lane >> 3) * B, c0 = (lane & 7) * B;
  float K[B][B], Gd[B][B];
  const uint64_t tie = sk_blk_load_exp<NP, true>(H, n, lane, K);  // bit a*B+b: H at the row maximum
  if (RECOMPUTE) {
#pragma unroll
    for (int a = 0; a < B; ++a)
#pragma unroll
      for (int b = 0; b < B; ++b) Gd[a][b] = K[a][b];
    sk_blk_iterate<NP, true>(Gd, n, iters, eps, lane, st);
  }
#pragma unroll
  for (int a = 0; a < B; ++a)
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const bool v = r0 + a < n && c0 + b < n;
      const float g = dM[v ? (r0 + a) * n + c0 + b : 0];
      Gd[a][b] = v ? g : 0.0f;
    }
  if (iters > 0) {
    SkBlkRev<B> sa, sb;
    sk_blk_rev_load<NP>(st, iters - 1, r0, c0, sa);
    int it = iters - 1;
    for (; it >= 1; it -= 2) {
      sk_blk_rev_load<NP>(st, it - 1, r0, c0, sb);
      sk_blk_rev_step<B>(Gd, K, sa);
      sk_blk_rev_load<NP>(st, it >= 2 ? it - 2 : 0, r0, c0, sa);
      sk_blk_rev_step<B>(Gd, K, sb);
    }
    if (it == 0) sk_blk_rev_step<B>(Gd, K, sa);
  }
  // through exp and the row-max shift (the gradient of the max split evenly
  // among tied maxima; it is zero in exact arithmetic)
#pragma unroll
  for (int a = 0; a < B; ++a) {
    float tot = 0.0f, cnt = 0.0f;
#pragma unroll
    for (int b = 0; b < B; ++b) {
      Gd[a][b] *= K[a][b];  // K is 0 outside the matrix
      tot += Gd[a][b];
      cnt += (tie >> (a * B + b)) & 1 ? 1.0f : 0.0f;
    }
    tot = group_sum<8>(tot);
    cnt = group_sum<8>(cnt);
    const float corr = cnt > 0.0f ? tot / cnt : 0.0f;
#pragma unroll
    for (int b = 0; b < B; ++b)
      if (r0 + a < n && c0 + b < n)
        dH[(r0 + a) * n + c0 + b] = Gd[a][b] - ((tie >> (a * B + b)) & 1 ? corr : 0.0f);
  }
}

}  // namespace mhc
