// Batched Sinkhorn-Knopp projection and its VJP (one wavefront per matrix).
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
// Row sums are butterflies over LR adjacent lanes, column sums butterflies
// over lanes LR apart; all `iters` rounds stay in registers.
//
// The VJP recomputes the forward and records, per iteration, the row and
// column sums and the cumulative row/column scale vectors R_k, C_k
// (4 * iters * NP floats per matrix, in LDS when it fits, else in the
// caller's workspace).  The pre-step matrices are rebuilt as R K C, which
// stays exact for masked (zeroed) columns, unlike dividing the scaled
// matrix by its scale.
#include "mhc_device.hpp"
#include "mhc_host.hpp"

namespace mhc {

template <int NP>
struct SkLayout {
  static constexpr int E = NP * NP >= 64 ? NP * NP / 64 : 1;
  static constexpr int LR = NP / E;
  static constexpr int G = NP * LR;
  static constexpr int MPW = 64 / G;
  static constexpr int W = MPW * NP;  // row (or column) slots per wavefront
};

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
  const int lm = lane % L::G;
  const int msub = lane / L::G;
  const int r = lm / L::LR;
  const int c0 = (lm % L::LR) * L::E;
  const int64_t ngroups = (batch + L::MPW - 1) / L::MPW;
  const int64_t nn = (int64_t)n * n;

  for (int64_t grp = (int64_t)blockIdx.x * wpb + wave; grp < ngroups;
       grp += (int64_t)gridDim.x * wpb) {
    const int64_t mat = grp * L::MPW + msub;
    const bool mvalid = mat < batch;
    const bool rvalid = mvalid && r < n;
    const float* H = logits + mat * nn + (int64_t)r * n;
    float P[L::E];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < L::E; ++e) {
      const bool v = rvalid && (c0 + e) < n;
      P[e] = v ? H[c0 + e] : -INFINITY;
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
      const float rsc = (rvalid && s > eps) ? 1.0f / s : 1.0f;
#pragma unroll
      for (int e = 0; e < L::E; ++e) P[e] *= rsc;
#pragma unroll
      for (int e = 0; e < L::E; ++e) {
        const float cs = strided_sum<L::LR, L::G>(P[e]);
        const bool cv = mvalid && (c0 + e) < n;
        const float csc = (cv && cs > eps) ? 1.0f / cs : 0.0f;
        P[e] *= csc;
      }
    }
    if (rvalid) {
      float* O = out + mat * nn + (int64_t)r * n;
#pragma unroll
      for (int e = 0; e < L::E; ++e)
        if ((c0 + e) < n) O[c0 + e] = P[e];
    }
  }
}

// state layout per wavefront: [4][iters][W]
//   0: row sums, 1: cumulative row scale R_k, 2: column sums, 3: cumulative column scale C_k
template <int NP, bool GLOBAL_STATE>
__global__ __launch_bounds__(kSkThreads) void sinkhorn_bwd_kernel(
    const float* __restrict__ logits, const float* __restrict__ dM, float* __restrict__ dlogits,
    int64_t batch, int n, int iters, float eps, float* __restrict__ gstate) {
  using L = SkLayout<NP>;
  extern __shared__ float sk_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wpb = blockDim.x >> 6;
  const int lm = lane % L::G;
  const int msub = lane / L::G;
  const int r = lm / L::LR;
  const int c0 = (lm % L::LR) * L::E;
  const int64_t ngroups = (batch + L::MPW - 1) / L::MPW;
  const int64_t nn = (int64_t)n * n;
  const int64_t per_wave = (int64_t)4 * iters * L::W;
  float* st;
  if constexpr (GLOBAL_STATE) {
    st = gstate + ((int64_t)blockIdx.x * wpb + wave) * per_wave;
  } else {
    st = sk_smem + (int64_t)wave * per_wave;
  }
  float* st_rs = st;
  float* st_R = st + (int64_t)iters * L::W;
  float* st_cs = st + (int64_t)2 * iters * L::W;
  float* st_C = st + (int64_t)3 * iters * L::W;
  const int rslot = msub * NP + r;
  const int cslot = msub * NP + c0;

  for (int64_t grp = (int64_t)blockIdx.x * wpb + wave; grp < ngroups;
       grp += (int64_t)gridDim.x * wpb) {
    const int64_t mat = grp * L::MPW + msub;
    const bool mvalid = mat < batch;
    const bool rvalid = mvalid && r < n;
    const float* H = logits + mat * nn + (int64_t)r * n;
    float Hr[L::E], K[L::E], P[L::E];
    float mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < L::E; ++e) {
      const bool v = rvalid && (c0 + e) < n;
      Hr[e] = v ? H[c0 + e] : -INFINITY;
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
      const float rsc = (rvalid && s > eps) ? 1.0f / s : 1.0f;
#pragma unroll
      for (int e = 0; e < L::E; ++e) P[e] *= rsc;
      Rc *= rsc;
      st_rs[(int64_t)it * L::W + rslot] = s;
      st_R[(int64_t)it * L::W + rslot] = Rc;
#pragma unroll
      for (int e = 0; e < L::E; ++e) {
        const float cs = strided_sum<L::LR, L::G>(P[e]);
        const bool cv = mvalid && (c0 + e) < n;
        const float csc = (cv && cs > eps) ? 1.0f / cs : 0.0f;
        P[e] *= csc;
        Cc[e] *= csc;
        st_cs[(int64_t)it * L::W + cslot + e] = cs;
        st_C[(int64_t)it * L::W + cslot + e] = Cc[e];
      }
    }
    // reverse sweep
    float Gd[L::E];
    {
      const float* D = dM + mat * nn + (int64_t)r * n;
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
      for (int e = 0; e < L::E; ++e)
        Cp[e] = it > 0 ? st_C[(int64_t)(it - 1) * L::W + cslot + e] : 1.0f;
      // column step: input R_k K C_{k-1}
#pragma unroll
      for (int e = 0; e < L::E; ++e) {
        const float pin = Rk * K[e] * Cp[e];
        const float dot = strided_sum<L::LR, L::G>(Gd[e] * pin);
        const float cs = st_cs[(int64_t)it * L::W + cslot + e];
        const bool cv = mvalid && (c0 + e) < n;
        if (cv && cs > eps) {
          const float sc = 1.0f / cs;
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
        const float sc = 1.0f / rs;
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
      float* O = dlogits + mat * nn + (int64_t)r * n;
      const float corr = cnt > 0.0f ? tot / cnt : 0.0f;
#pragma unroll
      for (int e = 0; e < L::E; ++e)
        if ((c0 + e) < n) O[c0 + e] = dsh[e] - (Hr[e] == mx ? corr : 0.0f);
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

namespace {

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

extern "C" size_t mhc_sinkhorn_bwd_workspace_bytes(int64_t batch, int n, int iters) {
  if (n < 1 || n > MHC_MAX_N || batch <= 0 || iters < 0) return 0;
  return plan_bwd(batch, n, iters, device_cu_count()).ws_bytes;
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
  const SkPlan p = plan_bwd(batch, n, iters, device_cu_count());
  MHC_CHECK_ARG(workspace_bytes >= p.ws_bytes && (p.ws_bytes == 0 || workspace != nullptr),
                "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes,
                p.ws_bytes);
  float* ws = (float*)workspace;
  hipStream_t s = (hipStream_t)stream;
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
