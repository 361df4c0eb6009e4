// Batched Sinkhorn-Knopp projection and its VJP (one wavefront per group of
// matrices; see mhc_sinkhorn.hpp for the lane layout and the semantics of
// mhc_mlx/reference.py:20-48, 58-69 that they follow).
#include "mhc_device.hpp"
#include "mhc_host.hpp"
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
