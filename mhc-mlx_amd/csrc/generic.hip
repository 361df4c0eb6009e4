// Runtime-n kernels for 16 < n <= 64 (the reference allows n up to 64:
// metal.py:71).  Compact code with runtime loops over streams; one workgroup
// per token (persistent), threads over channels.  The register-tiled kernels
// in fused_fwd.hip / fused_bwd.hip / stream_mix.hip cover n <= 16.
#include "mhc_device.hpp"
#include "mhc_generic.hpp"
#include "mhc_host.hpp"
#include "mhc_plan.hpp"
#include "mhc_reduce.hpp"

namespace mhc {

namespace {

constexpr int kGenThreads = 256;
constexpr int kGenMaxPar = MHC_MAX_N * MHC_MAX_N + 2 * MHC_MAX_N;

// params for token t: M [n*n], a [n], p [n] (activated), compact n-indexing
MHC_DEV void gen_stage(float* s, const float* M, const float* hp, const float* hq, int n,
                       int h_mode) {
  const int nn = n * n;
  for (int k = threadIdx.x; k < nn + 2 * n; k += blockDim.x) {
    float v;
    if (k < nn) {
      v = M ? M[k] : 0.0f;
    } else if (k < nn + n) {
      const int i = k - nn;
      v = h_mode == MHC_H_NONE ? 1.0f : (h_mode == MHC_H_RAW ? sigmoidf_(hp[i]) : hp[i]);
    } else {
      const int i = k - nn - n;
      v = h_mode == MHC_H_NONE ? 1.0f : (h_mode == MHC_H_RAW ? 2.0f * sigmoidf_(hq[i]) : hq[i]);
    }
    s[k] = v;
  }
}

MHC_DEV float gen_block_sum(float v, float* s_red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  if (lane == 0) s_red[wave] = v;
  __syncthreads();
  float t = 0.0f;
  for (int w = 0; w < nw; ++w) t += s_red[w];
  return t;
}

template <typename XT, typename OT>
__global__ __launch_bounds__(kGenThreads) void gen_fwd_kernel(GenArgs A) {
  __shared__ float s_par[kGenMaxPar];
  __shared__ float s_red[2][kGenThreads / 64];
  const int n = A.n, C = A.C, nn = n * n;
  const XT* X = (const XT*)A.x;
  OT* O = (OT*)A.out;
  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    __syncthreads();  // previous token done with s_par
    gen_stage(s_par, A.M + t * A.M_ts, A.hpre + t * A.h_ts, A.hpost + t * A.h_ts, n, A.h_mode);
    __syncthreads();
    const XT* xt = X + t * n * C;
    OT* ot = O + t * n * C;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
      float y = 0.0f;
      for (int i = 0; i < n; ++i) y = fmaf(s_par[nn + i], load1<XT>(xt + (int64_t)i * C + c), y);
      ss = fmaf(y, y, ss);
    }
    const float tot = gen_block_sum(ss, s_red[it & 1]);
    const float inv = 1.0f / sqrtf(tot / (float)C + A.eps);
    if (A.inv_rms && threadIdx.x == 0) A.inv_rms[t] = inv;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
      float y = 0.0f;
      for (int i = 0; i < n; ++i) y = fmaf(s_par[nn + i], load1<XT>(xt + (int64_t)i * C + c), y);
      const float yn = (y * inv) * A.w[c];
      for (int i = 0; i < n; ++i) {
        float acc = 0.0f;
        for (int j = 0; j < n; ++j) acc = fmaf(s_par[i * n + j], load1<XT>(xt + (int64_t)j * C + c), acc);
        store1<OT>(ot + (int64_t)i * C + c, fmaf(yn, s_par[nn + n + i], acc));
      }
    }
  }
}

// Backward.  Per token: dy/yn go to this workgroup's scratch rows so the
// parameter-gradient loops (threads over (i, j) pairs, loops over channels)
// can read them.  Layer-wide sums accumulate in LDS slots, each owned by one
// thread; dw accumulates in the workgroup's partial row.
template <typename XT, typename GT>
__global__ __launch_bounds__(kGenThreads) void gen_bwd_kernel(GenArgs A) {
  __shared__ float s_par[kGenMaxPar];
  __shared__ float s_acc[kGenMaxPar];
  __shared__ float s_red[2][2][kGenThreads / 64];
  const int n = A.n, C = A.C, nn = n * n, K = nn + 2 * n;
  const XT* X = (const XT*)A.x;
  const GT* Gd = (const GT*)A.g;
  XT* DX = (XT*)A.out;
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  float* sdy = A.scratch + (int64_t)blockIdx.x * 2 * A.C;
  float* syn = sdy + A.C;
  for (int c = threadIdx.x; c < A.P; c += blockDim.x) prow[c] = 0.0f;
  for (int k = threadIdx.x; k < K; k += blockDim.x) s_acc[k] = 0.0f;
  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    __syncthreads();
    gen_stage(s_par, A.M + t * A.M_ts, A.hpre + t * A.h_ts, A.hpost + t * A.h_ts, n, A.h_mode);
    __syncthreads();
    const XT* xt = X + t * n * C;
    const GT* gt = Gd + t * n * C;
    XT* dxt = DX + t * n * C;
    float ss = 0.0f, sr = 0.0f;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
      float y = 0.0f, d = 0.0f;
      for (int i = 0; i < n; ++i) {
        y = fmaf(s_par[nn + i], load1<XT>(xt + (int64_t)i * C + c), y);
        d = fmaf(s_par[nn + n + i], load1<GT>(gt + (int64_t)i * C + c), d);
      }
      ss = fmaf(y, y, ss);
      sr = fmaf(d * y, A.w[c], sr);
    }
    const float tss = gen_block_sum(ss, s_red[it & 1][0]);
    const float tsr = gen_block_sum(sr, s_red[it & 1][1]);
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
      float y = 0.0f, d = 0.0f;
      for (int i = 0; i < n; ++i) {
        y = fmaf(s_par[nn + i], load1<XT>(xt + (int64_t)i * C + c), y);
        d = fmaf(s_par[nn + n + i], load1<GT>(gt + (int64_t)i * C + c), d);
      }
      const float wc = A.w[c];
      const float yi = y * inv;
      const float dy = d * inv * wc - kf * y;
      sdy[c] = dy;
      syn[c] = yi * wc;
      prow[c] = fmaf(d, yi, prow[c]);
      for (int j = 0; j < n; ++j) {
        float acc = 0.0f;
        for (int i = 0; i < n; ++i) acc = fmaf(s_par[i * n + j], load1<GT>(gt + (int64_t)i * C + c), acc);
        store1<XT>(dxt + (int64_t)j * C + c, fmaf(s_par[nn + j], dy, acc));
      }
    }
    __syncthreads();  // sdy / syn visible to the workgroup
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
      float s = 0.0f;
      if (k < nn) {
        const int i = k / n, j = k % n;
        for (int c = 0; c < C; ++c)
          s = fmaf(load1<GT>(gt + (int64_t)i * C + c), load1<XT>(xt + (int64_t)j * C + c), s);
      } else if (k < nn + n) {
        const int j = k - nn;
        for (int c = 0; c < C; ++c) s = fmaf(sdy[c], load1<XT>(xt + (int64_t)j * C + c), s);
      } else {
        const int i = k - nn - n;
        for (int c = 0; c < C; ++c) s = fmaf(load1<GT>(gt + (int64_t)i * C + c), syn[c], s);
      }
      if (A.M_ts) {
        if (k < nn) {
          A.dM_tok[t * nn + k] = s;
        } else if (k < nn + n) {
          const float av = s_par[k];
          A.dpre_tok[t * n + (k - nn)] = A.h_mode == MHC_H_RAW ? s * av * (1.0f - av) : s;
        } else {
          const float pq = s_par[k];
          A.dpost_tok[t * n + (k - nn - n)] = A.h_mode == MHC_H_RAW ? s * pq * (1.0f - 0.5f * pq) : s;
        }
      } else {
        s_acc[k] += s;
      }
    }
  }
  __syncthreads();
  if (!A.M_ts)
    for (int k = threadIdx.x; k < K; k += blockDim.x) prow[A.Cp + k] = s_acc[k];
}

// post-combine / stream_mix_add forward: out_i = p_i (y_i + sum_j M_ij a_j x_j)
template <typename XT, typename YT, typename OT>
__global__ __launch_bounds__(kGenThreads) void gen_mix_fwd_kernel(GenArgs A) {
  __shared__ float s_par[kGenMaxPar];
  const int n = A.n, C = A.C, nn = n * n;
  gen_stage(s_par, A.M, A.hpre, A.hpost, n, A.h_mode);
  __syncthreads();
  const XT* X = (const XT*)A.x;
  const YT* Y = (const YT*)A.y;
  OT* O = (OT*)A.out;
  const int64_t items = A.T * C;
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = item / C;
    const int c = (int)(item - t * C);
    const int64_t base = t * n * C + c;
    for (int i = 0; i < n; ++i) {
      float acc = 0.0f;
      for (int j = 0; j < n; ++j)
        acc = fmaf(s_par[i * n + j] * s_par[nn + j], load1<XT>(X + base + (int64_t)j * C), acc);
      const float yv = Y ? load1<YT>(Y + base + (int64_t)i * C) : 0.0f;
      store1<OT>(O + base + (int64_t)i * C, s_par[nn + n + i] * (yv + acc));
    }
  }
}

// post-combine VJP: dx_j = a_j sum_i M_ij p_i g_i, dy_i = p_i g_i and the
// sums S_ij = sum g_i x_j, Yd_i = sum g_i y_i (one partial row per workgroup).
template <typename XT, typename YT, typename GT>
__global__ __launch_bounds__(kGenThreads) void gen_mix_bwd_kernel(GenArgs A) {
  __shared__ float s_par[kGenMaxPar];
  __shared__ float s_acc[MHC_MAX_N * MHC_MAX_N + MHC_MAX_N];
  const int n = A.n, C = A.C, nn = n * n, K = nn + n;
  gen_stage(s_par, A.M, A.hpre, A.hpost, n, A.h_mode);
  for (int k = threadIdx.x; k < K; k += blockDim.x) s_acc[k] = 0.0f;
  __syncthreads();
  const XT* X = (const XT*)A.x;
  const YT* Y = (const YT*)A.y;
  const GT* Gd = (const GT*)A.g;
  XT* DX = (XT*)A.out;
  YT* DY = (YT*)A.dy;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x) {
    const int64_t tb = t * n * C;
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
      for (int j = 0; j < n; ++j) {
        float acc = 0.0f;
        for (int i = 0; i < n; ++i)
          acc = fmaf(s_par[nn + n + i] * s_par[i * n + j], load1<GT>(Gd + tb + (int64_t)i * C + c), acc);
        store1<XT>(DX + tb + (int64_t)j * C + c, s_par[nn + j] * acc);
        if (DY) store1<YT>(DY + tb + (int64_t)j * C + c, s_par[nn + n + j] * load1<GT>(Gd + tb + (int64_t)j * C + c));
      }
    }
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
      float s = 0.0f;
      if (k < nn) {
        const int i = k / n, j = k % n;
        for (int c = 0; c < C; ++c)
          s = fmaf(load1<GT>(Gd + tb + (int64_t)i * C + c), load1<XT>(X + tb + (int64_t)j * C + c), s);
      } else if (Y) {
        const int i = k - nn;
        for (int c = 0; c < C; ++c)
          s = fmaf(load1<GT>(Gd + tb + (int64_t)i * C + c), load1<YT>(Y + tb + (int64_t)i * C + c), s);
      }
      s_acc[k] += s;
    }
  }
  __syncthreads();
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  for (int k = threadIdx.x; k < A.P; k += blockDim.x) prow[k] = k < K ? s_acc[k] : 0.0f;
}

template <typename F>
int by_x_dtype(int code, F&& f) {
  switch (code) {
    case MHC_DTYPE_F32: return f((float*)nullptr);
    case MHC_DTYPE_BF16: return f((__bf16*)nullptr);
    case MHC_DTYPE_F16: return f((_Float16*)nullptr);
    default: return set_error(MHC_ERR_INVALID_ARG, "unknown dtype code %d", code);
  }
}

// second dtype is either fp32 or the first one
template <typename T1, typename F>
int by_pair(int code2, F&& f) {
  if (code2 == MHC_DTYPE_F32) return f((float*)nullptr);
  if ((code2 == MHC_DTYPE_BF16 && std::is_same<T1, __bf16>::value) ||
      (code2 == MHC_DTYPE_F16 && std::is_same<T1, _Float16>::value))
    return f((T1*)nullptr);
  return set_error(MHC_ERR_INVALID_ARG, "unsupported dtype combination (second dtype %d)", code2);
}

}  // namespace

int64_t gen_grid(int64_t T) {
  return std::max<int64_t>(1, std::min<int64_t>(T, (int64_t)device_cu_count() * 8));
}

int gen_fused_fwd(const GenArgs& A, int xd, int od, hipStream_t s) {
  const int64_t blocks = gen_grid(A.T);
  return by_x_dtype(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return by_pair<XT>(od, [&](auto* op) {
      using OT = std::remove_pointer_t<decltype(op)>;
      hipLaunchKernelGGL((gen_fwd_kernel<XT, OT>), dim3((unsigned)blocks), dim3(kGenThreads), 0, s, A);
      MHC_CHECK_LAUNCH("gen_fwd_kernel");
      return MHC_OK;
    });
  });
}

int gen_fused_bwd(const GenArgs& A, int xd, int gd, hipStream_t s, int64_t* num_partials) {
  const int64_t blocks = gen_grid(A.T);
  *num_partials = blocks;
  return by_x_dtype(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return by_pair<XT>(gd, [&](auto* gp) {
      using GT = std::remove_pointer_t<decltype(gp)>;
      hipLaunchKernelGGL((gen_bwd_kernel<XT, GT>), dim3((unsigned)blocks), dim3(kGenThreads), 0, s, A);
      MHC_CHECK_LAUNCH("gen_bwd_kernel");
      return MHC_OK;
    });
  });
}

int gen_mix_fwd(const GenArgs& A, int xd, int yd, int od, hipStream_t s) {
  const int64_t blocks = std::max<int64_t>(
      1, std::min<int64_t>(ceil_div(A.T * A.C, kGenThreads), (int64_t)device_cu_count() * 8));
  return by_x_dtype(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return by_pair<XT>(yd, [&](auto* yp) {
      using YT = std::remove_pointer_t<decltype(yp)>;
      return by_pair<XT>(od, [&](auto* op) {
        using OT = std::remove_pointer_t<decltype(op)>;
        hipLaunchKernelGGL((gen_mix_fwd_kernel<XT, YT, OT>), dim3((unsigned)blocks), dim3(kGenThreads), 0,
                           s, A);
        MHC_CHECK_LAUNCH("gen_mix_fwd_kernel");
        return MHC_OK;
      });
    });
  });
}

int gen_mix_bwd(const GenArgs& A, int xd, int yd, int gd, hipStream_t s, int64_t blocks) {
  return by_x_dtype(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return by_pair<XT>(yd, [&](auto* yp) {
      using YT = std::remove_pointer_t<decltype(yp)>;
      return by_pair<XT>(gd, [&](auto* gp) {
        using GT = std::remove_pointer_t<decltype(gp)>;
        hipLaunchKernelGGL((gen_mix_bwd_kernel<XT, YT, GT>), dim3((unsigned)blocks), dim3(kGenThreads), 0,
                           s, A);
        MHC_CHECK_LAUNCH("gen_mix_bwd_kernel");
        return MHC_OK;
      });
    });
  });
}

}  // namespace mhc
