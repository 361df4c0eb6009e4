// Fused residual add + stream aggregate (mhc_mlx/utils.py:4-24,
// kernels/residual_add_agg.metal:39-66 via metal.py:1673-1731):
//   out[t,i,c] = x[t,i,c] + res[t,i,c]
//   y_agg[t,c] = sum_i a_i (x[t,i,c] + res[t,i,c])      (fp32, from the unrounded sum)
// and its VJP (an extension: the reference kernel has no VJP):
//   d_val_i = dout_i + a_i dy                    dx = dres = d_val
//   dh_pre_i = sum_{t,c} dy (x_i + res_i)
//
// HBM-bound streaming.  Work item = (token, chunk of V = 8 channels) over all
// n streams, one item per thread (grid-stride beyond 2^24 blocks).  The streams are
// visited in groups of G: the group's x and res chunks (2G 16-byte loads for
// 16-bit types) are all issued before the first add, so every thread keeps
// 2G loads in flight.  The backward splits the streams over grid.y (one
// group of 4 per block row) and writes one partial row of dh_pre per block,
// finished by the fixed-order row reduction (deterministic, no atomics).
#include "mhc_device.hpp"
#include "mhc_host.hpp"
#include "mhc_plan.hpp"
#include "mhc_reduce.hpp"

namespace mhc {

namespace {

constexpr int kResThreads = 256;
constexpr int kResV = 8;
constexpr int kResSplit = 64;

struct ResArgs {
  const void* x;
  const void* res;
  const void* g;     // bwd: dout (may be null)
  const float* gy;   // bwd: d y_agg (may be null)
  void* out;         // fwd: out; bwd: dx
  void* out2;        // bwd: dres
  float* y_agg;      // fwd
  const float* hpre;
  float* part;       // bwd partial rows (may be null: no dh_pre)
  int64_t T;
  int n;
  int C;
  int nchunks;
  int h_mode;
  int vec;
  int P;
};

MHC_DEV float act_pre(const ResArgs& A, int i) {
  const float h = A.hpre[i];
  return A.h_mode == MHC_H_RAW ? sigmoidf_(h) : h;
}

template <typename T>
MHC_DEV void load_c(Vec<T, kResV>& r, const T* p, bool vec, int valid) {
  if (vec && valid == kResV) r.load(p);
  else r.load_partial(p, valid);
}

template <typename T>
MHC_DEV void store_c(T* p, const float (&v)[kResV], bool vec, int valid) {
  if (vec && valid == kResV) store_vec<T, kResV, true>(p, v);
  else store_partial<T, kResV>(p, v, valid);
}

template <int G, typename XT, typename OT>
__global__ __launch_bounds__(kResThreads) void residual_add_agg_kernel(ResArgs A) {
  constexpr int V = kResV;
  __shared__ float s_a[MHC_MAX_N];
  for (int i = threadIdx.x; i < A.n; i += blockDim.x) s_a[i] = act_pre(A, i);
  __syncthreads();
  const int n = A.n, C = A.C;
  const int64_t items = A.T * A.nchunks;
  const XT* X = (const XT*)A.x;
  const XT* R = (const XT*)A.res;
  OT* O = (OT*)A.out;
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = item / A.nchunks;
    const int q = (int)(item - t * A.nchunks);
    const int c0 = q * V;
    const int valid = min(V, C - c0);
    const int64_t base = t * n * C + c0;
    float agg[V];
#pragma unroll
    for (int v = 0; v < V; ++v) agg[v] = 0.0f;
    for (int i0 = 0; i0 < n; i0 += G) {
      Vec<XT, V> xr[G], rr[G];
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (i0 + g < n) {
          load_c<XT>(xr[g], X + base + (int64_t)(i0 + g) * C, A.vec, valid);
          load_c<XT>(rr[g], R + base + (int64_t)(i0 + g) * C, A.vec, valid);
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (i0 + g < n) {
          const float a = s_a[i0 + g];
          float o[V];
#pragma unroll
          for (int v = 0; v < V; ++v) {
            o[v] = xr[g].get(v) + rr[g].get(v);
            agg[v] = fmaf(o[v], a, agg[v]);
          }
          store_c<OT>(O + base + (int64_t)(i0 + g) * C, o, A.vec, valid);
        }
      }
    }
    store_c<float>(A.y_agg + t * C + c0, agg, A.vec, valid);
  }
}

// grid.y = stream group (streams [blockIdx.y*G, +G)); block (bx, gy) writes
// columns [gy*G, gy*G+G) of partial row bx.
template <int G, typename XT, typename GT>
__global__ __launch_bounds__(kResThreads) void residual_add_agg_bwd_kernel(ResArgs A) {
  constexpr int V = kResV;
  __shared__ float s_stage[kResThreads / 64][G];
  const int n = A.n, C = A.C;
  const int i0 = blockIdx.y * G;
  float a[G];
#pragma unroll
  for (int g = 0; g < G; ++g) a[g] = (i0 + g < n) ? act_pre(A, i0 + g) : 0.0f;
  const int64_t items = A.T * A.nchunks;
  const XT* X = (const XT*)A.x;
  const XT* R = (const XT*)A.res;
  const GT* Gd = (const GT*)A.g;
  XT* DX = (XT*)A.out;
  XT* DR = (XT*)A.out2;
  const bool want_dh = A.part != nullptr && A.gy != nullptr;
  float acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = 0.0f;
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = item / A.nchunks;
    const int q = (int)(item - t * A.nchunks);
    const int c0 = q * V;
    const int valid = min(V, C - c0);
    const int64_t base = t * n * C + c0;
    Vec<float, V> gyr;
    if (A.gy) load_c<float>(gyr, A.gy + t * C + c0, A.vec, valid);
    else gyr.zero();
    Vec<GT, V> gr[G];
    Vec<XT, V> xr[G], rr[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (i0 + g < n) {
        const int64_t off = base + (int64_t)(i0 + g) * C;
        if (Gd) load_c<GT>(gr[g], Gd + off, A.vec, valid);
        else gr[g].zero();
        if (want_dh) {
          load_c<XT>(xr[g], X + off, A.vec, valid);
          load_c<XT>(rr[g], R + off, A.vec, valid);
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      if (i0 + g < n) {
        const int64_t off = base + (int64_t)(i0 + g) * C;
        float d[V];
#pragma unroll
        for (int v = 0; v < V; ++v) d[v] = fmaf(a[g], gyr.get(v), gr[g].get(v));
        if (DX) store_c<XT>(DX + off, d, A.vec, valid);
        if (DR) store_c<XT>(DR + off, d, A.vec, valid);
        if (want_dh) {
#pragma unroll
          for (int v = 0; v < V; ++v) acc[g] = fmaf(gyr.get(v), xr[g].get(v) + rr[g].get(v), acc[g]);
        }
      }
    }
  }
  if (A.part == nullptr) return;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float s = wave_sum(acc[g]);
    if ((threadIdx.x & 63) == 0) s_stage[threadIdx.x >> 6][g] = s;
  }
  __syncthreads();
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  if (threadIdx.x < G && i0 + (int)threadIdx.x < n) {
    float s = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += s_stage[w][threadIdx.x];
    prow[i0 + threadIdx.x] = s;
  }
  if (blockIdx.y == 0)
    for (int c = n + (int)threadIdx.x; c < A.P; c += blockDim.x) prow[c] = 0.0f;
}

__global__ __launch_bounds__(64) void residual_final_kernel(const float* __restrict__ part2, int S, int P,
                                                            int n, int h_mode,
                                                            const float* __restrict__ hpre,
                                                            float* __restrict__ dpre) {
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    float s = 0.0f;
    for (int k = 0; k < S; ++k) s += part2[(int64_t)k * P + j];
    if (h_mode == MHC_H_RAW) {
      const float a = sigmoidf_(hpre[j]);
      s *= a * (1.0f - a);
    }
    dpre[j] = s;
  }
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------

int res_group(int n) { return n <= 4 ? 4 : 8; }
// The backward holds dout, x and res of a group in registers: groups of 4.
constexpr int kResBwdGroup = 4;

// One item per thread (the grid-stride loop then runs once) measured best on
// MI355X: 646 us at 32768 x 4 x 4096 bf16 (72.7% of 8 TB/s) against 675-700 us
// for persistent grids of 2-32 blocks per CU.  MHC_RES_GRID > 0 caps the grid
// at that many blocks per CU (tuning override).
int64_t res_fwd_grid(int64_t items, int cus) {
  const int64_t g = ceil_div(items, kResThreads);
  const int per_cu = knob(kKnobResGrid, -1);
  if (per_cu < 0) return std::max<int64_t>(1, std::min<int64_t>(g, kMaxGrid));
  return std::max<int64_t>(1, std::min<int64_t>(g, (int64_t)cus * std::max(per_cu, 1)));
}

int64_t res_bwd_grid(int64_t T, int n, int C, int cus) {
  const int64_t groups = ceil_div(n, kResBwdGroup);
  const int64_t g = ceil_div(T * ceil_div(C, kResV), kResThreads);
  return std::max<int64_t>(1, std::min<int64_t>(g, (int64_t)cus * 8 / groups + 1));
}

bool res_vec_ok(int C, std::initializer_list<std::pair<const void*, int>> ptrs) {
  if (C % kResV != 0) return false;
  for (auto& pr : ptrs) {
    if (pr.first == nullptr) continue;
    const int al = std::min(16, kResV * pr.second);
    if (!aligned(pr.first, al)) return false;
  }
  return true;
}

template <typename F>
int res_by_dtype(int code, F&& f) {
  switch (code) {
    case MHC_DTYPE_F32: return f((float*)nullptr);
    case MHC_DTYPE_BF16: return f((__bf16*)nullptr);
    case MHC_DTYPE_F16: return f((_Float16*)nullptr);
    default: return set_error(MHC_ERR_INVALID_ARG, "unknown dtype code %d", code);
  }
}

template <typename F>
int res_by_group(int n, F&& f) {
  if (res_group(n) == 4) return f(std::integral_constant<int, 4>{});
  return f(std::integral_constant<int, 8>{});
}

}  // namespace
}  // namespace mhc

using namespace mhc;

extern "C" int mhc_residual_add_agg_fwd(const void* x, const void* res, int dtype, const float* h_pre,
                                        int h_mode, void* out, int out_dtype, float* y_agg, int64_t T,
                                        int n, int C, void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1 && T >= 0, "invalid T=%lld / C=%d", (long long)T, C);
  MHC_CHECK_ARG(h_mode == MHC_H_ACTIVATED || h_mode == MHC_H_RAW, "invalid h_mode %d", h_mode);
  if (T == 0) return MHC_OK;
  MHC_CHECK_ARG(x && res && h_pre && out && y_agg, "null pointer argument");
  MHC_CHECK_ARG(dtype_bytes(dtype) && dtype_bytes(out_dtype), "unknown dtype code");
  ResArgs A{};
  A.x = x; A.res = res; A.out = out; A.y_agg = y_agg; A.hpre = h_pre; A.T = T; A.n = n; A.C = C;
  A.h_mode = h_mode;
  A.nchunks = (int)ceil_div(C, kResV);
  A.vec = res_vec_ok(C, {{x, dtype_bytes(dtype)}, {res, dtype_bytes(dtype)}, {out, dtype_bytes(out_dtype)},
                         {y_agg, 4}});
  const int64_t blocks = res_fwd_grid(T * A.nchunks, device_cu_count());
  hipStream_t s = (hipStream_t)stream;
  return res_by_group(n, [&](auto gc) {
    constexpr int G = decltype(gc)::value;
    return res_by_dtype(dtype, [&](auto* xp) {
      using XT = std::remove_pointer_t<decltype(xp)>;
      return res_by_dtype(out_dtype, [&](auto* op) {
        using OT = std::remove_pointer_t<decltype(op)>;
        hipLaunchKernelGGL((residual_add_agg_kernel<G, XT, OT>), dim3((unsigned)blocks), dim3(kResThreads),
                           0, s, A);
        MHC_CHECK_LAUNCH("residual_add_agg_kernel");
        return MHC_OK;
      });
    });
  });
}

extern "C" size_t mhc_residual_add_agg_bwd_workspace_bytes(int64_t T, int n, int C) {
  if (T <= 0 || n < 1 || n > MHC_MAX_N || C < 1) return 0;
  const int64_t G = res_bwd_grid(T, n, C, device_cu_count());
  return (size_t)(G + kResSplit) * (size_t)round_up(n, 4) * sizeof(float);
}

extern "C" int mhc_residual_add_agg_bwd(const void* x, const void* res, int dtype, const void* dout,
                                        int dout_dtype, const float* dy_agg, const float* h_pre,
                                        int h_mode, void* dx, void* dres, float* dh_pre, void* workspace,
                                        size_t workspace_bytes, int64_t T, int n, int C, void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1 && T >= 0, "invalid T=%lld / C=%d", (long long)T, C);
  MHC_CHECK_ARG(h_mode == MHC_H_ACTIVATED || h_mode == MHC_H_RAW, "invalid h_mode %d", h_mode);
  MHC_CHECK_ARG(dtype_bytes(dtype), "unknown dtype code %d", dtype);
  MHC_CHECK_ARG(!dout || dout_dtype == MHC_DTYPE_F32 || dout_dtype == dtype,
                "dout_dtype must be fp32 or the inputs' dtype");
  MHC_CHECK_ARG(h_pre, "h_pre is required");
  const int cus = device_cu_count();
  if (T == 0) {
    // no tokens: dh_pre = 0 (a kernel write, not a memset, so the call stays capturable)
    if (dh_pre) {
      hipLaunchKernelGGL(residual_final_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, nullptr, 0, 4, n,
                         MHC_H_ACTIVATED, h_pre, dh_pre);
      MHC_CHECK_LAUNCH("residual_final_kernel");
    }
    return MHC_OK;
  }
  MHC_CHECK_ARG(!dh_pre || (x && res), "x and res are required for dh_pre");
  const int64_t G = res_bwd_grid(T, n, C, cus);
  const int P = round_up(n, 4);
  if (dh_pre) {
    const size_t need = (size_t)(G + kResSplit) * P * sizeof(float);
    MHC_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 16),
                  "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, need);
  }
  ResArgs A{};
  A.x = x; A.res = res; A.g = dout; A.gy = dy_agg; A.out = dx; A.out2 = dres; A.hpre = h_pre;
  A.part = dh_pre ? (float*)workspace : nullptr;
  A.T = T; A.n = n; A.C = C; A.nchunks = (int)ceil_div(C, kResV); A.h_mode = h_mode; A.P = P;
  const int gdt = dout ? dout_dtype : dtype;
  A.vec = res_vec_ok(C, {{x, dtype_bytes(dtype)}, {res, dtype_bytes(dtype)}, {dout, dtype_bytes(gdt)},
                         {dy_agg, 4}, {dx, dtype_bytes(dtype)}, {dres, dtype_bytes(dtype)}});
  hipStream_t s = (hipStream_t)stream;
  const int groups = (int)ceil_div(n, kResBwdGroup);
  int rc = res_by_dtype(dtype, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    auto launch = [&](auto* gp) {
      using GT = std::remove_pointer_t<decltype(gp)>;
      hipLaunchKernelGGL((residual_add_agg_bwd_kernel<kResBwdGroup, XT, GT>),
                         dim3((unsigned)G, (unsigned)groups), dim3(kResThreads), 0, s, A);
      MHC_CHECK_LAUNCH("residual_add_agg_bwd_kernel");
      return MHC_OK;
    };
    if (gdt == MHC_DTYPE_F32) return launch((float*)nullptr);
    return launch((XT*)nullptr);
  });
  if (rc != MHC_OK || !dh_pre) return rc;
  float* part2 = (float*)workspace + (size_t)G * P;
  const int S = (int)std::min<int64_t>(kResSplit, G);
  const int rows = (int)ceil_div(G, S);
  const int S_used = (int)ceil_div(G, rows);
  hipLaunchKernelGGL(reduce_rows_kernel, dim3((unsigned)ceil_div(P / 4, 256), (unsigned)S_used), dim3(256), 0,
                     s, (const float*)workspace, part2, G, P, rows);
  MHC_CHECK_LAUNCH("reduce_rows_kernel");
  hipLaunchKernelGGL(residual_final_kernel, dim3(1), dim3(64), 0, s, part2, S_used, P, n, h_mode, h_pre,
                     dh_pre);
  MHC_CHECK_LAUNCH("residual_final_kernel");
  return MHC_OK;
}
