// MHCRewire kernels (mhc_mlx/layer.py:302-337, 469-492):
//   pre-scale     x_pre[t,i,c] = a_i x[t,i,c]
//   post-combine  out[t,i,c] = p_i (y[t,i,c] + sum_j M_ij a_j x[t,j,c])
// and their VJPs.  With h_mode == MHC_H_NONE (a = p = 1) the post-combine is
// stream_mix_add (metal.py:954-1014: out = M x + y_dist).
//
// Work item = (token, chunk of V channels x n streams); items are processed
// grid-stride by a persistent grid.  The VJPs accumulate the per-stream sums
// (S_ij = sum g_i x_j, Yd_i = sum g_i y_i, Sa_i = sum g_i x_i) per thread,
// reduce them over the workgroup at the end into one partial row per
// workgroup and finish with the fixed-order row reduction.
#include "mhc_device.hpp"
#include "mhc_generic.hpp"
#include "mhc_host.hpp"
#include "mhc_mix32.hpp"
#include "mhc_plan.hpp"
#include "mhc_reduce.hpp"

namespace mhc {

namespace {

constexpr int kMixThreads = 256;
constexpr int kMixSplit = 64;

// Channels per work item: 16 bytes per lane of the widest tensor for n <= 8
// (8 channels when every tensor is 16-bit, 4 when one is fp32), so each
// lane's access of any tensor is one coalesced load or store of at most 16 bytes.
constexpr int mix_v(int nmax, int max_elem_bytes) {
  return nmax == 0 ? 1 : (nmax <= 8 ? 16 / max_elem_bytes : 64 / nmax);
}

template <int NMAX, typename... Ts>
struct MixCfg {
  static constexpr int kMaxBytes = std::max({ElemTraits<Ts>::kBytes...});
  static constexpr int V = mix_v(NMAX, kMaxBytes);
};

struct MixArgs {
  const void* x;
  const void* y;
  const void* g;
  void* out;   // fwd: out; bwd: dx
  void* dy;    // bwd only (may be null)
  const void* acc;  // stream_scale bwd: optional dx accumulator
  const float* M;
  const float* hpre;
  const float* hpost;
  float* part;
  int64_t T;
  int n;
  int C;
  int nchunks;
  int h_mode;
  int vec;
  int P;
};

// Mf (NMAX x NMAX, Mf_ij = p_i M_ij a_j), a, p into LDS.
template <int NMAX>
MHC_DEV void mix_stage(float* buf, const MixArgs& A) {
  const int n = A.n;
  for (int idx = threadIdx.x; idx < NMAX * NMAX + 2 * NMAX; idx += blockDim.x) {
    float v = 0.0f;
    auto act_a = [&](int i) {
      if (A.h_mode == MHC_H_NONE) return 1.0f;
      return A.h_mode == MHC_H_RAW ? sigmoidf_(A.hpre[i]) : A.hpre[i];
    };
    auto act_p = [&](int i) {
      if (A.h_mode == MHC_H_NONE) return 1.0f;
      return A.h_mode == MHC_H_RAW ? 2.0f * sigmoidf_(A.hpost[i]) : A.hpost[i];
    };
    if (idx < NMAX * NMAX) {
      const int i = idx / NMAX, j = idx % NMAX;
      if (i < n && j < n && A.M) v = act_p(i) * A.M[i * n + j] * act_a(j);
    } else if (idx < NMAX * NMAX + NMAX) {
      const int i = idx - NMAX * NMAX;
      if (i < n) v = act_a(i);
    } else {
      const int i = idx - NMAX * NMAX - NMAX;
      if (i < n) v = act_p(i);
    }
    buf[idx] = v;
  }
}

template <typename T, int V>
MHC_DEV void load_chunk(Vec<T, V>& r, const T* p, bool vec, int valid) {
  if (vec && valid == V) r.load(p);
  else r.load_partial(p, valid);
}

template <typename T, int V>
MHC_DEV void store_chunk(T* p, const float (&v)[V], bool vec, int valid) {
  if (vec && valid == V) store_vec<T, V>(p, v);
  else store_partial<T, V>(p, v, valid);
}

// (token, chunk) of a grid-stride walk over T x nchunks items, advanced by
// the fixed stride without a 64-bit division per item.
struct ItemWalk {
  int64_t t, dt;
  int q, dq, nch;
  MHC_DEV ItemWalk(int64_t first, int64_t stride, int nchunks) : nch(nchunks) {
    t = first / nchunks;
    q = (int)(first - t * nchunks);
    dt = stride / nchunks;
    dq = (int)(stride - dt * nchunks);
  }
  MHC_DEV void next() {
    t += dt;
    q += dq;
    if (q >= nch) {
      q -= nch;
      ++t;
    }
  }
};

// FULL: n == NMAX, every chunk whole and 16-byte aligned, y present (and for
// the VJP dy too, n <= 8): the item loop has no per-item conditions, so all
// of an item's loads are issued together.
template <int NMAX, typename XT, typename YT, typename OT, bool FULL>
__global__ __launch_bounds__(kMixThreads) void mix_add_fwd_kernel(MixArgs A) {
  constexpr int V = MixCfg<NMAX, XT, YT, OT>::V;
  __shared__ float s_par[NMAX * NMAX + 2 * NMAX];
  mix_stage<NMAX>(s_par, A);
  __syncthreads();
  // n <= 4: Mf and p in scalar registers for the whole grid-stride loop
  constexpr bool UREG = NMAX <= 4;
  float mf[UREG ? NMAX * NMAX : 1], ps[UREG ? NMAX : 1];
  if constexpr (UREG) {
#pragma unroll
    for (int k = 0; k < NMAX * NMAX; ++k) mf[k] = uniform_f(s_par[k]);
#pragma unroll
    for (int i = 0; i < NMAX; ++i) ps[i] = uniform_f(s_par[NMAX * NMAX + NMAX + i]);
  }
  auto mf_at = [&](int k) -> float {
    if constexpr (UREG) return mf[k]; else return s_par[k];
  };
  auto p_at = [&](int i) -> float {
    if constexpr (UREG) return ps[i]; else return s_par[NMAX * NMAX + NMAX + i];
  };
  const int n = A.n, C = A.C;
  const int64_t items = A.T * A.nchunks;
  const XT* __restrict__ X = (const XT*)A.x;
  const YT* __restrict__ Y = (const YT*)A.y;
  OT* __restrict__ O = (OT*)A.out;
  if constexpr (FULL) {
    for (ItemWalk w((int64_t)blockIdx.x * blockDim.x + threadIdx.x, (int64_t)gridDim.x * blockDim.x, A.nchunks);
         w.t < A.T; w.next()) {
      const int64_t base = w.t * NMAX * C + w.q * V;
      Vec<XT, V> xr[NMAX];
      Vec<YT, V> yr[NMAX];
#pragma unroll
      for (int j = 0; j < NMAX; ++j) {
        xr[j].load(X + base + (int64_t)j * C);
        yr[j].load(Y + base + (int64_t)j * C);
      }
      issue_fence();
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          float acc = 0.0f;
#pragma unroll
          for (int j = 0; j < NMAX; ++j) acc = fmaf(mf_at(i * NMAX + j), xr[j].get(v), acc);
          o[v] = fmaf(p_at(i), yr[i].get(v), acc);
        }
        store_vec<OT, V>(O + base + (int64_t)i * C, o);
      }
    }
    return;
  }
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = item / A.nchunks;
    const int q = (int)(item - t * A.nchunks);
    const int c0 = q * V;
    const int valid = min(V, C - c0);
    const int64_t base = t * n * C + c0;
    // every load of the item goes out before the first store
    Vec<XT, V> xr[NMAX];
    Vec<YT, V> yr[NMAX];
#pragma unroll
    for (int j = 0; j < NMAX; ++j) {
      if (j < n) load_chunk<XT, V>(xr[j], X + base + (int64_t)j * C, A.vec, valid);
      else xr[j].zero();
      if (j < n && Y) load_chunk<YT, V>(yr[j], Y + base + (int64_t)j * C, A.vec, valid);
      else yr[j].zero();
    }
#pragma unroll
    for (int i = 0; i < NMAX; ++i) {
      if (i < n) {
        const float p = p_at(i);
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          float acc = 0.0f;
#pragma unroll
          for (int j = 0; j < NMAX; ++j) acc = fmaf(mf_at(i * NMAX + j), xr[j].get(v), acc);
          o[v] = fmaf(p, yr[i].get(v), acc);
        }
        store_chunk<OT, V>(O + base + (int64_t)i * C, o, A.vec, valid);
      }
    }
  }
}

// VJP of the post-combine.  Per-thread sums: S_ij (NMAX^2) then Yd_i (NMAX).
template <int NMAX, typename XT, typename YT, typename GT, bool FULL>
__global__ __launch_bounds__(kMixThreads) void mix_add_bwd_kernel(MixArgs A) {
  constexpr int V = MixCfg<NMAX, XT, YT, GT>::V;
  constexpr int K = NMAX * NMAX + NMAX;
  constexpr int NBLK = (K + 63) / 64;
  constexpr bool REG = NMAX <= 8;
  __shared__ float s_par[NMAX * NMAX + 2 * NMAX];
  __shared__ float s_stage[(kMixThreads / 64) * 64];
  mix_stage<NMAX>(s_par, A);
  __syncthreads();
  constexpr bool UREG = NMAX <= 4;
  float mf[UREG ? NMAX * NMAX : 1], ps[UREG ? NMAX : 1];
  if constexpr (UREG) {
#pragma unroll
    for (int k = 0; k < NMAX * NMAX; ++k) mf[k] = uniform_f(s_par[k]);
#pragma unroll
    for (int i = 0; i < NMAX; ++i) ps[i] = uniform_f(s_par[NMAX * NMAX + NMAX + i]);
  }
  auto mf_at = [&](int k) -> float {
    if constexpr (UREG) return mf[k]; else return s_par[k];
  };
  auto p_at = [&](int i) -> float {
    if constexpr (UREG) return ps[i]; else return s_par[NMAX * NMAX + NMAX + i];
  };
  const int lane = threadIdx.x & 63;
  const int n = A.n, C = A.C;
  const int64_t items = A.T * A.nchunks;
  const XT* __restrict__ X = (const XT*)A.x;
  const YT* __restrict__ Y = (const YT*)A.y;
  const GT* __restrict__ Gd = (const GT*)A.g;
  XT* __restrict__ DX = (XT*)A.out;
  YT* __restrict__ DY = (YT*)A.dy;
  // REG: full per-thread sums; else one lane-owned butterfly result per block
  float acc[REG ? 64 * NBLK : 1];
  float accL[NBLK];
#pragma unroll
  for (int k = 0; k < (REG ? 64 * NBLK : 1); ++k) acc[k] = 0.0f;
#pragma unroll
  for (int b = 0; b < NBLK; ++b) accL[b] = 0.0f;
  static_assert(!FULL || REG, "the unconditional item loop keeps per-thread sums");
  if constexpr (FULL) {
    for (ItemWalk w((int64_t)blockIdx.x * blockDim.x + threadIdx.x, (int64_t)gridDim.x * blockDim.x, A.nchunks);
         w.t < A.T; w.next()) {
      const int64_t base = w.t * NMAX * C + w.q * V;
      Vec<XT, V> xr[NMAX];
      Vec<GT, V> gr[NMAX];
      Vec<YT, V> yr[NMAX];
#pragma unroll
      for (int j = 0; j < NMAX; ++j) {
        xr[j].load(X + base + (int64_t)j * C);
        gr[j].load(Gd + base + (int64_t)j * C);
        yr[j].load(Y + base + (int64_t)j * C);
      }
      issue_fence();
      // dx_j = sum_i Mf_ij g_i, dy_i = p_i g_i
#pragma unroll
      for (int j = 0; j < NMAX; ++j) {
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          float sum = 0.0f;
#pragma unroll
          for (int i = 0; i < NMAX; ++i) sum = fmaf(mf_at(i * NMAX + j), gr[i].get(v), sum);
          o[v] = sum;
        }
        store_vec<XT, V>(DX + base + (int64_t)j * C, o);
      }
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) o[v] = p_at(i) * gr[i].get(v);
        store_vec<YT, V>(DY + base + (int64_t)i * C, o);
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          const float gv = gr[i].get(v);
#pragma unroll
          for (int j = 0; j < NMAX; ++j) acc[i * NMAX + j] = fmaf(gv, xr[j].get(v), acc[i * NMAX + j]);
          acc[NMAX * NMAX + i] = fmaf(gv, yr[i].get(v), acc[NMAX * NMAX + i]);
        }
      }
    }
  }
  const int64_t nitems_pad =
      FULL ? 0 : ceil_div(items, (int64_t)gridDim.x * blockDim.x) * gridDim.x * blockDim.x;
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < nitems_pad;
       item += (int64_t)gridDim.x * blockDim.x) {
    const bool act = item < items;
    const int64_t t = act ? item / A.nchunks : 0;
    const int q = act ? (int)(item - t * A.nchunks) : 0;
    const int c0 = q * V;
    const int valid = act ? min(V, C - c0) : 0;
    const int64_t base = t * n * C + c0;
    Vec<XT, V> xr[NMAX];
    Vec<GT, V> gr[NMAX];
    Vec<YT, V> yr[NMAX];
#pragma unroll
    for (int j = 0; j < NMAX; ++j) {
      if (act && j < n) {
        load_chunk<XT, V>(xr[j], X + base + (int64_t)j * C, A.vec, valid);
        load_chunk<GT, V>(gr[j], Gd + base + (int64_t)j * C, A.vec, valid);
        if (Y) load_chunk<YT, V>(yr[j], Y + base + (int64_t)j * C, A.vec, valid);
        else yr[j].zero();
      } else {
        xr[j].zero();
        gr[j].zero();
        yr[j].zero();
      }
    }
    if (act) {
      // dx_j = sum_i Mf_ij g_i
#pragma unroll
      for (int j = 0; j < NMAX; ++j) {
        if (j < n) {
          float o[V];
#pragma unroll
          for (int v = 0; v < V; ++v) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < NMAX; ++i) s = fmaf(mf_at(i * NMAX + j), gr[i].get(v), s);
            o[v] = s;
          }
          store_chunk<XT, V>(DX + base + (int64_t)j * C, o, A.vec, valid);
        }
      }
      // dy_i = p_i g_i
      if (DY) {
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          if (i < n) {
            const float p = p_at(i);
            float o[V];
#pragma unroll
            for (int v = 0; v < V; ++v) o[v] = p * gr[i].get(v);
            store_chunk<YT, V>(DY + base + (int64_t)i * C, o, A.vec, valid);
          }
        }
      }
    }
    if constexpr (REG) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          const float gv = gr[i].get(v);
#pragma unroll
          for (int j = 0; j < NMAX; ++j) acc[i * NMAX + j] = fmaf(gv, xr[j].get(v), acc[i * NMAX + j]);
          acc[NMAX * NMAX + i] = fmaf(gv, yr[i].get(v), acc[NMAX * NMAX + i]);
        }
      }
    } else {
#pragma unroll
      for (int b = 0; b < NBLK; ++b) {
        float pv[64];
#pragma unroll
        for (int kk = 0; kk < 64; ++kk) {
          const int k = 64 * b + kk;
          float s = 0.0f;
          if (k < NMAX * NMAX) {
            const int i = k / NMAX, j = k % NMAX;
#pragma unroll
            for (int v = 0; v < V; ++v) s = fmaf(gr[i].get(v), xr[j].get(v), s);
          } else if (k < K) {
            const int i = k - NMAX * NMAX;
#pragma unroll
            for (int v = 0; v < V; ++v) s = fmaf(gr[i].get(v), yr[i].get(v), s);
          }
          pv[kk] = s;
        }
        wave_reduce_scatter<1>(pv, lane);
        accL[b] += pv[0];
      }
    }
  }
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  // reduce the sums into this workgroup's row (n-indexed: S then Yd)
  {
    const int wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
#pragma unroll
    for (int b = 0; b < NBLK; ++b) {
      float v;
      if constexpr (REG) {
        float pv[64];
#pragma unroll
        for (int kk = 0; kk < 64; ++kk) pv[kk] = acc[(64 * b + kk) % (REG ? 64 * NBLK : 1)];
        wave_reduce_scatter<1>(pv, lane);
        v = pv[0];
      } else {
        v = accL[b];
      }
      __syncthreads();
      s_stage[wave * 64 + lane] = v;
      __syncthreads();
      if (threadIdx.x < 64) {
        float s = 0.0f;
        for (int w = 0; w < nwaves; ++w) s += s_stage[w * 64 + threadIdx.x];
        const int k = 64 * b + threadIdx.x;
        if (k < NMAX * NMAX) {
          const int i = k / NMAX, j = k % NMAX;
          if (i < n && j < n) prow[i * n + j] = s;
        } else if (k < K) {
          const int i = k - NMAX * NMAX;
          if (i < n) prow[n * n + i] = s;
        }
      }
    }
    if (threadIdx.x == 0)
      for (int c = n * n + n; c < A.P; ++c) prow[c] = 0.0f;
  }
}

// Sums over the S <= 64 rows of part2 (row stride P) of columns
// c0 .. c0 + 3 (those below K): row `lane` per lane, the four columns' loads
// in flight together, then a fixed-order wave butterfly; every lane returns
// the four sums.
static_assert(kMixSplit <= 64, "col_sums4 takes one partial row per lane");
MHC_DEV void col_sums4(const float* __restrict__ part2, int S, int P, int c0, int K, int lane,
                       float (&v)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (lane < S && c0 + e < K) ? part2[(int64_t)lane * P + c0 + e] : 0.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = wave_sum(v[e]);
}

// Final: sum S partial rows, then dM / dh_pre / dh_post (one block).  One
// thread per column adds the S rows in row order (coalesced across the
// threads); M and the activated a, p are staged in LDS first, so the n-long
// dot products below read LDS only.
__global__ __launch_bounds__(256) void mix_final_kernel(const float* __restrict__ part2, int S,
                                                        int P, int n, int h_mode,
                                                        const float* __restrict__ M,
                                                        const float* __restrict__ hpre,
                                                        const float* __restrict__ hpost,
                                                        float* __restrict__ dM,
                                                        float* __restrict__ dpre,
                                                        float* __restrict__ dpost) {
  extern __shared__ float s_sum[];  // [n*n + n]: S then Yd; then M [n*n], a [n], p [n]
  const int K = n * n + n;
  float* s_M = s_sum + K;
  float* s_a = s_M + n * n;
  float* s_p = s_a + n;
  for (int c = threadIdx.x; c < K; c += blockDim.x) {
    const float* src = part2 + c;
    float acc = 0.0f;
#pragma unroll 8
    for (int r = 0; r < S; ++r) acc += src[(int64_t)r * P];
    s_sum[c] = acc;
  }
  for (int k = threadIdx.x; k < n * n; k += blockDim.x) s_M[k] = M[k];
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    float a = 1.0f, p = 1.0f;
    if (h_mode == MHC_H_RAW) {
      a = sigmoidf_(hpre[i]);
      p = 2.0f * sigmoidf_(hpost[i]);
    } else if (h_mode == MHC_H_ACTIVATED) {
      a = hpre[i];
      p = hpost[i];
    }
    s_a[i] = a;
    s_p[i] = p;
  }
  __syncthreads();
  for (int k = threadIdx.x; k < n * n; k += blockDim.x) {
    const int i = k / n, j = k % n;
    dM[k] = h_mode == MHC_H_NONE ? s_sum[k] : s_p[i] * s_sum[k] * s_a[j];
  }
  if (h_mode == MHC_H_NONE) return;
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    float acc = 0.0f;
    for (int i = 0; i < n; ++i) acc = fmaf(s_p[i] * s_M[i * n + j], s_sum[i * n + j], acc);
    if (h_mode == MHC_H_RAW) {
      const float a = s_a[j];
      acc *= a * (1.0f - a);
    }
    dpre[j] = acc;
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    float acc = 0.0f;
    for (int j = 0; j < n; ++j) acc = fmaf(s_M[i * n + j] * s_a[j], s_sum[i * n + j], acc);
    acc += s_sum[n * n + i];
    if (h_mode == MHC_H_RAW) {
      const float sg = 0.5f * s_p[i];
      acc *= 2.0f * sg * (1.0f - sg);
    }
    dpost[i] = acc;
  }
}

// pre-scale forward: out_i = a_i x_i.  grid.y = stream i; x dimension over
// (token, chunk of 8 channels).
// FULL (every chunk whole and 16-byte aligned): kScaleU items per thread per
// step, their loads issued together ahead of their stores.
constexpr int kScaleU = 4;

template <typename XT, typename OT, bool FULL>
__global__ __launch_bounds__(kMixThreads) void scale_fwd_kernel(MixArgs A) {
  constexpr int V = 8;
  const int i = blockIdx.y;
  const float hv = A.hpre[i];
  const float a = A.h_mode == MHC_H_RAW ? sigmoidf_(hv) : hv;
  const int n = A.n, C = A.C;
  const int64_t items = A.T * A.nchunks;
  const XT* __restrict__ X = (const XT*)A.x;
  OT* __restrict__ O = (OT*)A.out;
  if constexpr (FULL) {
    ItemWalk w((int64_t)blockIdx.x * blockDim.x + threadIdx.x, (int64_t)gridDim.x * blockDim.x, A.nchunks);
    while (w.t < A.T) {
      int64_t off[kScaleU];
      bool on[kScaleU];
      Vec<XT, V> xr[kScaleU];
#pragma unroll
      for (int u = 0; u < kScaleU; ++u) {
        on[u] = w.t < A.T;
        off[u] = on[u] ? (w.t * n + i) * C + w.q * V : 0;
        if (on[u]) xr[u].load(X + off[u]);
        w.next();
      }
      issue_fence();
#pragma unroll
      for (int u = 0; u < kScaleU; ++u) {
        if (!on[u]) continue;
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) o[v] = a * xr[u].get(v);
        store_vec<OT, V>(O + off[u], o);
      }
    }
    return;
  }
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = item / A.nchunks;
    const int q = (int)(item - t * A.nchunks);
    const int c0 = q * V;
    const int valid = min(V, C - c0);
    const int64_t off = (t * n + i) * C + c0;
    Vec<XT, V> xr;
    load_chunk<XT, V>(xr, X + off, A.vec, valid);
    float o[V];
#pragma unroll
    for (int v = 0; v < V; ++v) o[v] = a * xr.get(v);
    store_chunk<OT, V>(O + off, o, A.vec, valid);
  }
}

// The pre-scale over the tensor as one flat array (whole 16-byte chunks,
// aligned): chunk c lies in row c / nchunks, i.e. stream (c / nchunks) % n,
// so consecutive lanes and workgroups stream consecutive memory as a plain
// elementwise kernel does, one chunk per thread.
template <typename XT, typename OT>
__global__ __launch_bounds__(kMixThreads) void scale_fwd_flat_kernel(MixArgs A, uint32_t total) {
  constexpr int V = 16 / (ElemTraits<XT>::kBytes > ElemTraits<OT>::kBytes ? ElemTraits<XT>::kBytes
                                                                             : ElemTraits<OT>::kBytes);
  const uint32_t c = blockIdx.x * (uint32_t)blockDim.x + threadIdx.x;
  if (c >= total) return;
  const XT* __restrict__ X = (const XT*)A.x;
  OT* __restrict__ O = (OT*)A.out;
  Vec<XT, V> xr;
  xr.load(X + (int64_t)c * V);
  const uint32_t i = (c / (uint32_t)A.nchunks) % (uint32_t)A.n;
  const float hv = A.hpre[i];
  const float a = A.h_mode == MHC_H_RAW ? sigmoidf_(hv) : hv;
  float o[V];
#pragma unroll
  for (int v = 0; v < V; ++v) o[v] = a * xr.get(v);
  store_vec<OT, V>(O + (int64_t)c * V, o);
}

// pre-scale VJP: dx_i = a_i g_i (+ acc), Sa_i = sum g_i x_i.  grid.y = stream
// i; block (bx, i) writes column i of partial row bx.
template <typename XT, typename GT, bool FULL>
__global__ __launch_bounds__(kMixThreads) void scale_bwd_kernel(MixArgs A) {
  constexpr int V = 8;
  __shared__ float s_stage[kMixThreads / 64];
  const int i = blockIdx.y;
  const float hv = A.hpre[i];
  const float a = A.h_mode == MHC_H_RAW ? sigmoidf_(hv) : hv;
  const int n = A.n, C = A.C;
  const int64_t items = A.T * A.nchunks;
  const XT* __restrict__ X = (const XT*)A.x;
  const GT* __restrict__ Gd = (const GT*)A.g;
  const XT* __restrict__ ACC = (const XT*)A.acc;
  XT* __restrict__ DX = (XT*)A.out;
  float acc = 0.0f;
  if constexpr (FULL) {
    // the dx accumulator (ACC) is absent on this path
    ItemWalk w((int64_t)blockIdx.x * blockDim.x + threadIdx.x, (int64_t)gridDim.x * blockDim.x, A.nchunks);
    while (w.t < A.T) {
      int64_t off[kScaleU];
      bool on[kScaleU];
      Vec<XT, V> xr[kScaleU];
      Vec<GT, V> gr[kScaleU];
#pragma unroll
      for (int u = 0; u < kScaleU; ++u) {
        on[u] = w.t < A.T;
        off[u] = on[u] ? (w.t * n + i) * C + w.q * V : 0;
        if (on[u]) {
          xr[u].load(X + off[u]);
          gr[u].load(Gd + off[u]);
        } else {
          xr[u].zero();
          gr[u].zero();
        }
        w.next();
      }
      issue_fence();
#pragma unroll
      for (int u = 0; u < kScaleU; ++u) {
#pragma unroll
        for (int v = 0; v < V; ++v) acc = fmaf(gr[u].get(v), xr[u].get(v), acc);
        if (!on[u]) continue;
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) o[v] = a * gr[u].get(v);
        store_vec<XT, V>(DX + off[u], o);
      }
    }
  }
  // general path (FULL: nothing left)
  for (int64_t item = FULL ? items : (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < items;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = item / A.nchunks;
    const int q = (int)(item - t * A.nchunks);
    const int c0 = q * V;
    const int valid = min(V, C - c0);
    const int64_t off = (t * n + i) * C + c0;
    Vec<XT, V> xr;
    Vec<GT, V> gr;
    load_chunk<XT, V>(xr, X + off, A.vec, valid);
    load_chunk<GT, V>(gr, Gd + off, A.vec, valid);
    float o[V];
    if (ACC) {
      Vec<XT, V> ar;
      load_chunk<XT, V>(ar, ACC + off, A.vec, valid);
#pragma unroll
      for (int v = 0; v < V; ++v) o[v] = fmaf(a, gr.get(v), ar.get(v));
    } else {
#pragma unroll
      for (int v = 0; v < V; ++v) o[v] = a * gr.get(v);
    }
#pragma unroll
    for (int v = 0; v < V; ++v) acc = fmaf(gr.get(v), xr.get(v), acc);
    store_chunk<XT, V>(DX + off, o, A.vec, valid);
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) s_stage[threadIdx.x >> 6] = acc;
  __syncthreads();
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += s_stage[w];
    prow[i] = s;
    if (i == 0)
      for (int c = n; c < A.P; ++c) prow[c] = 0.0f;
  }
}

// The pre-scale VJP as a flat pass: 16-bit x and dout of one dtype, whole
// aligned 8-channel chunks, nchunks a multiple of 64 and n * nchunks of 256.
// The grid's thread count is a multiple of n * nchunks, so each thread's
// chunks lie in one stream and each wave's in one row; block b adds its
// waves' sums into its partial row in wave order.  ACC: dx = a g + dx_accum
// (the accumulator in dx's dtype, read in the same pass; it may be dx itself:
// each element is read before the store that depends on it).
template <typename XT, bool ACC>
__global__ __launch_bounds__(kMixThreads) void scale_bwd_flat_kernel(MixArgs A, uint32_t total) {
  constexpr int V = 8;
  __shared__ float s_stage[kMixThreads / 64];
  const uint32_t first = blockIdx.x * (uint32_t)kMixThreads + threadIdx.x;
  const uint32_t stride = gridDim.x * (uint32_t)kMixThreads;
  const uint32_t nch = (uint32_t)A.nchunks, n = (uint32_t)A.n;
  const int i = (int)((first / nch) % n);
  const float hv = A.hpre[i];
  const float a = A.h_mode == MHC_H_RAW ? sigmoidf_(hv) : hv;
  const XT* __restrict__ X = (const XT*)A.x;
  const XT* __restrict__ Gd = (const XT*)A.g;
  const XT* ACCP = (const XT*)A.acc;
  XT* DX = (XT*)A.out;
  float acc = 0.0f;
  for (uint32_t c = first; c < total; c += kScaleU * stride) {
    Vec<XT, V> xr[kScaleU], gr[kScaleU], ar[ACC ? kScaleU : 1];
    bool on[kScaleU];
#pragma unroll
    for (int u = 0; u < kScaleU; ++u) {
      const uint32_t cu = c + u * stride;
      on[u] = cu < total;
      if (on[u]) {
        xr[u].load(X + (int64_t)cu * V);
        gr[u].load(Gd + (int64_t)cu * V);
        if constexpr (ACC) ar[u].load(ACCP + (int64_t)cu * V);
      } else {
        xr[u].zero();
        gr[u].zero();
        if constexpr (ACC) ar[u].zero();
      }
    }
    issue_fence();
#pragma unroll
    for (int u = 0; u < kScaleU; ++u) {
#pragma unroll
      for (int v = 0; v < V; ++v) acc = fmaf(gr[u].get(v), xr[u].get(v), acc);
      if (!on[u]) continue;
      float o[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if constexpr (ACC) o[v] = fmaf(a, gr[u].get(v), ar[u].get(v));
        else o[v] = a * gr[u].get(v);
      }
      store_vec<XT, V>(DX + (int64_t)(c + u * stride) * V, o);
    }
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) s_stage[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float* prow = A.part + (int64_t)blockIdx.x * A.P;
    for (int j = 0; j < A.P; ++j) prow[j] = 0.0f;
    for (int w = 0; w < kMixThreads / 64; ++w) {
      const uint32_t cw = blockIdx.x * (uint32_t)kMixThreads + 64u * (uint32_t)w;
      prow[(cw / nch) % n] += s_stage[w];
    }
  }
}

__global__ __launch_bounds__(64) void scale_final_kernel(const float* __restrict__ part2, int S,
                                                         int P, int n, int h_mode,
                                                         const float* __restrict__ hpre,
                                                         float* __restrict__ dpre) {
  const int lane = threadIdx.x & 63;
  for (int c0 = 0; c0 < n; c0 += 4) {
    float v[4];
    col_sums4(part2, S, P, c0, n, lane, v);
    if (lane < 4 && c0 + lane < n) {
      const int j = c0 + lane;
      float s = v[0];
#pragma unroll
      for (int e = 1; e < 4; ++e)
        if (lane == e) s = v[e];
      if (h_mode == MHC_H_RAW) {
        const float a = sigmoidf_(hpre[j]);
        s *= a * (1.0f - a);
      }
      dpre[j] = s;
    }
  }
}

// ---------------------------------------------------------------------------
// host helpers
// ---------------------------------------------------------------------------

int mix_vec_width(int nmax, std::initializer_list<int> dtype_sizes) {
  int eb = 2;
  for (int b : dtype_sizes) eb = std::max(eb, b);
  return mix_v(nmax, eb);
}

// Grid of a grid-stride kernel over `work` items: at most `per_cu`
// workgroups per CU (per_cu < 0: one item per thread, up to kMaxGrid).
// `k` names the tuning knob that overrides per_cu.
int64_t mix_grid(int64_t work, int cus, Knob k, int per_cu = 8) {
  per_cu = knob(k, per_cu);
  int64_t g = ceil_div(work, kMixThreads);
  g = std::min<int64_t>(g, per_cu < 0 ? kMaxGrid : (int64_t)cus * std::max(per_cu, 1));
  return std::max<int64_t>(g, 1);
}

// Workgroups along x of the per-stream scale kernels (grid.y = n): at most
// 8 per CU over all streams by default; the knob `k` overrides the per-CU
// count (< 0: one item per thread).
int64_t scale_grid(int64_t T, int n, int C, Knob k) {
  const int per_cu = knob(k, 8);
  const int64_t g = ceil_div(T * ceil_div(C, 8), kMixThreads);
  const int64_t cap = per_cu < 0 ? kMaxGrid : (int64_t)device_cu_count() * std::max(per_cu, 1) / n + 1;
  return std::max<int64_t>(1, std::min<int64_t>(g, cap));
}

bool io_vec_ok(int C, int V, std::initializer_list<std::pair<const void*, int>> ptrs) {
  if (C % V != 0) return false;
  for (auto& pr : ptrs) {
    if (pr.first == nullptr) continue;
    const int al = std::min(16, V * pr.second);
    if (!aligned(pr.first, al) || ((int64_t)C * pr.second) % al != 0) return false;
  }
  return true;
}

template <typename F>
int by_nmax(int n, F&& f) {
  switch (nmax_for(n)) {
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    default: return f(std::integral_constant<int, 16>{});
  }
}

// second / third dtype: fp32 or the same as the first
template <typename T1, typename F>
int by_pair(int code2, F&& f) {
  if (code2 == MHC_DTYPE_F32) return f((float*)nullptr);
  if ((code2 == MHC_DTYPE_BF16 && std::is_same<T1, __bf16>::value) ||
      (code2 == MHC_DTYPE_F16 && std::is_same<T1, _Float16>::value))
    return f((T1*)nullptr);
  return set_error(MHC_ERR_INVALID_ARG, "unsupported dtype combination (dtype %d with %s)", code2,
                   std::is_same<T1, float>::value ? "fp32" : "a 16-bit first operand");
}

template <typename F>
int by_dtype(int code, F&& f) {
  switch (code) {
    case MHC_DTYPE_F32: return f((float*)nullptr);
    case MHC_DTYPE_BF16: return f((__bf16*)nullptr);
    case MHC_DTYPE_F16: return f((_Float16*)nullptr);
    default: return set_error(MHC_ERR_INVALID_ARG, "unknown dtype code %d", code);
  }
}

int mix_rows(int n) { return round_up(n * n + n, 4); }

}  // namespace
}  // namespace mhc

using namespace mhc;

extern "C" int mhc_stream_mix_add_fwd(const void* x, int x_dtype, const void* y, int y_dtype,
                                      const float* M, const float* h_pre, const float* h_post,
                                      int h_mode, void* out, int out_dtype, int64_t T, int n, int C,
                                      void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1 && T >= 0, "invalid T=%lld / C=%d", (long long)T, C);
  MHC_CHECK_ARG(h_mode == MHC_H_NONE || h_mode == MHC_H_ACTIVATED || h_mode == MHC_H_RAW,
                "invalid h_mode %d", h_mode);
  if (T == 0) return MHC_OK;
  MHC_CHECK_ARG(x && M && out, "null pointer argument");
  MHC_CHECK_ARG(h_mode == MHC_H_NONE || (h_pre && h_post), "h_pre/h_post required");
  MHC_CHECK_ARG(dtype_bytes(x_dtype) && dtype_bytes(out_dtype) && (!y || dtype_bytes(y_dtype)),
                "unknown dtype code");
  MixArgs A{};
  A.x = x; A.y = y; A.out = out; A.M = M; A.hpre = h_pre; A.hpost = h_post; A.T = T; A.n = n;
  A.C = C; A.h_mode = h_mode;
  const int V = mix_vec_width(nmax_for(n), {dtype_bytes(x_dtype), y ? dtype_bytes(y_dtype) : 2,
                                            dtype_bytes(out_dtype)});
  A.nchunks = (int)ceil_div(C, V);
  A.vec = io_vec_ok(C, V, {{x, dtype_bytes(x_dtype)}, {y, y ? dtype_bytes(y_dtype) : 4},
                           {out, dtype_bytes(out_dtype)}});
  const int64_t blocks = mix_grid(T * A.nchunks, device_cu_count(), kKnobMixFwdGrid, 8);
  hipStream_t s = (hipStream_t)stream;
  const int ydt = y ? y_dtype : x_dtype;
  if (nmax_for(n) == 0) {
    Mix32Args F{};
    F.x = x; F.y = y; F.out = out; F.M = M; F.hpre = h_pre; F.hpost = h_post; F.T = T; F.n = n; F.C = C;
    F.h_mode = h_mode;
    const int rc = mix32_fwd(F, x_dtype, ydt, out_dtype, s);
    if (rc != 1) return rc;
    GenArgs G{};
    G.x = x; G.y = y; G.out = out; G.M = M; G.hpre = h_pre; G.hpost = h_post; G.T = T; G.n = n;
    G.C = C; G.h_mode = h_mode;
    return gen_mix_fwd(G, x_dtype, ydt, out_dtype, s);
  }
  return by_nmax(n, [&](auto nm) {
    constexpr int NM = decltype(nm)::value;
    return by_dtype(x_dtype, [&](auto* xp) {
      using XT = std::remove_pointer_t<decltype(xp)>;
      return by_pair<XT>(ydt, [&](auto* yp) {
        using YT = std::remove_pointer_t<decltype(yp)>;
        return by_pair<XT>(out_dtype, [&](auto* op) {
          using OT = std::remove_pointer_t<decltype(op)>;
          if (n == NM && A.vec && y)
            hipLaunchKernelGGL((mix_add_fwd_kernel<NM, XT, YT, OT, true>), dim3((unsigned)blocks),
                               dim3(kMixThreads), 0, s, A);
          else
            hipLaunchKernelGGL((mix_add_fwd_kernel<NM, XT, YT, OT, false>), dim3((unsigned)blocks),
                               dim3(kMixThreads), 0, s, A);
          MHC_CHECK_LAUNCH("mix_add_fwd_kernel");
          return MHC_OK;
        });
      });
    });
  });
}

extern "C" size_t mhc_stream_mix_add_bwd_workspace_bytes(int64_t T, int n, int C) {
  if (T <= 0 || n < 1 || n > MHC_MAX_N || C < 1) return 0;
  // the narrowest item (fp32 operands) gives the most items and so the largest grid
  const int V = mix_vec_width(nmax_for(n), {4});
  const int64_t G = mix_grid(T * ceil_div(C, V), device_cu_count(), kKnobMixBwdGrid, 8);
  return (size_t)(G + kMixSplit) * (size_t)mix_rows(n) * sizeof(float);
}

extern "C" int mhc_stream_mix_add_bwd(const void* x, int x_dtype, const void* y, int y_dtype,
                                      const void* dout, int dout_dtype, const float* M,
                                      const float* h_pre, const float* h_post, int h_mode,
                                      void* dx, int dx_dtype, void* dy, int dy_dtype, float* dM,
                                      float* dh_pre, float* dh_post, void* workspace,
                                      size_t workspace_bytes, int64_t T, int n, int C,
                                      void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1 && T >= 1, "invalid T=%lld / C=%d", (long long)T, C);
  MHC_CHECK_ARG(h_mode == MHC_H_NONE || h_mode == MHC_H_ACTIVATED || h_mode == MHC_H_RAW,
                "invalid h_mode %d", h_mode);
  MHC_CHECK_ARG(x && dout && M && dx && dM, "null pointer argument");
  MHC_CHECK_ARG(h_mode == MHC_H_NONE || (h_pre && h_post && dh_pre && dh_post),
                "h_pre/h_post and their gradients are required");
  MHC_CHECK_ARG(dx_dtype == x_dtype, "dx_dtype must equal x_dtype");
  MHC_CHECK_ARG(!dy || !y || dy_dtype == y_dtype, "dy_dtype must equal y_dtype");
  MHC_CHECK_ARG(dtype_bytes(x_dtype) && dtype_bytes(dout_dtype), "unknown dtype code");
  const int ydt = y ? y_dtype : (dy ? dy_dtype : x_dtype);
  MHC_CHECK_ARG(dtype_bytes(ydt), "unknown dtype code");
  const int V = mix_vec_width(nmax_for(n), {dtype_bytes(x_dtype), dtype_bytes(ydt), dtype_bytes(dout_dtype)});
  const int nch = (int)ceil_div(C, V);
  const int64_t G = mix_grid(T * nch, device_cu_count(), kKnobMixBwdGrid, 8);
  const int P = mix_rows(n);
  const size_t need = (size_t)(G + kMixSplit) * P * sizeof(float);
  MHC_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 16),
                "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, need);
  MixArgs A{};
  A.x = x; A.y = y; A.g = dout; A.out = dx; A.dy = dy; A.M = M; A.hpre = h_pre; A.hpost = h_post;
  A.part = (float*)workspace; A.T = T; A.n = n; A.C = C; A.nchunks = nch; A.h_mode = h_mode; A.P = P;
  A.vec = io_vec_ok(C, V, {{x, dtype_bytes(x_dtype)}, {y, dtype_bytes(ydt)},
                           {dout, dtype_bytes(dout_dtype)}, {dy, dtype_bytes(ydt)}});
  hipStream_t s = (hipStream_t)stream;
  int rc;
  int64_t rows = G;  // partial rows written (the MFMA kernel may write fewer)
  if (nmax_for(n) == 0) {
    Mix32Args F{};
    F.x = x; F.y = y; F.g = dout; F.out = dx; F.dy = dy; F.M = M; F.hpre = h_pre; F.hpost = h_post;
    F.part = (float*)workspace; F.T = T; F.n = n; F.C = C; F.h_mode = h_mode; F.P = P;
    rc = mix32_bwd(F, x_dtype, ydt, dout_dtype, G, s, &rows);
    if (rc == 1) {
      GenArgs Gg{};
      Gg.x = x; Gg.y = y; Gg.g = dout; Gg.out = dx; Gg.dy = dy; Gg.M = M; Gg.hpre = h_pre;
      Gg.hpost = h_post; Gg.part = (float*)workspace; Gg.T = T; Gg.n = n; Gg.C = C; Gg.P = P;
      Gg.h_mode = h_mode;
      rows = G;
      rc = gen_mix_bwd(Gg, x_dtype, ydt, dout_dtype, s, G);
    }
  } else rc = by_nmax(n, [&](auto nm) {
    constexpr int NM = decltype(nm)::value;
    return by_dtype(x_dtype, [&](auto* xp) {
      using XT = std::remove_pointer_t<decltype(xp)>;
      return by_pair<XT>(ydt, [&](auto* yp) {
        using YT = std::remove_pointer_t<decltype(yp)>;
        return by_pair<XT>(dout_dtype, [&](auto* gp) {
          using GT = std::remove_pointer_t<decltype(gp)>;
          if constexpr (NM <= 8) {
            if (n == NM && A.vec && y && dy) {
              hipLaunchKernelGGL((mix_add_bwd_kernel<NM, XT, YT, GT, true>), dim3((unsigned)G),
                                 dim3(kMixThreads), 0, s, A);
              MHC_CHECK_LAUNCH("mix_add_bwd_kernel");
              return MHC_OK;
            }
          }
          hipLaunchKernelGGL((mix_add_bwd_kernel<NM, XT, YT, GT, false>), dim3((unsigned)G),
                             dim3(kMixThreads), 0, s, A);
          MHC_CHECK_LAUNCH("mix_add_bwd_kernel");
          return MHC_OK;
        });
      });
    });
  });
  if (rc != MHC_OK) return rc;
  float* part2 = (float*)workspace + (size_t)G * P;
  // about 64 rows per split: the split sums run in parallel workgroups, and
  // mix_final_kernel (one workgroup) then adds few rows per column
  const int S = (int)std::min<int64_t>(kMixSplit, ceil_div(rows, 64));
  const int per = (int)ceil_div(rows, S);
  const int S_used = (int)ceil_div(rows, per);
  hipLaunchKernelGGL(reduce_rows_kernel, dim3((unsigned)ceil_div(P / 4, 256), (unsigned)S_used),
                     dim3(256), 0, s, (const float*)workspace, part2, rows, P, per);
  MHC_CHECK_LAUNCH("reduce_rows_kernel");
  hipLaunchKernelGGL(mix_final_kernel, dim3(1), dim3(256), (size_t)(2 * n * n + 3 * n) * sizeof(float), s,
                     part2, S_used, P, n, h_mode, M, h_pre, h_post, dM, dh_pre, dh_post);
  MHC_CHECK_LAUNCH("mix_final_kernel");
  return MHC_OK;
}

extern "C" int mhc_stream_scale_fwd(const void* x, int x_dtype, const float* h_pre, int h_mode,
                                    void* out, int out_dtype, int64_t T, int n, int C,
                                    void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1 && T >= 0, "invalid T=%lld / C=%d", (long long)T, C);
  MHC_CHECK_ARG(h_mode == MHC_H_ACTIVATED || h_mode == MHC_H_RAW, "invalid h_mode %d", h_mode);
  if (T == 0) return MHC_OK;
  MHC_CHECK_ARG(x && h_pre && out, "null pointer argument");
  MHC_CHECK_ARG(dtype_bytes(x_dtype) && dtype_bytes(out_dtype), "unknown dtype code");
  MixArgs A{};
  A.x = x; A.out = out; A.hpre = h_pre; A.T = T; A.n = n; A.C = C; A.h_mode = h_mode;
  A.nchunks = (int)ceil_div(C, 8);
  A.vec = io_vec_ok(C, 8, {{x, dtype_bytes(x_dtype)}, {out, dtype_bytes(out_dtype)}});
  const int64_t bx = scale_grid(T, n, C, kKnobScaleFwdGrid);
  hipStream_t s = (hipStream_t)stream;
  const int vf = 16 / std::max(dtype_bytes(x_dtype), dtype_bytes(out_dtype));
  const int64_t flat_chunks = T * n * (int64_t)(C / vf);
  const bool flat = knob(kKnobScaleFwdFlat, 1) != 0 && C % vf == 0 && flat_chunks < (int64_t)UINT32_MAX - kMixThreads &&
                    io_vec_ok(C, vf, {{x, dtype_bytes(x_dtype)}, {out, dtype_bytes(out_dtype)}});
  return by_dtype(x_dtype, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return by_pair<XT>(out_dtype, [&](auto* op) {
      using OT = std::remove_pointer_t<decltype(op)>;
      if (flat) {
        MixArgs F = A;
        F.nchunks = C / vf;
        hipLaunchKernelGGL((scale_fwd_flat_kernel<XT, OT>), dim3((unsigned)ceil_div(flat_chunks, kMixThreads)),
                           dim3(kMixThreads), 0, s, F, (uint32_t)flat_chunks);
      } else if (A.vec)
        hipLaunchKernelGGL((scale_fwd_kernel<XT, OT, true>), dim3((unsigned)bx, (unsigned)n),
                           dim3(kMixThreads), 0, s, A);
      else
        hipLaunchKernelGGL((scale_fwd_kernel<XT, OT, false>), dim3((unsigned)bx, (unsigned)n),
                           dim3(kMixThreads), 0, s, A);
      MHC_CHECK_LAUNCH("scale_fwd_kernel");
      return MHC_OK;
    });
  });
}

namespace {
int64_t scale_bwd_grid(int64_t T, int n, int C) { return scale_grid(T, n, C, kKnobScaleBwdGrid); }
}  // namespace

extern "C" size_t mhc_stream_scale_bwd_workspace_bytes(int64_t T, int n, int C) {
  if (T <= 0 || n < 1 || n > MHC_MAX_N || C < 1) return 0;
  const int64_t G = scale_bwd_grid(T, n, C);
  return (size_t)(G + kMixSplit) * (size_t)round_up(n, 4) * sizeof(float);
}

extern "C" int mhc_stream_scale_bwd(const void* x, int x_dtype, const void* dout, int dout_dtype,
                                    const float* h_pre, int h_mode, const void* dx_accum, void* dx,
                                    int dx_dtype, float* dh_pre, void* workspace,
                                    size_t workspace_bytes, int64_t T, int n, int C,
                                    void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1 && T >= 1, "invalid T=%lld / C=%d", (long long)T, C);
  MHC_CHECK_ARG(h_mode == MHC_H_ACTIVATED || h_mode == MHC_H_RAW, "invalid h_mode %d", h_mode);
  MHC_CHECK_ARG(x && dout && h_pre && dx && dh_pre, "null pointer argument");
  MHC_CHECK_ARG(dx_dtype == x_dtype, "dx_dtype must equal x_dtype");
  MHC_CHECK_ARG(dtype_bytes(x_dtype) && dtype_bytes(dout_dtype), "unknown dtype code");
  const int64_t G = scale_bwd_grid(T, n, C);
  const int P = round_up(n, 4);
  const size_t need = (size_t)(G + kMixSplit) * P * sizeof(float);
  MHC_CHECK_ARG(workspace && workspace_bytes >= need && aligned(workspace, 16),
                "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, need);
  MixArgs A{};
  A.x = x; A.g = dout; A.acc = dx_accum; A.out = dx; A.hpre = h_pre;
  A.part = (float*)workspace; A.T = T; A.n = n; A.C = C; A.nchunks = (int)ceil_div(C, 8);
  A.h_mode = h_mode; A.P = P;
  A.vec = io_vec_ok(C, 8, {{x, dtype_bytes(x_dtype)}, {dout, dtype_bytes(dout_dtype)},
                           {dx_accum, dtype_bytes(x_dtype)}, {dx, dtype_bytes(x_dtype)}});
  hipStream_t s = (hipStream_t)stream;
  // flat pass: a grid of whole multiples of n * nchunks / 256 workgroups, within the workspace's rows
  const int64_t total = T * n * (int64_t)A.nchunks;
  const int64_t m = (int64_t)n * A.nchunks / kMixThreads;
  int64_t Gf = 0;
  if (knob(kKnobScaleBwdFlat, 1) != 0 && A.vec && x_dtype == dout_dtype && dtype_bytes(x_dtype) == 2 &&
      C % 8 == 0 && A.nchunks % 64 == 0 && ((int64_t)n * A.nchunks) % kMixThreads == 0 && total < INT32_MAX)
    Gf = std::min<int64_t>(G, total / kMixThreads) / m * m;
  int64_t rows_used = G;
  int rc;
  if (Gf > 0) {
    rows_used = Gf;
    rc = by_dtype(x_dtype, [&](auto* xp) {
      using XT = std::remove_pointer_t<decltype(xp)>;
      if constexpr (ElemTraits<XT>::kBytes == 2) {
        if (dx_accum)
          hipLaunchKernelGGL((scale_bwd_flat_kernel<XT, true>), dim3((unsigned)Gf), dim3(kMixThreads), 0, s, A,
                             (uint32_t)total);
        else
          hipLaunchKernelGGL((scale_bwd_flat_kernel<XT, false>), dim3((unsigned)Gf), dim3(kMixThreads), 0, s, A,
                             (uint32_t)total);
        MHC_CHECK_LAUNCH("scale_bwd_flat_kernel");
        return MHC_OK;
      } else {
        return set_error(MHC_ERR_INVALID_ARG, "flat pre-scale VJP needs 16-bit data");
      }
    });
  } else rc = by_dtype(x_dtype, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return by_pair<XT>(dout_dtype, [&](auto* gp) {
      using GT = std::remove_pointer_t<decltype(gp)>;
      if (A.vec && !dx_accum)
        hipLaunchKernelGGL((scale_bwd_kernel<XT, GT, true>), dim3((unsigned)G, (unsigned)n),
                           dim3(kMixThreads), 0, s, A);
      else
        hipLaunchKernelGGL((scale_bwd_kernel<XT, GT, false>), dim3((unsigned)G, (unsigned)n),
                           dim3(kMixThreads), 0, s, A);
      MHC_CHECK_LAUNCH("scale_bwd_kernel");
      return MHC_OK;
    });
  });
  if (rc != MHC_OK) return rc;
  float* part2 = (float*)workspace + (size_t)G * P;
  const int S = (int)std::min<int64_t>(kMixSplit, rows_used);
  const int rows = (int)ceil_div(rows_used, S);
  const int S_used = (int)ceil_div(rows_used, rows);
  hipLaunchKernelGGL(reduce_rows_kernel, dim3((unsigned)ceil_div(P / 4, 256), (unsigned)S_used),
                     dim3(256), 0, s, (const float*)workspace, part2, rows_used, P, rows);
  MHC_CHECK_LAUNCH("reduce_rows_kernel");
  hipLaunchKernelGGL(scale_final_kernel, dim3(1), dim3(64), 0, s, part2, S_used, P, n, h_mode, h_pre,
                     dh_pre);
  MHC_CHECK_LAUNCH("scale_final_kernel");
  return MHC_OK;
}
