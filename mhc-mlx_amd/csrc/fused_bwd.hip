// Fused mHC backward (the VJP of mhc_mlx/metal.py:2787-2857 / the MLX
// autograd of reference.py:148-184), for layer-wide or per-token parameters.
//
// With g = dout, a = activated H_pre, p = activated H_post, w = rms weight:
//   y   = sum_i a_i x_i                 inv = 1/sqrt(mean_c y^2 + eps)
//   dyn = sum_i p_i g_i                 d_r = sum_c dyn * y * w
//   dy  = dyn*inv*w - (inv^3/C)*d_r*y
//   dx_j  = sum_i M_ij g_i + a_j dy
//   dM_ij = sum g_i x_j   dA_j = sum dy x_j   dP_i = sum g_i y inv w
//   dw_c  = sum_t dyn * y * inv
//
// Stage 1 (bwd_tile_kernel and the specialised kernels): persistent
// workgroups, one token at a time.  One block reduction per token yields inv
// and d_r; then dx is written and the parameter-gradient contributions are
// accumulated.  Each workgroup finally writes one row of partial sums (dw over
// its tokens and, for layer-wide parameters, dM/dA/dP).  Per-token parameter
// gradients are reduced across the workgroup per token and written directly.
// Stage 2 (reduce kernels): fixed-order sum of the partial rows — the
// result is bitwise reproducible for a given device and shape.
#include <type_traits>

#include "mhc_device.hpp"
#include "mhc_generic.hpp"
#include "mhc_mfma32.hpp"
#include "mhc_host.hpp"
#include "mhc_plan.hpp"
#include "mhc_reduce.hpp"
#include "mhc_sinkhorn.hpp"

namespace mhc {

struct BwdArgs {
  const void* x;
  const void* g;
  void* dx;
  const float* M;
  const float* hpre;
  const float* hpost;
  const float* w;
  float* part;
  float* dM_tok;
  float* dpre_tok;
  float* dpost_tok;
  int64_t T;
  int64_t M_ts;
  int64_t h_ts;
  int n;
  int C;
  int Cp;
  int P;
  int nchunks;
  int reload;
  int h_mode;
  int vec;
  float eps;
};

constexpr int kReduceSplit = 64;

// ---------------------------------------------------------------------------
// Tile backward: every n <= 16 shape that the specialised kernels below do
// not take (fp32 or mixed dtypes above n = 8, n that is not 4, 8 or 16, C
// beyond the register-resident kernels, rows without 16-byte alignment).
//
// 256 threads, one token at a time (grid-stride).  Per token:
//   A. one pass over the token's chunks (V channels per thread) for the two
//      RMS sums, sum_c y^2 and sum_c dyn y w; a block reduction gives inv and
//      kf.  A token of one tile (C <= CT) is staged in LDS by this pass.
//   B. per tile of CT = 256 V channels:
//      (a) each thread takes its chunk of every stream again (from LDS for a
//          one-tile token, else from global memory) and forms y, dyn, dy, yn,
//          its dw term and dx; it writes x and g as fp32 rows of the tile
//          buffers, with yn and dy as one more row of each;
//      (b) after a barrier, the parameter sums are accumulated from LDS as
//          one product: [g; dy] [x; yn]^T holds dM (rows and columns < n),
//          dA (the dy row) and dP (the yn column).  Each thread owns one 4x4
//          block of that (NMAX+1)^2 matrix and one group of the tile's
//          4-channel steps, so it holds 16 sums.
// The sums run in a fixed order per thread and are then added over the
// channel groups in group order: the result is bitwise reproducible for a
// device and shape.  No NMAX needs scratch memory.
// ---------------------------------------------------------------------------
template <int NMAX>
struct TileCfg {
  static constexpr int V = NMAX == 16 ? 2 : 4;  // channels per thread and chunk
  static constexpr int CT = 256 * V;            // channels per tile
  static constexpr int RS = CT + 4;             // LDS row stride in floats: rows start 4 banks apart
  static constexpr int ROWS = NMAX + 1;         // the streams, then yn (x buffer) or dy (g buffer)
  static constexpr int NB = NMAX / 4 + 1;       // 4x4 blocks per side of the (NMAX+1)^2 sums
  static constexpr int G = 256 / (NB * NB);     // channel groups per block
  static constexpr int RED = 17;                // LDS stride of one thread's 16 sums in the final reduction
  static_assert(256 * RED <= ROWS * RS, "reduction scratch must fit in one tile buffer");
};
constexpr int kTileThreads = 256;

template <int NMAX, typename XT, typename GT, bool PT>
__global__ __launch_bounds__(kTileThreads) void bwd_tile_kernel(BwdArgs A) {
  using Cfg = TileCfg<NMAX>;
  constexpr int V = Cfg::V, CT = Cfg::CT, RS = Cfg::RS, ROWS = Cfg::ROWS, NB = Cfg::NB, G = Cfg::G;
  constexpr int RED = Cfg::RED;
  __shared__ __attribute__((aligned(16))) float s_x[ROWS * RS];  // x_j rows, then yn
  __shared__ __attribute__((aligned(16))) float s_g[ROWS * RS];  // g_i rows, then dy
  __shared__ float s_Mt[NMAX * NMAX];                               // s_Mt[j * NMAX + i] = M_ij
  __shared__ float s_a[NMAX], s_p[NMAX];
  __shared__ float s_sum[2][kTileThreads / 64];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = A.n;
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  const int nchunks = A.nchunks;
  const int ntiles = (C + CT - 1) / CT;
  const bool resident = ntiles == 1;
  const bool vec = A.vec != 0;
  const XT* __restrict__ X = (const XT*)A.x;
  const GT* __restrict__ Gr = (const GT*)A.g;
  XT* __restrict__ DX = (XT*)A.dx;
  const float* __restrict__ Wt = A.w;
  float* prow = A.part + (int64_t)blockIdx.x * A.P;

  // parameter-sum block (bi, bj) and channel group of this thread
  const int blk = tid / G;
  const int grp = tid - blk * G;
  const bool owner = blk < NB * NB;
  const int bi = owner ? blk / NB : 0;
  const int bj = owner ? blk - bi * NB : 0;
  float acc[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) acc[k] = 0.0f;
  float dwr[V];  // dw of this thread's channels, one-tile tokens
#pragma unroll
  for (int v = 0; v < V; ++v) dwr[v] = 0.0f;

  // rows n..NMAX-1 are never written and must read as zero
  for (int k = tid; k < ROWS * RS; k += kTileThreads) {
    s_x[k] = 0.0f;
    s_g[k] = 0.0f;
  }
  if (!resident)
    for (int c = tid; c < C; c += kTileThreads) prow[c] = 0.0f;

  auto stage_params = [&](int64_t t) {
    const float* Mp = A.M + t * A.M_ts;
    const float* hp = A.hpre + t * A.h_ts;
    const float* hq = A.hpost + t * A.h_ts;
    for (int idx = tid; idx < NMAX * NMAX + 2 * NMAX; idx += kTileThreads) {
      if (idx < NMAX * NMAX) {
        const int j = idx / NMAX, i = idx - j * NMAX;
        s_Mt[idx] = (i < n && j < n) ? Mp[i * n + j] : 0.0f;
      } else if (idx < NMAX * NMAX + NMAX) {
        const int i = idx - NMAX * NMAX;
        float v = 0.0f;
        if (i < n) v = A.h_mode == MHC_H_RAW ? sigmoidf_(hp[i]) : hp[i];
        s_a[i] = v;
      } else {
        const int i = idx - NMAX * NMAX - NMAX;
        float v = 0.0f;
        if (i < n) v = A.h_mode == MHC_H_RAW ? 2.0f * sigmoidf_(hq[i]) : hq[i];
        s_p[i] = v;
      }
    }
  };

  // the 16 sums of every thread added over the channel groups; emit(R, S, value) for each (R, S)
  // of the (NMAX+1)^2 matrix.  Uses s_x as scratch and leaves it zero; brackets itself with barriers.
  auto reduce_sums = [&](auto&& emit) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      s_x[tid * RED + k] = acc[k];
      acc[k] = 0.0f;
    }
    __syncthreads();
    for (int o = tid; o < NB * NB * 16; o += kTileThreads) {
      const int b = o >> 4, k = o & 15;
      float s = 0.0f;
      for (int q = 0; q < G; ++q) s += s_x[(b * G + q) * RED + k];
      const int bb = b / NB;
      emit(4 * bb + (k >> 2), 4 * (b - bb * NB) + (k & 3), s);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 16; ++k) s_x[tid * RED + k] = 0.0f;
    __syncthreads();
  };

  if (!PT) stage_params(0);
  __syncthreads();

  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x) {
    if constexpr (PT) {
      stage_params(t);
      __syncthreads();
    }
    const XT* xt = X + t * nC;
    const GT* gt = Gr + t * nC;
    XT* dxt = DX + t * nC;

    // ---- A: the RMS sums (cached loads: a token of several tiles is read again in B)
    float ss = 0.0f, sr = 0.0f;
    for (int q = tid; q < nchunks; q += kTileThreads) {
      const int c0 = q * V;
      const int valid = min(V, C - c0);
      float y[V], dyn[V];
#pragma unroll
      for (int v = 0; v < V; ++v) y[v] = dyn[v] = 0.0f;
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
        if (i < n) {
          Vec<XT, V> xv;
          Vec<GT, V> gv;
          if (vec && valid == V) {
            xv.template load<false>(xt + (int64_t)i * C + c0);
            gv.template load<false>(gt + (int64_t)i * C + c0);
          } else {
            xv.load_partial(xt + (int64_t)i * C + c0, valid);
            gv.load_partial(gt + (int64_t)i * C + c0, valid);
          }
          const float ai = s_a[i], pi = s_p[i];
#pragma unroll
          for (int v = 0; v < V; ++v) {
            const float xf = xv.get(v), gf = gv.get(v);
            y[v] = fmaf(ai, xf, y[v]);
            dyn[v] = fmaf(pi, gf, dyn[v]);
            if (resident) {
              s_x[i * RS + c0 + v] = xf;
              s_g[i * RS + c0 + v] = gf;
            }
          }
        }
      }
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float wv = v < valid ? Wt[c0 + v] : 0.0f;
        ss = fmaf(y[v], y[v], ss);
        sr = fmaf(dyn[v] * y[v], wv, sr);
      }
    }
    ss = wave_sum(ss);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_sum[0][wave] = ss;
      s_sum[1][wave] = sr;
    }
    __syncthreads();
    float tss = 0.0f, tsr = 0.0f;
#pragma unroll
    for (int w = 0; w < kTileThreads / 64; ++w) {
      tss += s_sum[0][w];
      tsr += s_sum[1][w];
    }
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;

    // ---- B: per tile, (a) dx, dw and the tile rows, (b) the parameter sums
    for (int tl = 0; tl < ntiles; ++tl) {
      const int cl = tid * V;
      const int c0 = tl * CT + cl;
      const int valid = max(0, min(V, C - c0));
      float y[V], dyn[V], gr[NMAX][V];
#pragma unroll
      for (int v = 0; v < V; ++v) y[v] = dyn[v] = 0.0f;
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
        float xf[V], gf[V];
#pragma unroll
        for (int v = 0; v < V; ++v) xf[v] = gf[v] = 0.0f;
        if (i < n && valid > 0) {
          if (resident) {
#pragma unroll
            for (int v = 0; v < V; ++v) {
              xf[v] = s_x[i * RS + cl + v];
              gf[v] = s_g[i * RS + cl + v];
            }
          } else {
            Vec<XT, V> xv;
            Vec<GT, V> gv;
            if (vec && valid == V) {
              xv.load(xt + (int64_t)i * C + c0);
              gv.load(gt + (int64_t)i * C + c0);
            } else {
              xv.load_partial(xt + (int64_t)i * C + c0, valid);
              gv.load_partial(gt + (int64_t)i * C + c0, valid);
            }
#pragma unroll
            for (int v = 0; v < V; ++v) {
              xf[v] = xv.get(v);
              gf[v] = gv.get(v);
            }
          }
        }
        const float ai = s_a[i], pi = s_p[i];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          y[v] = fmaf(ai, xf[v], y[v]);
          dyn[v] = fmaf(pi, gf[v], dyn[v]);
          gr[i][v] = gf[v];
        }
        if (!resident && i < n) {
#pragma unroll
          for (int v = 0; v < V; ++v) {
            s_x[i * RS + cl + v] = xf[v];
            s_g[i * RS + cl + v] = gf[v];
          }
        }
      }
      float dy[V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float wv = v < valid ? Wt[c0 + v] : 0.0f;
        const float yi = y[v] * inv;
        dy[v] = dyn[v] * inv * wv - kf * y[v];
        s_x[NMAX * RS + cl + v] = yi * wv;
        s_g[NMAX * RS + cl + v] = dy[v];
        const float dwt = dyn[v] * yi;
        if (resident) dwr[v] += dwt;
        else if (v < valid) prow[c0 + v] += dwt;
      }
      if (valid > 0) {
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
          if (j < n) {
            float o[V];
#pragma unroll
            for (int v = 0; v < V; ++v) {
              float s = 0.0f;
#pragma unroll
              for (int i = 0; i < NMAX; ++i) s = fmaf(s_Mt[j * NMAX + i], gr[i][v], s);
              o[v] = fmaf(s_a[j], dy[v], s);
            }
            XT* dst = dxt + (int64_t)j * C + c0;
            if (vec && valid == V) store_vec<XT, V>(dst, o);
            else store_partial<XT, V>(dst, o, valid);
          }
        }
      }
      __syncthreads();
      if (owner) {
        const int qend = (min(CT, C - tl * CT) + 3) >> 2;
        for (int q = grp; q < qend; q += G) {
          float4 gq[4], xq[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int R = 4 * bi + r;
            gq[r] = R < ROWS ? *reinterpret_cast<const float4*>(&s_g[R * RS + 4 * q]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            const int S = 4 * bj + r;
            xq[r] = S < ROWS ? *reinterpret_cast<const float4*>(&s_x[S * RS + 4 * q]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              float a = acc[4 * r + s];
              a = fmaf(gq[r].x, xq[s].x, a);
              a = fmaf(gq[r].y, xq[s].y, a);
              a = fmaf(gq[r].z, xq[s].z, a);
              a = fmaf(gq[r].w, xq[s].w, a);
              acc[4 * r + s] = a;
            }
        }
      }
      __syncthreads();
    }

    if constexpr (PT) {
      reduce_sums([&](int R, int S, float s) {
        if (R < n && S < n) {
          A.dM_tok[t * n * n + R * n + S] = s;
        } else if (R == NMAX && S < n) {
          const float av = s_a[S];
          A.dpre_tok[t * n + S] = A.h_mode == MHC_H_RAW ? s * av * (1.0f - av) : s;
        } else if (R < n && S == NMAX) {
          const float pq = s_p[R];
          A.dpost_tok[t * n + R] = A.h_mode == MHC_H_RAW ? s * pq * (1.0f - 0.5f * pq) : s;
        }
      });
    }
  }

  // ---- this workgroup's partial row: dw, then (layer-wide) dM, dA, dP
  if (resident) {
    const int c0 = tid * V;
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (c0 + v < C) prow[c0 + v] = dwr[v];
  }
  if (tid == 0)
    for (int c = C; c < A.Cp; ++c) prow[c] = 0.0f;
  if constexpr (!PT) {
    reduce_sums([&](int R, int S, float s) {
      if (R < n && S < n) prow[A.Cp + R * n + S] = s;
      else if (R == NMAX && S < n) prow[A.Cp + n * n + S] = s;
      else if (R < n && S == NMAX) prow[A.Cp + n * n + n + R] = s;
    });
    if (tid == 0)
      for (int c = A.Cp + n * n + 2 * n; c < A.P; ++c) prow[c] = 0.0f;
  }
}

// ---------------------------------------------------------------------------
// Layer-wide parameters, n <= 8: the headline shape (n = 4).
//
// Thread `tid` owns CHK chunks of V channels (chunk q = tid + k * blockDim.x)
// for every token the workgroup visits, so its slice of dw and the n^2 + 2n
// parameter-gradient sums stay in registers for the whole kernel.  x and g
// are held packed (two 16-bit elements per VGPR) across the RMS barrier and
// unpacked again after it; the fp32 copies of phase A are not kept live.
// With 16-bit x and g, dM_ij = sum g_i x_j runs on v_dot2 over the packed
// words (two channels per instruction, exact bf16/fp16 products, fp32 sum).
// ---------------------------------------------------------------------------

template <typename XT, typename GT>
struct LwCfg {
  static constexpr int kElem = ElemTraits<XT>::kBytes > ElemTraits<GT>::kBytes ? ElemTraits<XT>::kBytes
                                                                                : ElemTraits<GT>::kBytes;
};

template <int NMAX, typename XT, typename GT>
constexpr int lw_vec() {
  return 16 / LwCfg<XT, GT>::kElem;
}

// Largest workgroup of the layer-wide backward.  n <= 4 keeps a 1024-thread
// bound (128 VGPRs).  n = 8 (64 dM sums per thread) is bounded at 512
// threads, so it gets 256 VGPRs without spilling and 16-byte chunks.
constexpr int lw_max_threads(int nmax) { return nmax <= 4 ? 1024 : 512; }

template <typename T>
MHC_DEV float dot2_acc(uint32_t g, uint32_t x, float acc);
template <>
MHC_DEV float dot2_acc<__bf16>(uint32_t g, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, g), __builtin_bit_cast(bf16x2, x), acc,
                                         false);
}
template <>
MHC_DEV float dot2_acc<_Float16>(uint32_t g, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, g), __builtin_bit_cast(f16x2, x), acc, false);
}

// Opaque to the optimiser: forces values derived from `w` to be recomputed.
MHC_DEV void reg_fence(uint32_t& w) { asm volatile("" : "+v"(w)); }

// FULL: n == NMAX, 16-byte aligned rows and every owned chunk complete, so
// the token loop has no per-stream or per-chunk conditions.
// Waves per SIMD the layer-wide backward's registers are capped at (a
// build-time tuning knob).
#ifndef MHC_BWD_WPE
#define MHC_BWD_WPE 4
#endif

// PT: per-token parameters (M_ts = n*n, h_ts = n).  The token's M, a and p
// are loaded at the top of each token, and its dM, dA and dP sums go through
// the same wave + LDS reduction at the end of each token to the per-token
// outputs (dA and dP through the activation chain when RAW); only dw stays
// in registers across tokens.
//
// PIPE (layer-wide full tiles, n == 4): the next token's x and g are loaded
// right after this token's phase A, into a second set of registers, so they
// are in flight across the barrier and phase B and are issued before this
// token's dx stores.  On gfx9 a vmcnt wait counts stores as well: loads
// issued after the stores would make the next token's first wait also wait
// for this token's stores.  The second register set (32 VGPRs) bounds the
// workgroup at 512 threads and three waves per SIMD, i.e. one workgroup per
// CU, which the overlap more than pays for (config 2: 565 -> 559 us at one
// workgroup per CU against two).
template <int NMAX, typename XT, typename GT, int CHK, bool FULL, bool PT = false, bool PIPE = false>
__global__ __attribute__((amdgpu_flat_work_group_size(64, (PIPE || !FULL) ? 512 : lw_max_threads(NMAX)),
                          amdgpu_waves_per_eu(PIPE ? 3 : (NMAX <= 4 && FULL ? MHC_BWD_WPE : 2))))
void fused_bwd_lw_kernel(BwdArgs A) {
  static_assert(!PIPE || (FULL && !PT), "pipelined loads for layer-wide full tiles only");
  constexpr int V = lw_vec<NMAX, XT, GT>();
  constexpr int K = NMAX * NMAX + 2 * NMAX;
  constexpr bool DOT = std::is_same<XT, GT>::value && ElemTraits<XT>::kBytes == 2;
  __shared__ float s_red[2][2][16];
  __shared__ float s_acc[16][K];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int n = FULL ? NMAX : A.n;
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  const XT* __restrict__ X = (const XT*)A.x;
  const GT* __restrict__ Gr = (const GT*)A.g;
  XT* __restrict__ DX = (XT*)A.dx;
  float* prow = A.part + (int64_t)blockIdx.x * A.P;

  float Ms[NMAX * NMAX], as[NMAX], ps[NMAX];
  auto load_params = [&](const float* Mt, const float* hp, const float* hq) {
#pragma unroll
    for (int i = 0; i < NMAX; ++i) {
      float av = 0.0f, pq = 0.0f;
      if (i < n) {
        av = hp[i];
        pq = hq[i];
        if (A.h_mode == MHC_H_RAW) {
          av = sigmoidf_(av);
          pq = 2.0f * sigmoidf_(pq);
        }
      }
      as[i] = uniform_f(av);
      ps[i] = uniform_f(pq);
#pragma unroll
      for (int j = 0; j < NMAX; ++j) Ms[i * NMAX + j] = uniform_f((i < n && j < n) ? Mt[i * n + j] : 0.0f);
    }
  };
  if constexpr (!PT) load_params(A.M, A.hpre, A.hpost);

  int c0[CHK], valid[CHK];
  float wv[CHK][V], dwv[CHK][V];
#pragma unroll
  for (int k = 0; k < CHK; ++k) {
    const int q = tid + k * blockDim.x;
    c0[k] = q * V;
    valid[k] = FULL ? V : (q < A.nchunks ? min(V, C - c0[k]) : 0);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      wv[k][v] = v < valid[k] ? A.w[c0[k] + v] : 0.0f;
      dwv[k][v] = 0.0f;
    }
  }
  float accM[NMAX * NMAX], accA[NMAX], accP[NMAX];
#pragma unroll
  for (int k = 0; k < NMAX * NMAX; ++k) accM[k] = 0.0f;
#pragma unroll
  for (int k = 0; k < NMAX; ++k) accA[k] = accP[k] = 0.0f;

  auto load_tok = [&](Vec<XT, V> (&xa)[CHK][NMAX], Vec<GT, V> (&ga)[CHK][NMAX], int64_t t) {
    const XT* xt = X + t * nC;
    const GT* gt = Gr + t * nC;
#pragma unroll
    for (int k = 0; k < CHK; ++k) {
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
        if (FULL || (i < n && valid[k] == V && A.vec)) {
          xa[k][i].load(xt + (int64_t)i * C + c0[k]);
          ga[k][i].load(gt + (int64_t)i * C + c0[k]);
        } else if (i < n && valid[k] > 0) {
          xa[k][i].load_partial(xt + (int64_t)i * C + c0[k], valid[k]);
          ga[k][i].load_partial(gt + (int64_t)i * C + c0[k], valid[k]);
        } else {
          xa[k][i].zero();
          ga[k][i].zero();
        }
      }
    }
  };
  Vec<XT, V> xr[CHK][NMAX];
  Vec<GT, V> gr[CHK][NMAX];
  if constexpr (PIPE) {
    if ((int64_t)blockIdx.x < A.T) load_tok(xr, gr, blockIdx.x);
    // wait for the first token here: entering the loop with its loads pending
    // (no stores issued after them) would make the loop-top waits of every
    // token as strict as the first one's, i.e. wait for the previous token's
    // dx stores
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
  }

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    XT* dxt = DX + t * nC;
    if constexpr (PT) load_params(A.M + t * A.M_ts, A.hpre + t * A.h_ts, A.hpost + t * A.h_ts);
    if constexpr (!PIPE) load_tok(xr, gr, t);
    // ---- phase A: y, dyn and the per-token sums  sum y^2, sum dyn*y*w
    float y[CHK][V], dyn[CHK][V];
    float ss = 0.0f, sr = 0.0f;
#pragma unroll
    for (int k = 0; k < CHK; ++k) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        float ya = 0.0f, da = 0.0f;
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          ya = fmaf(as[i], xr[k][i].get(v), ya);
          da = fmaf(ps[i], gr[k][i].get(v), da);
        }
        y[k][v] = ya;
        dyn[k][v] = da;
        ss = fmaf(ya, ya, ss);
        sr = fmaf(da * ya, wv[k][v], sr);
      }
    }
    ss = wave_sum(ss);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_red[it & 1][0][wave] = ss;
      s_red[it & 1][1][wave] = sr;
    }
    Vec<XT, V> xn[CHK][NMAX];
    Vec<GT, V> gn[CHK][NMAX];
    if constexpr (PIPE) {
      if (t + gridDim.x < A.T) load_tok(xn, gn, t + gridDim.x);
    }
    lds_barrier();
    float tss = 0.0f, tsr = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
      tss += s_red[it & 1][0][w];
      tsr += s_red[it & 1][1][w];
    }
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;

    // ---- phase B: dx, dw and the parameter-gradient sums, two channels
    // at a time so dx is packed as it is produced (only the packed dx words
    // of one chunk are live, never n*V fp32 values).
#pragma unroll
    for (int k = 0; k < CHK; ++k) {
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
#pragma unroll
        for (int w = 0; w < Vec<XT, V>::kWords; ++w) reg_fence(xr[k][i].w[w]);
#pragma unroll
        for (int w = 0; w < Vec<GT, V>::kWords; ++w) reg_fence(gr[k][i].w[w]);
      }
      float dxo[NMAX][V];
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float yi = y[k][v] * inv;
        const float dy = dyn[k][v] * inv * wv[k][v] - kf * y[k][v];
        const float yn = yi * wv[k][v];
        dwv[k][v] = fmaf(dyn[k][v], yi, dwv[k][v]);
        float gs[NMAX], xs[NMAX];
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          gs[i] = gr[k][i].get(v);
          xs[i] = xr[k][i].get(v);
        }
        // dx_j = sum_i M_ij g_i + a_j dy
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
          float acc = as[j] * dy;
#pragma unroll
          for (int i = 0; i < NMAX; ++i) acc = fmaf(Ms[i * NMAX + j], gs[i], acc);
          dxo[j][v] = acc;
        }
        // dA_j += dy x_j,  dP_i += g_i yn  (and dM without dot2)
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          accA[i] = fmaf(dy, xs[i], accA[i]);
          accP[i] = fmaf(gs[i], yn, accP[i]);
        }
        if constexpr (!DOT) {
#pragma unroll
          for (int i = 0; i < NMAX; ++i) {
#pragma unroll
            for (int j = 0; j < NMAX; ++j) accM[i * NMAX + j] = fmaf(gs[i], xs[j], accM[i * NMAX + j]);
          }
        } else if (v & 1) {
          const int w = v >> 1;
#pragma unroll
          for (int i = 0; i < NMAX; ++i) {
#pragma unroll
            for (int j = 0; j < NMAX; ++j)
              accM[i * NMAX + j] = dot2_acc<XT>(gr[k][i].w[w], xr[k][j].w[w], accM[i * NMAX + j]);
          }
        }
      }
      if (FULL || valid[k] > 0) {
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
          if (FULL || j < n) {
            XT* dst = dxt + (int64_t)j * C + c0[k];
            if (FULL || (A.vec && valid[k] == V)) store_vec<XT, V>(dst, dxo[j]);
            else store_partial<XT, V>(dst, dxo[j], valid[k]);
          }
        }
      }
    }
    if constexpr (PT) {
      // the token's parameter sums: wave sums, then the waves in order
#pragma unroll
      for (int k = 0; k < NMAX * NMAX; ++k) {
        const float v = wave_sum(accM[k]);
        accM[k] = 0.0f;
        if (lane == 0) s_acc[wave][k] = v;
      }
#pragma unroll
      for (int k = 0; k < NMAX; ++k) {
        const float va = wave_sum(accA[k]), vp = wave_sum(accP[k]);
        accA[k] = accP[k] = 0.0f;
        if (lane == 0) {
          s_acc[wave][NMAX * NMAX + k] = va;
          s_acc[wave][NMAX * NMAX + NMAX + k] = vp;
        }
      }
      __syncthreads();
      for (int k = tid; k < K; k += blockDim.x) {
        float sum = 0.0f;
        for (int w = 0; w < nwaves; ++w) sum += s_acc[w][k];
        if (k < NMAX * NMAX) {
          const int i = k / NMAX, j = k % NMAX;
          if (i < n && j < n) A.dM_tok[t * n * n + i * n + j] = sum;
        } else if (k < NMAX * NMAX + NMAX) {
          const int j = k - NMAX * NMAX;
          if (j < n) {
            const float av = as[j];
            A.dpre_tok[t * n + j] = A.h_mode == MHC_H_RAW ? sum * av * (1.0f - av) : sum;
          }
        } else {
          const int i = k - NMAX * NMAX - NMAX;
          if (i < n) {
            const float pq = ps[i];
            A.dpost_tok[t * n + i] = A.h_mode == MHC_H_RAW ? sum * pq * (1.0f - 0.5f * pq) : sum;
          }
        }
      }
    }
    if constexpr (PIPE) {
#pragma unroll
      for (int k = 0; k < CHK; ++k)
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          xr[k][i] = xn[k][i];
          gr[k][i] = gn[k][i];
        }
    }
  }

  // ---- this workgroup's partial row: dw slice, then wave and block sums
#pragma unroll
  for (int k = 0; k < CHK; ++k) {
#pragma unroll
    for (int v = 0; v < V; ++v)
      if (v < valid[k]) prow[c0[k] + v] = dwv[k][v];
  }
  if (tid == 0)
    for (int c = C; c < A.Cp; ++c) prow[c] = 0.0f;
  if constexpr (PT) return;  // per-token sums are already out; the row is dw only
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float v = k < NMAX * NMAX ? accM[k] : (k < NMAX * NMAX + NMAX ? accA[k - NMAX * NMAX]
                                                                        : accP[k - NMAX * NMAX - NMAX]);
    const float s = wave_sum(v);
    if (lane == 0) s_acc[wave][k] = s;
  }
  __syncthreads();
  for (int k = tid; k < K; k += blockDim.x) {
    float s = 0.0f;
    for (int w = 0; w < nwaves; ++w) s += s_acc[w][k];
    int dst = -1;
    if (k < NMAX * NMAX) {
      const int i = k / NMAX, j = k % NMAX;
      if (i < n && j < n) dst = i * n + j;
    } else if (k < NMAX * NMAX + NMAX) {
      if (k - NMAX * NMAX < n) dst = n * n + (k - NMAX * NMAX);
    } else {
      if (k - NMAX * NMAX - NMAX < n) dst = n * n + n + (k - NMAX * NMAX - NMAX);
    }
    if (dst >= 0) prow[A.Cp + dst] = s;
  }
  if (tid == 0)
    for (int c = A.Cp + n * n + 2 * n; c < A.P; ++c) prow[c] = 0.0f;
}

// ---------------------------------------------------------------------------
// Per-token parameters, n == 16, 16-bit x and dout, C <= 1024 (config 3).
//
// Per token the parameter gradients are n^2 + 2n = 288 sums over C
// channels; the n x n block dM = G X^T is a GEMM with K = C and runs on
// MFMA (v_mfma_f32_16x16x16 bf16/fp16: exact 16-bit products, fp32
// accumulation).  Thread `tid` owns channels [4 tid, 4 tid + 4) of every
// stream (8-byte coalesced loads).  Each wave copies its 256-channel slice of
// x and g into LDS rows (one row per stream, padded by 16 bytes) and
// accumulates dM over that slice with 16 MFMA steps; the four slices are
// added in wave order after a second barrier.  dx, dy and the dw
// accumulation stay on the VALU with M read as LDS broadcasts; dA and dP are
// reduce-scattered across each wave.  Parameters of the next token are
// staged in a three-slot LDS ring while the current one is processed.
// ---------------------------------------------------------------------------

constexpr int kPt16Row = 256 + 8;  // 16-bit elements per LDS row: 256 channels + 16-byte pad
constexpr int kPt16K = 16 * 16 + 2 * 16;

template <typename XT>
MHC_DEV void pt16_stage(float* buf, const BwdArgs& A, int64_t t) {
  // buf: M^T [16][16] (buf[j*16 + i] = M[i][j]), a [16], p [16]
  const float* M = A.M + t * 256;
  for (int k = threadIdx.x; k < kPt16K; k += blockDim.x) {
    if (k < 256) {
      buf[(k & 15) * 16 + (k >> 4)] = M[k];
    } else if (k < 272) {
      const float h = A.hpre[t * 16 + (k - 256)];
      buf[k] = A.h_mode == MHC_H_RAW ? sigmoidf_(h) : h;
    } else {
      const float h = A.hpost[t * 16 + (k - 272)];
      buf[k] = A.h_mode == MHC_H_RAW ? 2.0f * sigmoidf_(h) : h;
    }
  }
}

template <typename XT>
__global__ __launch_bounds__(256) void fused_bwd_pt16_kernel(BwdArgs A) {
  constexpr int N = 16, V = 4;
  __shared__ uint16_t s_x[4][N][kPt16Row];
  __shared__ uint16_t s_g[4][N][kPt16Row];
  __shared__ float s_par[3][kPt16K];
  // written after the first barrier of a token and read before the first
  // barrier of the next one: one buffer suffices
  __shared__ float s_part[4][256];
  __shared__ float s_rows[4][4][32];
  __shared__ float s_red[2][2][4];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int C = A.C;
  const int c0 = tid * V;
  const int64_t nC = (int64_t)N * C;
  float* prow = A.part + (int64_t)blockIdx.x * A.P;

  float wv[V], dwv[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    wv[v] = A.w[c0 + v];
    dwv[v] = 0.0f;
  }
  if ((int64_t)blockIdx.x < A.T) pt16_stage<XT>(s_par[0], A, blockIdx.x);
  __syncthreads();

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const float* par = s_par[it % 3];
    const int64_t tn = t + gridDim.x;
    if (tn < A.T) pt16_stage<XT>(s_par[(it + 1) % 3], A, tn);
    const uint2* xt = reinterpret_cast<const uint2*>((const XT*)A.x + t * nC + c0);
    const uint2* gt = reinterpret_cast<const uint2*>((const XT*)A.g + t * nC + c0);
    uint2 xr[N], gr[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const u32x2 u = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(xt + (int64_t)i * (C / V)));
      const u32x2 q = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(gt + (int64_t)i * (C / V)));
      xr[i] = make_uint2(u.x, u.y);
      gr[i] = make_uint2(q.x, q.y);
    }
    // this wave's slice of x and g, row = stream, for the MFMA below
#pragma unroll
    for (int i = 0; i < N; ++i) {
      *reinterpret_cast<uint2*>(&s_x[wave][i][lane * V]) = xr[i];
      *reinterpret_cast<uint2*>(&s_g[wave][i][lane * V]) = gr[i];
    }
    // y, dyn and the two per-token sums
    float y[V], dyn[V];
    float ss = 0.0f, sr = 0.0f;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float ya = 0.0f, da = 0.0f;
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const uint32_t wx = (v & 2) ? xr[i].y : xr[i].x;
        const uint32_t wg = (v & 2) ? gr[i].y : gr[i].x;
        ya = fmaf(par[256 + i], (v & 1) ? hi16<XT>(wx) : lo16<XT>(wx), ya);
        da = fmaf(par[272 + i], (v & 1) ? hi16<XT>(wg) : lo16<XT>(wg), da);
      }
      y[v] = ya;
      dyn[v] = da;
      ss = fmaf(ya, ya, ss);
      sr = fmaf(da * ya, wv[v], sr);
    }
    ss = wave_sum(ss);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_red[it & 1][0][wave] = ss;
      s_red[it & 1][1][wave] = sr;
    }
    __syncthreads();
    float tss = 0.0f, tsr = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
      tss += s_red[it & 1][0][w];
      tsr += s_red[it & 1][1][w];
    }
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;
    float dy[V], yn[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const float yi = y[v] * inv;
      dy[v] = dyn[v] * inv * wv[v] - kf * y[v];
      yn[v] = yi * wv[v];
      dwv[v] = fmaf(dyn[v], yi, dwv[v]);
    }
    // dx_j = sum_i M_ij g_i + a_j dy  (M^T rows are LDS broadcasts)
    XT* dxt = (XT*)A.dx + t * nC + c0;
#pragma unroll 4
    for (int j = 0; j < N; ++j) {
      const float aj = par[256 + j];
      float o[V];
#pragma unroll
      for (int v = 0; v < V; ++v) o[v] = aj * dy[v];
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const float m = par[j * 16 + i];
        o[0] = fmaf(m, lo16<XT>(gr[i].x), o[0]);
        o[1] = fmaf(m, hi16<XT>(gr[i].x), o[1]);
        o[2] = fmaf(m, lo16<XT>(gr[i].y), o[2]);
        o[3] = fmaf(m, hi16<XT>(gr[i].y), o[3]);
      }
      st_nt(reinterpret_cast<uint32_t*>(dxt + (int64_t)j * C), pack2<XT>(o[0], o[1]), pack2<XT>(o[2], o[3]));
    }
    // dA_j = sum dy x_j, dP_i = sum g_i yn: lane partials summed across each
    // 16-lane row (DPP), then one value per lane goes to LDS; the four rows
    // and four waves are added after the barrier
    {
      float oa = 0.0f, op = 0.0f;
      const int r = lane & 15;
#pragma unroll
      for (int i = 0; i < N; ++i) {
        float sa = 0.0f, sp = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
          const uint32_t wx = (v & 2) ? xr[i].y : xr[i].x;
          const uint32_t wg = (v & 2) ? gr[i].y : gr[i].x;
          sa = fmaf(dy[v], (v & 1) ? hi16<XT>(wx) : lo16<XT>(wx), sa);
          sp = fmaf((v & 1) ? hi16<XT>(wg) : lo16<XT>(wg), yn[v], sp);
        }
        sa = group_sum<16>(sa);
        sp = group_sum<16>(sp);
        oa = r == i ? sa : oa;
        op = r == i ? sp : op;
      }
      s_rows[wave][lane >> 4][r] = oa;
      s_rows[wave][lane >> 4][16 + r] = op;
    }
    // dM over this wave's 256 channels on MFMA: A = G (rows i), B = X^T
    {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      const int r = lane & 15;
      const int kq = 4 * (lane >> 4);
#pragma unroll
      for (int ks = 0; ks < 16; ++ks) {
        const uint2 a = *reinterpret_cast<const uint2*>(&s_g[wave][r][ks * 16 + kq]);
        const uint2 b = *reinterpret_cast<const uint2*>(&s_x[wave][r][ks * 16 + kq]);
        acc = mfma16<XT>(a, b, acc);
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) s_part[wave][(kq + v) * 16 + r] = acc[v];
    }
    __syncthreads();
    for (int k = tid; k < kPt16K; k += blockDim.x) {
      float s = 0.0f;
      if (k < 256) {
        for (int w = 0; w < nwaves; ++w) s += s_part[w][k];
      } else {
        for (int w = 0; w < nwaves; ++w)
          s += (s_rows[w][0][k - 256] + s_rows[w][1][k - 256]) + (s_rows[w][2][k - 256] + s_rows[w][3][k - 256]);
      }
      if (k < 256) {
        A.dM_tok[t * 256 + k] = s;
      } else if (k < 272) {
        const float av = par[k];
        A.dpre_tok[t * 16 + (k - 256)] = A.h_mode == MHC_H_RAW ? s * av * (1.0f - av) : s;
      } else {
        const float pq = par[k];
        A.dpost_tok[t * 16 + (k - 272)] = A.h_mode == MHC_H_RAW ? s * pq * (1.0f - 0.5f * pq) : s;
      }
    }
  }
#pragma unroll
  for (int v = 0; v < V; ++v) prow[c0 + v] = dwv[v];
}

// ---------------------------------------------------------------------------
// n == 16, 16-bit x == dout, C a multiple of 128: every 16 x 16 contraction
// on MFMA (per-token parameters, config 3; layer-wide n == 16 uses the
// generic kernel).
//
// Lane layout as in the MFMA forward (fused_fwd.hip): wave w owns SPW
// 128-channel slabs; per slab, lane (q = lane >> 4, r = lane & 15) loads
// streams 4q .. 4q+3 of channels [8r, 8r + 8) of x and of g (16-byte loads).
// Two slabs per wave halve the per-wave work that does not scale with the
// channels (parameter activations and splits, the per-token sums).  Per channel v of that range
// the B operands are streams 4q .. 4q+3 of channel 8r + v, and
//   y   = a^T X,  dyn = p^T G                  (before the RMS barrier)
//   dx  = M^T G + a dy                          (after it; a dy is the C input)
// with M, a, p split into three 16-bit terms (split3), so the products are
// those of the fp32 parameters with the 16-bit data.  dM = G X^T has K = C:
// each wave stages its slab of x and g in LDS as rows of one stream and
// accumulates dM over its channels with 8 MFMAs; the waves' parts are added
// in wave order.  After the RMS barrier the lane reads its x and g back from
// that slab instead of keeping them in registers across the barrier.  Both
// per-token barriers order LDS data only (lds_barrier): a full
// __syncthreads() would also wait for the token's dx stores.  dA and dP are lane partials summed across each
// 16-lane row (DPP) and across waves in order; dw stays in registers across
// the tokens of the (persistent) workgroup and ends in its partial row.
// ---------------------------------------------------------------------------

constexpr int kMf16Row = 128 + 8;  // LDS row (16-bit elements): 68 dwords, 4 mod 64 banks
constexpr int kMf16MaxWaves = 8;

// LW: layer-wide parameters (one M, a, p for every token).  The token's dM,
// dA and dP are then added into per-thread sums across the workgroup's
// tokens and end in its partial row after the dw slice, unactivated (the
// reduction applies the activation chain to the totals).
// WIDE: two slabs per wave with up to 8 waves, C up to 2048 (one workgroup
// per CU: its staged slabs take ~140 KB of LDS).
// PIPE: the next token's x and g are loaded once this token's slabs are
// staged (the registers are free then), so the loads are in flight across
// the RMS barrier and the dx pass, and are issued before this token's dx
// stores (a vmcnt wait counts stores too: loads issued after them would
// wait for them).
template <typename XT, int SPW, bool RAW, bool LW, bool WIDE = false, bool PIPE = false>
__global__ __launch_bounds__(SPW == 2 && !WIDE ? 256 : 512) __attribute__((amdgpu_waves_per_eu(2)))
void fused_bwd_mfma16_kernel(BwdArgs A) {
  constexpr int N = 16;
  constexpr int64_t PS = LW ? 0 : 16;   // parameter strides per token
  constexpr int64_t MS = LW ? 0 : 256;
  constexpr int KP = 256 + 32;          // dM, dA, dP of a token
  constexpr int KPT = (KP + 63) / 64;   // k per thread at 64 threads
  float lw_acc[KPT];                    // LW: sums of k = tid + e * blockDim.x
#pragma unroll
  for (int e = 0; e < KPT; ++e) lw_acc[e] = 0.0f;
  constexpr int SLAB = 2 * N * kMf16Row;  // 16-bit elements of one staged slab (x rows, then g rows)
  extern __shared__ uint16_t mf_lds[];
  constexpr int MW = SPW == 2 && !WIDE ? 4 : kMf16MaxWaves;  // waves per workgroup at most
  __shared__ float s_red[2][2][MW];
  __shared__ float s_dm[MW][256];
  __shared__ float s_ap[MW][32];
  __shared__ float s_act[2][32];  // activated a, p of the token (parity-buffered)
  __shared__ __align__(16) float s_w[WIDE ? 2048 : 1024];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int C = A.C;
  const int64_t nC = (int64_t)N * C;
  uint16_t* slab_lds = mf_lds + (size_t)wave * SPW * SLAB;
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  int cb[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) cb[s] = (wave * SPW + s) * 128 + 8 * r;

  float dwv[SPW][8];
#pragma unroll
  for (int s = 0; s < SPW; ++s)
#pragma unroll
    for (int v = 0; v < 8; ++v) dwv[s][v] = 0.0f;
  // rms weight of the workgroup's channels, staged once
  for (int c = tid; c < C; c += blockDim.x) s_w[c] = A.w[c];

  // the token's parameters are loaded one token ahead (registers): a, p of
  // streams 4q..4q+3 and column r of M, rows 4q..4q+3
  float4 nh = make_float4(0.f, 0.f, 0.f, 0.f), ng = nh, nm = nh;
  if ((int64_t)blockIdx.x < A.T) {
    const int64_t t0 = blockIdx.x;
    nh = *reinterpret_cast<const float4*>(A.hpre + t0 * PS + 4 * q);
    ng = *reinterpret_cast<const float4*>(A.hpost + t0 * PS + 4 * q);
    const float* M0 = A.M + t0 * MS + (4 * q) * 16 + r;
    nm = make_float4(M0[0], M0[16], M0[32], M0[48]);
  }
  Vec<XT, 8> xr[SPW][4], gr[SPW][4];
  auto load_tok = [&](int64_t t) {
    const XT* xt = (const XT*)A.x + t * nC;
    const XT* gt = (const XT*)A.g + t * nC;
#pragma unroll
    for (int s = 0; s < SPW; ++s)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        xr[s][k].load(xt + (int64_t)(4 * q + k) * C + cb[s]);
        gr[s][k].load(gt + (int64_t)(4 * q + k) * C + cb[s]);
      }
  };
  if constexpr (PIPE) {
    if ((int64_t)blockIdx.x < A.T) load_tok(blockIdx.x);
  }
  __syncthreads();

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const float4 h4 = nh, g4 = ng, m4 = nm;
    float y[SPW][8], dyn[SPW][8];
    float ss = 0.0f, sr = 0.0f;
    f32x4 dm = {0.0f, 0.0f, 0.0f, 0.0f};
    float av[4];
    {
      if constexpr (!PIPE) load_tok(t);
      {
        const int64_t tn = t + gridDim.x;
        if (tn < A.T) {
          nh = *reinterpret_cast<const float4*>(A.hpre + tn * PS + 4 * q);
          ng = *reinterpret_cast<const float4*>(A.hpost + tn * PS + 4 * q);
          const float* Mn = A.M + tn * MS + (4 * q) * 16 + r;
          nm = make_float4(Mn[0], Mn[16], Mn[32], Mn[48]);
        }
      }
      float pv[4];
      av[0] = h4.x; av[1] = h4.y; av[2] = h4.z; av[3] = h4.w;
      pv[0] = g4.x; pv[1] = g4.y; pv[2] = g4.z; pv[3] = g4.w;
      if constexpr (RAW) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          av[k] = sigmoid_fast(av[k]);
          pv[k] = 2.0f * sigmoid_fast(pv[k]);
        }
      }
      if (wave == 0 && r == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          s_act[it & 1][4 * q + k] = av[k];
          s_act[it & 1][16 + 4 * q + k] = pv[k];
        }
      }
      uint2 aa[3], ap[3];
      split3x4<XT>(av, aa);
      split3x4<XT>(pv, ap);
#pragma unroll
      for (int s = 0; s < SPW; ++s) {
        uint16_t* sx = slab_lds + s * SLAB;
        uint16_t* sg = sx + N * kMf16Row;
        const float4 w0 = *reinterpret_cast<const float4*>(&s_w[cb[s]]);
        const float4 w1 = *reinterpret_cast<const float4*>(&s_w[cb[s] + 4]);
        const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        // stage the slab (one LDS row per stream): dM below, dx / dA / dP after the barrier
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          *reinterpret_cast<uint4*>(&sx[(4 * q + k) * kMf16Row + 8 * r]) =
              make_uint4(xr[s][k].w[0], xr[s][k].w[1], xr[s][k].w[2], xr[s][k].w[3]);
          *reinterpret_cast<uint4*>(&sg[(4 * q + k) * kMf16Row + 8 * r]) =
              make_uint4(gr[s][k].w[0], gr[s][k].w[1], gr[s][k].w[2], gr[s][k].w[3]);
        }
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int wd = v >> 1;
          uint2 bx, bg;
          if (v & 1) {
            bx = make_uint2(pack_hi16<XT>(xr[s][0].w[wd], xr[s][1].w[wd]), pack_hi16<XT>(xr[s][2].w[wd], xr[s][3].w[wd]));
            bg = make_uint2(pack_hi16<XT>(gr[s][0].w[wd], gr[s][1].w[wd]), pack_hi16<XT>(gr[s][2].w[wd], gr[s][3].w[wd]));
          } else {
            bx = make_uint2(pack_lo16<XT>(xr[s][0].w[wd], xr[s][1].w[wd]), pack_lo16<XT>(xr[s][2].w[wd], xr[s][3].w[wd]));
            bg = make_uint2(pack_lo16<XT>(gr[s][0].w[wd], gr[s][1].w[wd]), pack_lo16<XT>(gr[s][2].w[wd], gr[s][3].w[wd]));
          }
          f32x4 accy = {0.0f, 0.0f, 0.0f, 0.0f}, accd = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int e = 2; e >= 0; --e) {
            accy = mfma16<XT>(aa[e], bx, accy);
            accd = mfma16<XT>(ap[e], bg, accd);
          }
          y[s][v] = accy[0];
          dyn[s][v] = accd[0];
          ss = fmaf(accy[0], accy[0], ss);
          sr = fmaf(accd[0] * accy[0], wv[v], sr);
        }
        // dM over the slab: A = G rows (stream i), B = X^T, K = 16 channels per step
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const uint2 a = *reinterpret_cast<const uint2*>(&sg[r * kMf16Row + 16 * kk + 4 * q]);
          const uint2 b = *reinterpret_cast<const uint2*>(&sx[r * kMf16Row + 16 * kk + 4 * q]);
          dm = mfma16<XT>(a, b, dm);
        }
      }
    }
    if constexpr (PIPE) {
      if (t + gridDim.x < A.T) load_tok(t + gridDim.x);
    }
    // the four lanes of a column hold the same y and dyn: count them once
    ss = q == 0 ? ss : 0.0f;
    sr = q == 0 ? sr : 0.0f;
    ss = wave_sum(ss);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_red[it & 1][0][wave] = ss;
      s_red[it & 1][1][wave] = sr;
    }
    lds_barrier();
    // s_dm / s_ap are written after this barrier and read after the next one:
    // a wave can only write them again once every wave has passed this
    // barrier of the following token, i.e. finished reading them.
#pragma unroll
    for (int k = 0; k < 4; ++k) s_dm[wave][(4 * q + k) * 16 + r] = dm[k];
    float tss = 0.0f, tsr = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
      tss += s_red[it & 1][0][w];
      tsr += s_red[it & 1][1][w];
    }
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;

    // column r of M (rows 4q..4q+3) as the A operand of M^T
    uint2 amt[3];
    {
      const float mv[4] = {m4.x, m4.y, m4.z, m4.w};
      split3x4<XT>(mv, amt);
    }
    float dA[4] = {0.0f, 0.0f, 0.0f, 0.0f}, dP[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    XT* dxt = (XT*)A.dx + t * nC;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const uint16_t* sx = slab_lds + s * SLAB;
      const uint16_t* sg = sx + N * kMf16Row;
      const float4 w0 = *reinterpret_cast<const float4*>(&s_w[cb[s]]);
      const float4 w1 = *reinterpret_cast<const float4*>(&s_w[cb[s] + 4]);
      const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      // dy, yn (and the dw contribution) per channel
      float dyv[8], ynv[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const float yi = y[s][v] * inv;
        dyv[v] = dyn[s][v] * inv * wv[v] - kf * y[s][v];
        ynv[v] = yi * wv[v];
        dwv[s][v] = fmaf(dyn[s][v], yi, dwv[s][v]);
      }
      {
        // dx = M^T g + a dy on MFMA (a dy enters as the accumulator), and dP, from g
        Vec<XT, 8> gr[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint4 ug = *reinterpret_cast<const uint4*>(&sg[(4 * q + k) * kMf16Row + 8 * r]);
          gr[k].w[0] = ug.x; gr[k].w[1] = ug.y; gr[k].w[2] = ug.z; gr[k].w[3] = ug.w;
        }
        uint32_t ow[4][4];
        f32x4 even;  // dx of the even channel, packed with the odd one (one cvt per pair)
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int wd = v >> 1;
          uint2 bg;
          if (v & 1)
            bg = make_uint2(pack_hi16<XT>(gr[0].w[wd], gr[1].w[wd]), pack_hi16<XT>(gr[2].w[wd], gr[3].w[wd]));
          else
            bg = make_uint2(pack_lo16<XT>(gr[0].w[wd], gr[1].w[wd]), pack_lo16<XT>(gr[2].w[wd], gr[3].w[wd]));
          f32x4 acc = {av[0] * dyv[v], av[1] * dyv[v], av[2] * dyv[v], av[3] * dyv[v]};
#pragma unroll
          for (int e = 2; e >= 0; --e) acc = mfma16<XT>(amt[e], bg, acc);
          if (v & 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) ow[k][wd] = pack2<XT>(even[k], acc[k]);
          } else {
            even = acc;
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
          st_nt(reinterpret_cast<uint32_t*>(dxt + (int64_t)(4 * q + k) * C + cb[s]), ow[k][0], ow[k][1], ow[k][2],
                ow[k][3]);
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int v = 0; v < 8; ++v) dP[k] = fmaf(gr[k].get(v), ynv[v], dP[k]);
      }
      // dA from x, one stream row at a time
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        Vec<XT, 8> xv;
        const uint4 ux = *reinterpret_cast<const uint4*>(&sx[(4 * q + k) * kMf16Row + 8 * r]);
        xv.w[0] = ux.x; xv.w[1] = ux.y; xv.w[2] = ux.z; xv.w[3] = ux.w;
#pragma unroll
        for (int v = 0; v < 8; ++v) dA[k] = fmaf(dyv[v], xv.get(v), dA[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      dA[k] = group_sum<16>(dA[k]);
      dP[k] = group_sum<16>(dP[k]);
    }
    if (r == 0) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        s_ap[wave][4 * q + k] = dA[k];
        s_ap[wave][16 + 4 * q + k] = dP[k];
      }
    }
    lds_barrier();
    if constexpr (LW) {
#pragma unroll
      for (int e = 0; e < KPT; ++e) {
        const int k = tid + e * blockDim.x;
        if (k < KP) {
          float sum = 0.0f;
          if (k < 256) {
            for (int w = 0; w < nwaves; ++w) sum += s_dm[w][k];
          } else {
            for (int w = 0; w < nwaves; ++w) sum += s_ap[w][k - 256];
          }
          lw_acc[e] += sum;
        }
      }
    } else
    for (int k = tid; k < KP; k += blockDim.x) {
      float sum = 0.0f;
      if (k < 256) {
        for (int w = 0; w < nwaves; ++w) sum += s_dm[w][k];
        A.dM_tok[t * 256 + k] = sum;
      } else if (k < 272) {
        for (int w = 0; w < nwaves; ++w) sum += s_ap[w][k - 256];
        const int j = k - 256;
        if constexpr (RAW) {
          const float ajv = s_act[it & 1][j];
          sum *= ajv * (1.0f - ajv);
        }
        A.dpre_tok[t * 16 + j] = sum;
      } else {
        for (int w = 0; w < nwaves; ++w) sum += s_ap[w][k - 256];
        const int i = k - 272;
        if constexpr (RAW) {
          const float piv = s_act[it & 1][16 + i];
          sum *= piv * (1.0f - 0.5f * piv);
        }
        A.dpost_tok[t * 16 + i] = sum;
      }
    }
  }
  if (q == 0) {
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      *reinterpret_cast<float4*>(prow + cb[s]) = make_float4(dwv[s][0], dwv[s][1], dwv[s][2], dwv[s][3]);
      *reinterpret_cast<float4*>(prow + cb[s] + 4) = make_float4(dwv[s][4], dwv[s][5], dwv[s][6], dwv[s][7]);
    }
  }
  if constexpr (LW) {
    // [Cp | dM 256 | dA 16 | dP 16]: P = Cp + KP, no padding columns
#pragma unroll
    for (int e = 0; e < KPT; ++e) {
      const int k = tid + e * blockDim.x;
      if (k < KP) prow[A.Cp + k] = lw_acc[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Stage 2: fixed-order column sums of the G partial rows, two launches
// (per-token parameters, where only d_w is left: one, col_sum_kernel in
// mhc_reduce.hpp).
//
// reduce_rows_kernel (mhc_reduce.hpp) folds the G rows into S <= kReduceSplit
// rows (part2); param_finish_kernel adds those S rows, writes the final sums
// with the activation chain and, for layer-wide n <= SKNP, runs the Sinkhorn
// VJP dH_res = VJP(H_res, dM) on wavefront 0 of the workgroup that owns the
// parameter columns.  The kernel boundary between the two launches makes
// every XCD's rows visible without device-scope fences, and the association
// of every sum is fixed, so results are bitwise reproducible.
//
// param_finish_kernel: a workgroup owns kFinCols float4 columns and splits
// the S rows over kFinPhases row phases (rows k = phase mod kFinPhases),
// combined in phase order through LDS.  The dw columns [0, Cp) and the
// parameter columns [Cp, P) are cut into workgroups separately, so the
// n^2 + 2n parameter sums of n <= 8 sit in one workgroup.
// ---------------------------------------------------------------------------

constexpr int kFinCols = 64;
constexpr int kFinPhases = 4;
constexpr int kFinThreads = kFinCols * kFinPhases;

struct RedArgs {
  const float* part2;
  int S;
  int P;
  int Cp;
  int C;
  int n;
  int nd;  // workgroups over the dw columns
  int per_token;
  int h_mode;
  const float* hpre;
  const float* hpost;
  float* dM;
  float* dpre;
  float* dpost;
  float* dw;
  const float* hres;  // SKNP > 0: H_res logits [n, n]
  float* dhres;
  int iters;
  float eps;
};

template <int SKNP>
__global__ __launch_bounds__(kFinThreads) void param_finish_kernel(RedArgs R) {
  extern __shared__ float fin_smem[];  // SKNP > 0: dM [n*n], then the VJP state
  __shared__ float4 s_part[kFinPhases][kFinCols];
  const int tid = threadIdx.x;
  const int col4 = tid % kFinCols;
  const int phase = tid / kFinCols;
  const int wg = blockIdx.x;
  int base, end;
  if (wg < R.nd) {
    base = wg * 4 * kFinCols;
    end = min(R.Cp, base + 4 * kFinCols);
  } else {
    base = R.Cp + (wg - R.nd) * 4 * kFinCols;
    end = min(R.P, base + 4 * kFinCols);
  }
  const int c = base + 4 * col4;
  const bool act = c < end;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (act) {
    // rows phase, phase + 4, ...: S <= 64 rows are 16 loads per thread, all
    // in flight together, added as four fixed chains
    const float* src = R.part2 + c;
    float4 u[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const int k = phase + m * kFinPhases;
      // the zero is a value, not the variable v: a conditional between two
      // lvalues becomes a select of addresses, which puts v in scratch
      u[m] = k < R.S ? *reinterpret_cast<const float4*>(src + (int64_t)k * R.P) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int k = phase + 16 * kFinPhases; k < R.S; k += kFinPhases)
      u[0] = f4add(u[0], *reinterpret_cast<const float4*>(src + (int64_t)k * R.P));
#pragma unroll
    for (int m = 4; m < 16; ++m) u[m & 3] = f4add(u[m & 3], u[m]);
    v = f4add(f4add(u[0], u[1]), f4add(u[2], u[3]));
  }
  s_part[phase][col4] = v;
  __syncthreads();
  const int n = R.n, nn = n * n;
  float* s_dM = fin_smem;
  if (phase == 0 && act) {
#pragma unroll
    for (int ph = 1; ph < kFinPhases; ++ph) {
      const float4 u = s_part[ph][col4];
      v = make_float4(v.x + u.x, v.y + u.y, v.z + u.z, v.w + u.w);
    }
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int col = c + e;
      float s = vv[e];
      if (col < R.C) {
        R.dw[col] = s;
      } else if (!R.per_token && col >= R.Cp) {
        const int k = col - R.Cp;
        if (k < nn) {
          if (R.dM != nullptr) R.dM[k] = s;
          if constexpr (SKNP > 0) s_dM[k] = s;
        } else if (k < nn + n) {
          const int j = k - nn;
          if (R.h_mode == MHC_H_RAW) {
            const float a = sigmoidf_(R.hpre[j]);
            s = s * a * (1.0f - a);
          }
          R.dpre[j] = s;
        } else if (k < nn + 2 * n) {
          const int i = k - nn - n;
          if (R.h_mode == MHC_H_RAW) {
            const float sg = sigmoidf_(R.hpost[i]);
            s = s * 2.0f * sg * (1.0f - sg);
          }
          R.dpost[i] = s;
        }
      }
    }
  }
  if constexpr (SKNP > 0) {
    if (wg == R.nd) {
      __syncthreads();  // s_dM complete
      if (tid < 64) {
        if (R.iters <= kSkRegIters)
          sk_bwd_group_reg<SKNP, kSkRegIters>(R.hres, s_dM, R.dhres, tid < SkLayout<SKNP>::G, n, R.iters, R.eps,
                                              tid);
        else
          sk_bwd_group<SKNP>(R.hres, s_dM, R.dhres, tid < SkLayout<SKNP>::G, n, R.iters, R.eps,
                             fin_smem + round_up(nn, 4), tid);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

namespace {

struct BwdLayout {
  int Cp;
  int P;
  int64_t gmax;
  size_t scratch_off;  // generic path: 2*C floats per workgroup after part2
  size_t bytes;
};

// Workspace: [part: one row per workgroup][part2: kReduceSplit rows][scratch]
BwdLayout bwd_layout(int64_t T, int n, int C, int per_token) {
  BwdLayout L{};
  L.Cp = round_up(C, 4);
  L.P = per_token ? L.Cp : L.Cp + round_up(n * n + 2 * n, 4);
  L.gmax = std::max<int64_t>(1, std::min<int64_t>(T, (int64_t)device_cu_count() * 8));
  L.scratch_off = (size_t)(L.gmax + kReduceSplit) * (size_t)L.P * sizeof(float);
  L.bytes = L.scratch_off;
  if (nmax_for(n) == 0) L.bytes += (size_t)L.gmax * 2 * (size_t)C * sizeof(float);
  return L;
}

void set_rows(BwdArgs& A, const BwdLayout& L) {
  A.Cp = L.Cp;
  A.P = L.P;
}

// Layer-wide n <= 8 (fused_bwd_lw_kernel).  Returns 1 when the shape is not
// covered (C too large for one chunk per thread), so the caller falls back
// to fused_bwd_kernel.
template <int NMAX, typename XT, typename GT, bool PT>
int launch_bwd_lw(BwdArgs A, const BwdLayout& L, int64_t* num_partials, hipStream_t stream) {
  constexpr int V = lw_vec<NMAX, XT, GT>();
  A.nchunks = (int)ceil_div(A.C, V);
  const int tpb = std::max(64, round_up(A.nchunks, 64));
  if (tpb > lw_max_threads(NMAX)) return 1;
  const bool full = A.n == NMAX && A.vec && A.C % V == 0 && A.nchunks == tpb;
  // Partial tiles (n below NMAX, a partial last chunk or workgroup) run here only at n <= 4 with
  // vector-aligned rows, on at most 512 threads (the variant's 256-VGPR bound); the others take the
  // tile kernel, whose narrower chunks need less alignment.
  if (!full && (NMAX > 4 || !A.vec || tpb > 512)) return 1;
  // Grid: the workspace's full row budget (8 workgroups per CU) streams
  // faster than one resident wave of workgroups (562 vs 576 us at config 2);
  // MHC_BWD_GRID overrides the count.
  // The pipelined variant (n == 4 full tiles up to 512 threads, MHC_BWD_PIPE
  // != 0) holds one workgroup per CU; two per CU keep the CUs busy while
  // one drains (config 2: 0.929 ms step at 512 workgroups vs 0.955 at the
  // non-pipelined default).
  const bool pipe = NMAX == 4 && !PT && full && tpb <= 512 && knob(kKnobBwdPipe, 1) != 0;
  int64_t blocks = pipe ? std::min<int64_t>(L.gmax, (int64_t)device_cu_count() * 2) : L.gmax;
  const int grid_pref = knob(kKnobBwdGrid, 0);
  if (grid_pref > 0) blocks = std::min<int64_t>(L.gmax, grid_pref);
  blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, A.T));
  set_rows(A, L);
  const dim3 g((unsigned)blocks), b(tpb);
  if constexpr (NMAX == 4 && !PT) {
    if (pipe) {
      hipLaunchKernelGGL((fused_bwd_lw_kernel<NMAX, XT, GT, 1, true, false, true>), g, b, 0, stream, A);
      MHC_CHECK_LAUNCH("fused_bwd_lw_kernel");
      *num_partials = blocks;
      return MHC_OK;
    }
  }
  if (full) {
    hipLaunchKernelGGL((fused_bwd_lw_kernel<NMAX, XT, GT, 1, true, PT>), g, b, 0, stream, A);
  } else if constexpr (NMAX <= 4) {
    hipLaunchKernelGGL((fused_bwd_lw_kernel<NMAX, XT, GT, 1, false, PT>), g, b, 0, stream, A);
  }
  MHC_CHECK_LAUNCH("fused_bwd_lw_kernel");
  *num_partials = blocks;
  return MHC_OK;
}

// n == 16 on MFMA (fused_bwd_mfma16_kernel), per-token or (LW) layer-wide
// parameters: 16-bit x == dout, C a multiple of 128 up to 1024, or up to
// 2048 with two slabs per wave (two 128-channel slabs per wave when C / 128
// is even, else one), 16-byte aligned operands.  Returns 1 when the shape is
// not covered.
template <typename XT, int SPW, bool LW, bool WIDE, bool PIPE>
int launch_mf16_variant(BwdArgs A, const BwdLayout& L, int waves, int64_t* num_partials, hipStream_t stream) {
  const size_t smem = (size_t)waves * SPW * 2 * 16 * kMf16Row * sizeof(uint16_t);
  const bool raw = A.h_mode == MHC_H_RAW;
  const void* kfn = raw ? (const void*)fused_bwd_mfma16_kernel<XT, SPW, true, LW, WIDE, PIPE>
                        : (const void*)fused_bwd_mfma16_kernel<XT, SPW, false, LW, WIDE, PIPE>;
  const int occ = occupancy_blocks(kfn, waves * 64, smem);
  if (occ <= 0) return 1;
  int64_t blocks = std::min<int64_t>(L.gmax, (int64_t)device_cu_count() * occ);
  const int grid_pref = knob(kKnobBwdGrid, 0);
  if (grid_pref > 0) blocks = std::min<int64_t>(L.gmax, grid_pref);
  blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, A.T));
  set_rows(A, L);
  const dim3 g((unsigned)blocks), b(waves * 64);
  if (raw) hipLaunchKernelGGL((fused_bwd_mfma16_kernel<XT, SPW, true, LW, WIDE, PIPE>), g, b, smem, stream, A);
  else hipLaunchKernelGGL((fused_bwd_mfma16_kernel<XT, SPW, false, LW, WIDE, PIPE>), g, b, smem, stream, A);
  MHC_CHECK_LAUNCH("fused_bwd_mfma16_kernel");
  *num_partials = blocks;
  return MHC_OK;
}

// Pipelined loads (MHC_BWD_PIPE, default on) hold the next token's x and g
// (32 VGPRs per slab) through the dx pass; with two slabs per wave and the
// layer-wide sums in registers that would spill, so that variant keeps its
// loads at the top of the token.
template <typename XT, int SPW, bool LW, bool WIDE>
int launch_mf16_pick(BwdArgs A, const BwdLayout& L, int waves, int64_t* num_partials, hipStream_t stream) {
  if constexpr (!(LW && SPW == 2)) {
    if (knob(kKnobBwdPipe, 1) != 0)
      return launch_mf16_variant<XT, SPW, LW, WIDE, true>(A, L, waves, num_partials, stream);
  }
  return launch_mf16_variant<XT, SPW, LW, WIDE, false>(A, L, waves, num_partials, stream);
}

template <typename XT, bool LW>
int launch_bwd_mfma16(BwdArgs A, const BwdLayout& L, int64_t* num_partials, hipStream_t stream) {
  if (A.n != 16 || A.C % 128 != 0 || A.C > 2048) return 1;
  if (LW && L.P != L.Cp + 256 + 32) return 1;
  if (!aligned(A.x, 16) || !aligned(A.g, 16) || !aligned(A.dx, 16) || !aligned(A.M, 16) ||
      !aligned(A.hpre, 16) || !aligned(A.hpost, 16) || !aligned(A.w, 16) || !aligned(A.part, 16))
    return 1;
  if (knob(kKnobBwdMfma, 1) == 0) return 1;
  const int S = A.C / 128;
  int spw = knob(kKnobBwdSpw, S % 2 == 0 ? 2 : 1);
  if (spw != 1 && spw != 2) spw = 1;
  if (S % spw != 0) spw = 1;
  const int waves = S / spw;
  if (spw == 1) {
    if (waves > kMf16MaxWaves) return 1;
    return launch_mf16_pick<XT, 1, LW, false>(A, L, waves, num_partials, stream);
  }
  if (waves <= 4) return launch_mf16_pick<XT, 2, LW, false>(A, L, waves, num_partials, stream);
  if (waves > kMf16MaxWaves) return 1;
  return launch_mf16_pick<XT, 2, LW, true>(A, L, waves, num_partials, stream);
}

// Per-token n == 16 with 16-bit x == dout and C a multiple of 256 up to 1024
// (fused_bwd_pt16_kernel).  Returns 1 when the shape is not covered.

template <typename XT>
int launch_bwd_pt16(BwdArgs A, const BwdLayout& L, int64_t* num_partials, hipStream_t stream) {
  if (A.n != 16 || A.C % 256 != 0 || A.C > 1024) return 1;
  if (!aligned(A.x, 8) || !aligned(A.g, 8) || !aligned(A.dx, 8)) return 1;
  const int tpb = A.C / 4;
  const void* kfn = (const void*)fused_bwd_pt16_kernel<XT>;
  const int occ = occupancy_blocks(kfn, tpb, 0);
  if (occ <= 0) return 1;
  int64_t blocks = std::min<int64_t>(L.gmax, (int64_t)device_cu_count() * occ);
  blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, A.T));
  set_rows(A, L);
  hipLaunchKernelGGL((fused_bwd_pt16_kernel<XT>), dim3((unsigned)blocks), dim3(tpb), 0, stream, A);
  MHC_CHECK_LAUNCH("fused_bwd_pt16_kernel");
  *num_partials = blocks;
  return MHC_OK;
}

// Tile backward (bwd_tile_kernel): every shape the kernels above do not take.
template <int NMAX, typename XT, typename GT, bool PT>
int launch_bwd_tile(BwdArgs A, const BwdLayout& L, int64_t* num_partials, hipStream_t stream) {
  constexpr int V = TileCfg<NMAX>::V;
  A.nchunks = (int)ceil_div(A.C, V);
  const int ax = std::min(16, V * ElemTraits<XT>::kBytes), ag = std::min(16, V * ElemTraits<GT>::kBytes);
  A.vec = A.C % V == 0 && aligned(A.x, ax) && aligned(A.dx, ax) && aligned(A.g, ag) ? 1 : 0;
  const void* kfn = (const void*)bwd_tile_kernel<NMAX, XT, GT, PT>;
  const int occ = occupancy_blocks(kfn, kTileThreads, 0);
  if (occ <= 0)
    return set_error(MHC_ERR_INVALID_ARG, "fused_bwd: no occupancy for the tile kernel (n=%d C=%d)", A.n, A.C);
  int64_t blocks = std::min<int64_t>(L.gmax, (int64_t)device_cu_count() * occ);
  const int grid_pref = knob(kKnobBwdGrid, 0);
  if (grid_pref > 0) blocks = std::min<int64_t>(L.gmax, grid_pref);
  blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, A.T));
  set_rows(A, L);
  hipLaunchKernelGGL((bwd_tile_kernel<NMAX, XT, GT, PT>), dim3((unsigned)blocks), dim3(kTileThreads), 0, stream, A);
  MHC_CHECK_LAUNCH("bwd_tile_kernel");
  *num_partials = blocks;
  return MHC_OK;
}

template <int NMAX, typename XT, typename GT, bool PT>
int launch_bwd(BwdArgs A, const BwdLayout& L, int64_t* num_partials, hipStream_t stream) {
  if constexpr (!PT && NMAX == 16 && std::is_same<XT, GT>::value && ElemTraits<XT>::kBytes == 2) {
    const int rc = launch_bwd_mfma16<XT, true>(A, L, num_partials, stream);
    if (rc != 1) return rc;
  }
  if constexpr (PT && NMAX == 16 && std::is_same<XT, GT>::value && ElemTraits<XT>::kBytes == 2) {
    int rc = launch_bwd_mfma16<XT, false>(A, L, num_partials, stream);
    if (rc != 1) return rc;
    rc = launch_bwd_pt16<XT>(A, L, num_partials, stream);
    if (rc != 1) return rc;
  }
  if constexpr (NMAX <= 8) {
    const int legacy = knob(kKnobBwdLegacy, 0);
    if (!legacy) {
      const int rc = launch_bwd_lw<NMAX, XT, GT, PT>(A, L, num_partials, stream);
      if (rc != 1) return rc;
    }
  }
  return launch_bwd_tile<NMAX, XT, GT, PT>(A, L, num_partials, stream);
}

template <typename XT, typename GT, bool PT>
int bwd_dispatch_n(const BwdArgs& A, const BwdLayout& L, int64_t* np, hipStream_t s) {
  switch (nmax_for(A.n)) {
    case 4: return launch_bwd<4, XT, GT, PT>(A, L, np, s);
    case 8: return launch_bwd<8, XT, GT, PT>(A, L, np, s);
    default: return launch_bwd<16, XT, GT, PT>(A, L, np, s);
  }
}

template <bool PT>
int bwd_dispatch_types(const BwdArgs& A, const BwdLayout& L, int xd, int gd, int64_t* np,
                       hipStream_t s) {
  if (xd == MHC_DTYPE_F32 && gd == MHC_DTYPE_F32) return bwd_dispatch_n<float, float, PT>(A, L, np, s);
  if (xd == MHC_DTYPE_BF16 && gd == MHC_DTYPE_BF16) return bwd_dispatch_n<__bf16, __bf16, PT>(A, L, np, s);
  if (xd == MHC_DTYPE_BF16 && gd == MHC_DTYPE_F32) return bwd_dispatch_n<__bf16, float, PT>(A, L, np, s);
  if (xd == MHC_DTYPE_F16 && gd == MHC_DTYPE_F16) return bwd_dispatch_n<_Float16, _Float16, PT>(A, L, np, s);
  if (xd == MHC_DTYPE_F16 && gd == MHC_DTYPE_F32) return bwd_dispatch_n<_Float16, float, PT>(A, L, np, s);
  return set_error(MHC_ERR_INVALID_ARG,
                   "fused_bwd: unsupported (x_dtype=%d, dout_dtype=%d); dout must be fp32 or x's dtype",
                   xd, gd);
}

}  // namespace
}  // namespace mhc

using namespace mhc;

extern "C" size_t mhc_fused_bwd_workspace_bytes(int64_t T, int n, int C, int per_token) {
  if (T <= 0 || n < 1 || n > MHC_MAX_N || C < 1) return 0;
  return bwd_layout(T, n, C, per_token).bytes;
}

extern "C" int mhc_fused_bwd_partials(const void* x, int x_dtype, const void* dout, int dout_dtype,
                                      const float* M, int64_t M_token_stride, const float* h_pre,
                                      const float* h_post, int64_t h_token_stride, int h_mode,
                                      const float* rms_weight, void* dx, int dx_dtype,
                                      float* dM_tok, float* dh_pre_tok, float* dh_post_tok,
                                      void* workspace, size_t workspace_bytes, int64_t T, int n,
                                      int C, float eps, int64_t* num_partials, void* stream) {
  clear_error();
  MHC_CHECK_ARG(num_partials != nullptr, "num_partials must not be NULL");
  *num_partials = 0;
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1, "C=%d must be positive", C);
  MHC_CHECK_ARG(T >= 0, "T=%lld must be >= 0", (long long)T);
  MHC_CHECK_ARG(h_mode == MHC_H_ACTIVATED || h_mode == MHC_H_RAW, "h_mode=%d must be ACTIVATED or RAW",
                h_mode);
  MHC_CHECK_ARG(M_token_stride == 0 || M_token_stride == (int64_t)n * n,
                "M_token_stride must be 0 or n*n");
  MHC_CHECK_ARG(h_token_stride == 0 || h_token_stride == n, "h_token_stride must be 0 or n");
  MHC_CHECK_ARG((M_token_stride == 0) == (h_token_stride == 0),
                "M and h must both be per-token or both layer-wide");
  MHC_CHECK_ARG(dx_dtype == x_dtype, "dx_dtype (%d) must equal x_dtype (%d)", dx_dtype, x_dtype);
  if (T == 0) return MHC_OK;
  const int per_token = M_token_stride != 0;
  MHC_CHECK_ARG(x && dout && M && h_pre && h_post && rms_weight && dx, "null pointer argument");
  MHC_CHECK_ARG(!per_token || (dM_tok && dh_pre_tok && dh_post_tok),
                "per-token mode needs dM_tok, dh_pre_tok and dh_post_tok");
  const BwdLayout L = bwd_layout(T, n, C, per_token);
  MHC_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.bytes,
                "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes,
                L.bytes);
  MHC_CHECK_ARG(aligned(workspace, 16), "workspace must be 16-byte aligned");
  const int xb = dtype_bytes(x_dtype), gb = dtype_bytes(dout_dtype);
  MHC_CHECK_ARG(xb > 0 && gb > 0, "unknown dtype code");
  BwdArgs A{};
  A.x = x; A.g = dout; A.dx = dx; A.M = M; A.hpre = h_pre; A.hpost = h_post; A.w = rms_weight;
  A.part = (float*)workspace; A.dM_tok = dM_tok; A.dpre_tok = dh_pre_tok; A.dpost_tok = dh_post_tok;
  A.T = T; A.M_ts = M_token_stride; A.h_ts = h_token_stride; A.n = n; A.C = C; A.h_mode = h_mode;
  A.eps = eps;
  MHC_CHECK_ARG(dout_dtype == MHC_DTYPE_F32 || dout_dtype == x_dtype,
                "dout_dtype (%d) must be fp32 or x_dtype (%d)", dout_dtype, x_dtype);
  if (nmax_for(n) == 0) {
    Mf32Args F{};
    F.x = x; F.g = dout; F.out = dx; F.M = M; F.hpre = h_pre; F.hpost = h_post; F.w = rms_weight;
    F.part = (float*)workspace; F.T = T; F.M_ts = M_token_stride; F.h_ts = h_token_stride; F.n = n; F.C = C;
    F.Cp = L.Cp; F.P = L.P; F.h_mode = h_mode; F.eps = eps;
    F.dM_tok = dM_tok; F.dpre_tok = dh_pre_tok; F.dpost_tok = dh_post_tok;
    const int rc = mf32_fused_bwd(F, x_dtype, dout_dtype, L.gmax, (hipStream_t)stream, num_partials);
    if (rc != 1) return rc;
    GenArgs G{};
    G.x = x; G.g = dout; G.out = dx; G.M = M; G.hpre = h_pre; G.hpost = h_post; G.w = rms_weight;
    G.part = (float*)workspace;
    G.scratch = (float*)((char*)workspace + L.scratch_off);
    G.dM_tok = dM_tok; G.dpre_tok = dh_pre_tok; G.dpost_tok = dh_post_tok;
    G.T = T; G.M_ts = M_token_stride; G.h_ts = h_token_stride; G.n = n; G.C = C; G.Cp = L.Cp;
    G.P = L.P; G.h_mode = h_mode; G.eps = eps;
    return gen_fused_bwd(G, x_dtype, dout_dtype, (hipStream_t)stream, num_partials);
  }
  const int V = bwd_vec_width(nmax_for(n));
  const int ax = std::min(16, V * xb), ag = std::min(16, V * gb);
  A.vec = (C % V == 0) && aligned(x, ax) && aligned(dx, ax) && aligned(dout, ag) &&
          ((int64_t)C * xb) % ax == 0 && ((int64_t)C * gb) % ag == 0 ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  return per_token ? bwd_dispatch_types<true>(A, L, x_dtype, dout_dtype, num_partials, s)
                   : bwd_dispatch_types<false>(A, L, x_dtype, dout_dtype, num_partials, s);
}

namespace mhc {
namespace {

// Reduce `G` partial rows: per-token parameters (d_w only) in one col_sum_kernel
// launch; otherwise reduce_rows_kernel (when G > kReduceSplit) then
// param_finish_kernel.
// With hres != NULL the Sinkhorn VJP of the reduced dM runs in the second
// launch; returns 1 when that fusion is not possible (per-token parameters,
// n > 8, or VJP state beyond the LDS budget).
int launch_param_reduce(const void* workspace, size_t workspace_bytes, int64_t G, int n, int C, int per_token,
                        const float* h_pre, const float* h_post, int h_mode, float* dM, float* dh_pre,
                        float* dh_post, float* dw, const float* hres, float* dhres, int iters, float eps,
                        hipStream_t s) {
  RedArgs R{};
  R.Cp = round_up(C, 4);
  R.P = per_token ? R.Cp : R.Cp + round_up(n * n + 2 * n, 4);
  R.nd = (int)ceil_div(R.Cp, 4 * kFinCols);
  const int nwg = R.nd + (int)ceil_div(R.P - R.Cp, 4 * kFinCols);
  int sknp = 0;
  size_t smem = 0;
  if (hres != nullptr) {
    if (per_token || n > 8) return 1;
    sknp = next_pow2(n);
    smem = ((size_t)round_up(n * n, 4) + (size_t)sk_state_floats(sknp, iters)) * sizeof(float);
    if (smem > 48 * 1024) return 1;
  }
  if (G > 0) {
    const size_t need = (size_t)(G + kReduceSplit) * (size_t)R.P * sizeof(float);
    MHC_CHECK_ARG(workspace != nullptr && workspace_bytes >= need,
                  "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, need);
    MHC_CHECK_ARG(aligned(workspace, 16), "workspace must be 16-byte aligned");
    if (per_token) {
      // only d_w is left to sum (the token's parameter gradients are written by the partials pass): one
      // launch, which takes the place of the two below
      hipLaunchKernelGGL(col_sum_kernel, dim3((unsigned)ceil_div(R.Cp, 4 * kColSumCols)),
                         dim3(kColSumCols * kColSumPhases), 0, s, (const float*)workspace, G, R.P, C, dw);
      MHC_CHECK_LAUNCH("col_sum_kernel");
      return MHC_OK;
    }
    if (G <= kReduceSplit) {
      // at most kReduceSplit rows: reduce_rows_kernel would copy them unchanged (one row per output
      // row), so param_finish_kernel reads them where they lie; one launch fewer at small batch
      R.S = (int)G;
      R.part2 = (const float*)workspace;
    } else {
      const int rows = (int)ceil_div(G, (int64_t)kReduceSplit);
      R.S = (int)ceil_div(G, rows);
      float* part2 = (float*)workspace + G * (int64_t)R.P;
      hipLaunchKernelGGL(reduce_rows_kernel, dim3((unsigned)ceil_div(R.P / 4, 256), (unsigned)R.S), dim3(256), 0,
                         s, (const float*)workspace, part2, G, R.P, rows);
      MHC_CHECK_LAUNCH("reduce_rows_kernel");
      R.part2 = part2;
    }
  } else {
    R.S = 0;  // no rows: every sum is zero
    R.part2 = nullptr;
  }
  R.C = C; R.n = n; R.per_token = per_token; R.h_mode = h_mode;
  R.hpre = h_pre; R.hpost = h_post; R.dM = dM; R.dpre = dh_pre; R.dpost = dh_post; R.dw = dw;
  R.hres = hres; R.dhres = dhres; R.iters = iters; R.eps = eps;
  const dim3 grid((unsigned)nwg);
  switch (sknp) {
    case 0: hipLaunchKernelGGL((param_finish_kernel<0>), grid, dim3(kFinThreads), 0, s, R); break;
    case 1: hipLaunchKernelGGL((param_finish_kernel<1>), grid, dim3(kFinThreads), smem, s, R); break;
    case 2: hipLaunchKernelGGL((param_finish_kernel<2>), grid, dim3(kFinThreads), smem, s, R); break;
    case 4: hipLaunchKernelGGL((param_finish_kernel<4>), grid, dim3(kFinThreads), smem, s, R); break;
    default: hipLaunchKernelGGL((param_finish_kernel<8>), grid, dim3(kFinThreads), smem, s, R); break;
  }
  MHC_CHECK_LAUNCH("param_finish_kernel");
  return MHC_OK;
}

}  // namespace
}  // namespace mhc

extern "C" int mhc_reduce_param_grads(const void* workspace, size_t workspace_bytes,
                                      int64_t num_partials, int n, int C, int per_token,
                                      const float* h_pre, const float* h_post, int h_mode,
                                      float* dM, float* dh_pre, float* dh_post,
                                      float* d_rms_weight, void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1, "C=%d must be positive", C);
  MHC_CHECK_ARG(d_rms_weight != nullptr, "d_rms_weight must not be NULL");
  MHC_CHECK_ARG(per_token || (dM && dh_pre && dh_post), "dM, dh_pre and dh_post must not be NULL");
  MHC_CHECK_ARG(per_token || h_mode != MHC_H_RAW || (h_pre && h_post),
                "raw-logit mode needs h_pre and h_post");
  MHC_CHECK_ARG(num_partials >= 0, "num_partials must be >= 0");
  return launch_param_reduce(workspace, workspace_bytes, num_partials, n, C, per_token, h_pre, h_post, h_mode,
                             dM, dh_pre, dh_post, d_rms_weight, nullptr, nullptr, 0, 0.0f,
                             (hipStream_t)stream);
}

extern "C" int mhc_fused_bwd(const void* x, int x_dtype, const void* dout, int dout_dtype,
                             const float* M, int64_t M_token_stride, const float* h_pre,
                             const float* h_post, int64_t h_token_stride, int h_mode,
                             const float* rms_weight, void* dx, int dx_dtype, float* dM,
                             float* dh_pre, float* dh_post, float* d_rms_weight, void* workspace,
                             size_t workspace_bytes, int64_t T, int n, int C, float eps,
                             void* stream) {
  const int per_token = M_token_stride != 0;
  int64_t np = 0;
  int rc = mhc_fused_bwd_partials(x, x_dtype, dout, dout_dtype, M, M_token_stride, h_pre, h_post,
                                  h_token_stride, h_mode, rms_weight, dx, dx_dtype,
                                  per_token ? dM : nullptr, per_token ? dh_pre : nullptr,
                                  per_token ? dh_post : nullptr, workspace, workspace_bytes, T, n,
                                  C, eps, &np, stream);
  if (rc != MHC_OK) return rc;
  return mhc_reduce_param_grads(workspace, workspace_bytes, np, n, C, per_token, h_pre, h_post,
                                h_mode, per_token ? nullptr : dM, per_token ? nullptr : dh_pre,
                                per_token ? nullptr : dh_post, d_rms_weight, stream);
}

// ---------------------------------------------------------------------------
// Layer-level backward (raw parameters in, raw-parameter gradients out)
// ---------------------------------------------------------------------------

namespace mhc {
namespace {

struct LayerBwdLayout {
  size_t bwd_bytes;  // mhc_fused_bwd_workspace_bytes
  size_t dM_off;     // layer-wide: reduced dM [n, n]
  size_t sk_off;     // Sinkhorn VJP workspace
  size_t bytes;
};

LayerBwdLayout layer_bwd_layout(int64_t T, int n, int C, int per_token, int iters) {
  LayerBwdLayout L{};
  L.bwd_bytes = bwd_layout(T, n, C, per_token).bytes;
  L.dM_off = (L.bwd_bytes + 255) / 256 * 256;
  L.sk_off = L.dM_off + (size_t)round_up(n * n, 64) * sizeof(float);
  L.bytes = L.sk_off + mhc_sinkhorn_bwd_workspace_bytes(per_token ? T : 1, n, iters);
  return L;
}

}  // namespace
}  // namespace mhc

extern "C" size_t mhc_layer_bwd_workspace_bytes(int64_t T, int n, int C, int per_token, int iters) {
  if (T <= 0 || n < 1 || n > MHC_MAX_N || C < 1 || iters < 0) return 0;
  return layer_bwd_layout(T, n, C, per_token, iters).bytes;
}

extern "C" int mhc_layer_bwd_reduce(void* workspace, size_t workspace_bytes, int64_t num_partials,
                                    const float* h_pre_raw, const float* h_post_raw, const float* h_res_raw,
                                    float* d_h_pre_raw, float* d_h_post_raw, float* d_h_res_raw,
                                    float* d_rms_weight, int64_t T, int n, int C, int per_token, int iters,
                                    float eps, void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1, "C=%d must be positive", C);
  MHC_CHECK_ARG(T >= 0 && num_partials >= 0, "T and num_partials must be >= 0");
  MHC_CHECK_ARG(iters >= 0, "iters=%d must be >= 0", iters);
  MHC_CHECK_ARG(h_pre_raw && h_post_raw && h_res_raw, "null parameter pointer");
  MHC_CHECK_ARG(d_h_pre_raw && d_h_post_raw && d_h_res_raw && d_rms_weight, "null gradient pointer");
  MHC_CHECK_ARG(num_partials == 0 || T > 0, "num_partials must be 0 when T == 0");
  hipStream_t s = (hipStream_t)stream;
  if (per_token && T == 0) return MHC_OK;
  const LayerBwdLayout L = layer_bwd_layout(std::max<int64_t>(T, 1), n, C, per_token, iters);
  MHC_CHECK_ARG(T == 0 || (workspace != nullptr && workspace_bytes >= L.bytes),
                "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, L.bytes);
  char* ws = (char*)workspace;
  int rc;
  if (per_token) {
    // d_h_res_raw holds dM per token (written by the partials pass); the
    // Sinkhorn VJP runs in place.
    rc = launch_param_reduce(ws, L.bwd_bytes, num_partials, n, C, 1, nullptr, nullptr, MHC_H_RAW, nullptr,
                             nullptr, nullptr, d_rms_weight, nullptr, nullptr, 0, 0.0f, s);
    if (rc != MHC_OK) return rc;
    const size_t skb = mhc_sinkhorn_bwd_workspace_bytes(T, n, iters);
    return mhc_sinkhorn_bwd(h_res_raw, d_h_res_raw, d_h_res_raw, T, n, iters, eps, skb ? ws + L.sk_off : nullptr,
                            skb, stream);
  }
  float* dM = T > 0 ? reinterpret_cast<float*>(ws + L.dM_off) : nullptr;
  rc = launch_param_reduce(ws, L.bwd_bytes, num_partials, n, C, 0, h_pre_raw, h_post_raw, MHC_H_RAW, dM,
                           d_h_pre_raw, d_h_post_raw, d_rms_weight, h_res_raw, d_h_res_raw, iters, eps, s);
  if (rc != 1) return rc;
  // VJP state too large for one workgroup's LDS (or n > 16): separate launch
  MHC_CHECK_ARG(T > 0, "T=0 with n=%d needs a workspace for the Sinkhorn VJP", n);
  rc = launch_param_reduce(ws, L.bwd_bytes, num_partials, n, C, 0, h_pre_raw, h_post_raw, MHC_H_RAW, dM,
                           d_h_pre_raw, d_h_post_raw, d_rms_weight, nullptr, nullptr, 0, 0.0f, s);
  if (rc != MHC_OK) return rc;
  const size_t skb = mhc_sinkhorn_bwd_workspace_bytes(1, n, iters);
  return mhc_sinkhorn_bwd(h_res_raw, dM, d_h_res_raw, 1, n, iters, eps, skb ? ws + L.sk_off : nullptr, skb,
                          stream);
}

extern "C" int mhc_layer_bwd(const void* x, int x_dtype, const void* dout, int dout_dtype,
                             const float* h_pre_raw, const float* h_post_raw, const float* h_res_raw,
                             const float* M, const float* rms_weight, void* dx, float* d_h_pre_raw,
                             float* d_h_post_raw, float* d_h_res_raw, float* d_rms_weight, void* workspace,
                             size_t workspace_bytes, int64_t T, int n, int C, int per_token, int iters,
                             float eps, void* stream) {
  clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1, "C=%d must be positive", C);
  MHC_CHECK_ARG(T >= 0, "T=%lld must be >= 0", (long long)T);
  MHC_CHECK_ARG(iters >= 0, "iters=%d must be >= 0", iters);
  MHC_CHECK_ARG(M != nullptr && rms_weight != nullptr, "null parameter pointer");
  MHC_CHECK_ARG(h_pre_raw && h_post_raw && h_res_raw, "null parameter pointer");
  MHC_CHECK_ARG(d_h_pre_raw && d_h_post_raw && d_h_res_raw && d_rms_weight, "null gradient pointer");
  int64_t np = 0;
  if (T > 0) {
    const LayerBwdLayout L = layer_bwd_layout(T, n, C, per_token, iters);
    MHC_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.bytes,
                  "workspace of %zu bytes is smaller than the %zu bytes required", workspace_bytes, L.bytes);
    const int rc = mhc_fused_bwd_partials(
        x, x_dtype, dout, dout_dtype, M, per_token ? (int64_t)n * n : 0, h_pre_raw, h_post_raw,
        per_token ? n : 0, MHC_H_RAW, rms_weight, dx, x_dtype, per_token ? d_h_res_raw : nullptr,
        per_token ? d_h_pre_raw : nullptr, per_token ? d_h_post_raw : nullptr, workspace, L.bwd_bytes, T, n, C,
        eps, &np, stream);
    if (rc != MHC_OK) return rc;
  }
  return mhc_layer_bwd_reduce(workspace, workspace_bytes, np, h_pre_raw, h_post_raw, h_res_raw, d_h_pre_raw,
                              d_h_post_raw, d_h_res_raw, d_rms_weight, T, n, C, per_token, iters, eps, stream);
}
