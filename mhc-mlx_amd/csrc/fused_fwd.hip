// Fused mHC forward: stream aggregate + RMSNorm + n x n stream mix + H_post
// residual add in one pass over x (mhc_mlx/reference.py:148-184).
//
// One workgroup processes one token at a time (persistent grid, grid-stride
// over tokens).  The token's n x C tile is split into channel chunks of V
// consecutive channels; thread `tid` owns chunks tid, tid + TPB, ... and
// keeps every stream of its chunks in registers (packed 16-bit when x is
// bf16/fp16) from the load until the store, so x is read from HBM exactly
// once.  Per token:
//   phase A  load chunk, y = sum_i a_i x_i, accumulate y^2
//   reduce   wave butterfly + one LDS slot per wave + one barrier
//   phase B  out_i = sum_j M_ij x_j + p_i * (y * inv) * w, store
// When the tile does not fit in registers (very large n*C) the kernel runs a
// second pass over x instead ("reload").
#include <type_traits>

#include "mhc_device.hpp"
#include "mhc_generic.hpp"
#include "mhc_mfma32.hpp"
#include "mhc_host.hpp"
#include "mhc_plan.hpp"
#include "mhc_sinkhorn.hpp"

namespace mhc {

// Kernel arguments, at most 112 bytes: the HIP runtime's launch costs ~0.65 us
// more on this part for larger argument blocks (2.85 against 3.5 us per launch,
// measured), which is a fifth of a single-launch forward's host time.
struct FwdArgs {
  const void* x;
  void* out;
  float* inv_rms;
  const float* M;
  const float* hpre;
  const float* hpost;
  const float* w;
  int64_t T;
  int M_ts;  // per-token strides (n * n and n; 0 for layer-wide parameters)
  int h_ts;
  int n;
  int C;
  int nchunks;
  uint8_t ch;
  uint8_t h_mode;
  uint8_t vec;
  uint8_t reload;
  float eps;
  // in-kernel Sinkhorn (layer-wide n <= 8, latency regime): iterations, logits, M written by block 0
  int iters;
  const float* hres;
  float* M_out;
};
static_assert(sizeof(FwdArgs) <= 112, "FwdArgs beyond the runtime's fast kernel-argument size");

// Stage (M padded to NMAX x NMAX, a, p) for token t into `buf`.
template <int NMAX>
MHC_DEV void fwd_stage_params(float* buf, const FwdArgs& A, int64_t t) {
  constexpr int NPAR = NMAX * NMAX + 2 * NMAX;
  const int n = A.n;
  const float* M = A.M + t * A.M_ts;
  const float* hp = A.hpre + t * A.h_ts;
  const float* hq = A.hpost + t * A.h_ts;
  for (int idx = threadIdx.x; idx < NPAR; idx += blockDim.x) {
    float v = 0.0f;
    if (idx < NMAX * NMAX) {
      const int i = idx / NMAX, j = idx % NMAX;
      if (i < n && j < n) v = M[i * n + j];
    } else if (idx < NMAX * NMAX + NMAX) {
      const int i = idx - NMAX * NMAX;
      if (i < n) v = A.h_mode == MHC_H_RAW ? sigmoidf_(hp[i]) : hp[i];
    } else {
      const int i = idx - NMAX * NMAX - NMAX;
      if (i < n) v = A.h_mode == MHC_H_RAW ? 2.0f * sigmoidf_(hq[i]) : hq[i];
    }
    buf[idx] = v;
  }
}

template <int NMAX, typename XT, typename OT, bool PT>
__global__ __launch_bounds__(1024) void fused_fwd_kernel(FwdArgs A) {
  constexpr int V = FwdCfg<NMAX>::V;
  constexpr int CH = FwdCfg<NMAX>::CH;
  constexpr int NPAR = NMAX * NMAX + 2 * NMAX;
  // Parameters live in registers (uniform) for small static n, else in LDS.
  constexpr bool PAR_LDS = PT || NMAX > 8;
  extern __shared__ float fwd_smem[];
  __shared__ float s_red[2][16];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int n = A.n;
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  const XT* __restrict__ X = (const XT*)A.x;
  OT* __restrict__ O = (OT*)A.out;
  const float* __restrict__ Wt = A.w;

  // static parameters in uniform registers
  float Ms[PAR_LDS ? 1 : NMAX * NMAX], as[PAR_LDS ? 1 : NMAX], ps[PAR_LDS ? 1 : NMAX];
  if constexpr (!PAR_LDS) {
#pragma unroll
    for (int i = 0; i < NMAX; ++i) {
      float av = 0.0f, pv = 0.0f;
      if (i < n) {
        av = A.hpre[i];
        pv = A.hpost[i];
        if (A.h_mode == MHC_H_RAW) {
          av = sigmoidf_(av);
          pv = 2.0f * sigmoidf_(pv);
        }
      }
      as[i] = uniform_f(av);
      ps[i] = uniform_f(pv);
#pragma unroll
      for (int j = 0; j < NMAX; ++j) Ms[i * NMAX + j] = (i < n && j < n) ? A.M[i * n + j] : 0.0f;
    }
  } else {
    if (PT) {
      if ((int64_t)blockIdx.x < A.T) fwd_stage_params<NMAX>(fwd_smem, A, blockIdx.x);
    } else {
      fwd_stage_params<NMAX>(fwd_smem, A, 0);
    }
    __syncthreads();
  }

  // rms weight of the owned chunks (register-resident path), in this thread's LDS slots
  // (s_w[(j * V + v) * blockDim.x + tid]): held in registers across the token loop they were what
  // the loop spilled, and the scratch reloads waited for every load in flight
  float* s_w = fwd_smem + (PAR_LDS ? (PT ? 3 : 1) * NPAR : 0);
  if (!A.reload) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      const int q = tid + j * blockDim.x;
      const int c0 = q * V;
      const bool act = (j < A.ch) && (q < A.nchunks);
#pragma unroll
      for (int v = 0; v < V; ++v)
        s_w[(j * V + v) * blockDim.x + tid] = (act && c0 + v < C) ? Wt[c0 + v] : 0.0f;
    }
  }

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const float* par = fwd_smem + (PT ? (it % 3) * NPAR : 0);
    if constexpr (PT) {
      const int64_t tn = t + gridDim.x;
      if (tn < A.T) fwd_stage_params<NMAX>(fwd_smem + ((it + 1) % 3) * NPAR, A, tn);
    }
    auto a_at = [&](int i) -> float {
      if constexpr (PAR_LDS) return par[NMAX * NMAX + i]; else return as[i];
    };
    auto p_at = [&](int i) -> float {
      if constexpr (PAR_LDS) return par[NMAX * NMAX + NMAX + i]; else return ps[i];
    };
    auto m_at = [&](int i, int j) -> float {
      if constexpr (PAR_LDS) return par[i * NMAX + j]; else return Ms[i * NMAX + j];
    };
    const XT* xt = X + t * nC;
    OT* ot = O + t * nC;

    if (!A.reload) {
      Vec<XT, V> xr[CH][NMAX];
      float y[CH][V];
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int q = tid + j * blockDim.x;
        const bool act = (j < A.ch) && (q < A.nchunks);
        const int c0 = q * V;
        const int valid = act ? min(V, C - c0) : 0;
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          if (act && i < n) {
            if (A.vec && valid == V) xr[j][i].load(xt + (int64_t)i * C + c0);
            else xr[j][i].load_partial(xt + (int64_t)i * C + c0, valid);
          } else {
            xr[j][i].zero();
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) {
          float acc = 0.0f;
#pragma unroll
          for (int i = 0; i < NMAX; ++i) acc = fmaf(a_at(i), xr[j][i].get(v), acc);
          y[j][v] = acc;
          ss = fmaf(acc, acc, ss);
        }
      }
      ss = wave_sum(ss);
      if (lane == 0) s_red[it & 1][wave] = ss;
      __syncthreads();
      float tot = 0.0f;
      for (int w = 0; w < nwaves; ++w) tot += s_red[it & 1][w];
      const float inv = 1.0f / sqrtf(tot / (float)C + A.eps);
      if (A.inv_rms != nullptr && tid == 0) A.inv_rms[t] = inv;
#pragma unroll
      for (int j = 0; j < CH; ++j) {
        const int q = tid + j * blockDim.x;
        const bool act = (j < A.ch) && (q < A.nchunks);
        if (!act) continue;
        const int c0 = q * V;
        const int valid = min(V, C - c0);
        float yn[V];
#pragma unroll
        for (int v = 0; v < V; ++v) yn[v] = (y[j][v] * inv) * s_w[(j * V + v) * blockDim.x + tid];
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          if (i < n) {
            float o[V];
#pragma unroll
            for (int v = 0; v < V; ++v) {
              float acc = 0.0f;
#pragma unroll
              for (int k = 0; k < NMAX; ++k) acc = fmaf(m_at(i, k), xr[j][k].get(v), acc);
              o[v] = fmaf(yn[v], p_at(i), acc);
            }
            OT* dst = ot + (int64_t)i * C + c0;
            if (A.vec && valid == V) store_vec<OT, V>(dst, o);
            else store_partial<OT, V>(dst, o, valid);
          }
        }
      }
    } else {
      // two passes over x (tile larger than the register budget)
      float ss = 0.0f;
      for (int q = tid; q < A.nchunks; q += blockDim.x) {
        const int c0 = q * V;
        const int valid = min(V, C - c0);
        float y[V];
#pragma unroll
        for (int v = 0; v < V; ++v) y[v] = 0.0f;
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          if (i < n) {
            Vec<XT, V> xv;
            if (A.vec && valid == V) xv.load(xt + (int64_t)i * C + c0);
            else xv.load_partial(xt + (int64_t)i * C + c0, valid);
#pragma unroll
            for (int v = 0; v < V; ++v) y[v] = fmaf(a_at(i), xv.get(v), y[v]);
          }
        }
#pragma unroll
        for (int v = 0; v < V; ++v) ss = fmaf(y[v], y[v], ss);
      }
      ss = wave_sum(ss);
      if (lane == 0) s_red[it & 1][wave] = ss;
      __syncthreads();
      float tot = 0.0f;
      for (int w = 0; w < nwaves; ++w) tot += s_red[it & 1][w];
      const float inv = 1.0f / sqrtf(tot / (float)C + A.eps);
      if (A.inv_rms != nullptr && tid == 0) A.inv_rms[t] = inv;
      for (int q = tid; q < A.nchunks; q += blockDim.x) {
        const int c0 = q * V;
        const int valid = min(V, C - c0);
        Vec<XT, V> xr[NMAX];
        float yn[V];
#pragma unroll
        for (int v = 0; v < V; ++v) yn[v] = 0.0f;
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          if (i < n) {
            if (A.vec && valid == V) xr[i].load(xt + (int64_t)i * C + c0);
            else xr[i].load_partial(xt + (int64_t)i * C + c0, valid);
          } else {
            xr[i].zero();
          }
#pragma unroll
          for (int v = 0; v < V; ++v) yn[v] = fmaf(a_at(i), xr[i].get(v), yn[v]);
        }
#pragma unroll
        for (int v = 0; v < V; ++v) yn[v] = (yn[v] * inv) * (c0 + v < C ? Wt[c0 + v] : 0.0f);
#pragma unroll
        for (int i = 0; i < NMAX; ++i) {
          if (i < n) {
            float o[V];
#pragma unroll
            for (int v = 0; v < V; ++v) {
              float acc = 0.0f;
#pragma unroll
              for (int k = 0; k < NMAX; ++k) acc = fmaf(m_at(i, k), xr[k].get(v), acc);
              o[v] = fmaf(yn[v], p_at(i), acc);
            }
            OT* dst = ot + (int64_t)i * C + c0;
            if (A.vec && valid == V) store_vec<OT, V>(dst, o);
            else store_partial<OT, V>(dst, o, valid);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Layer-wide parameters, n == NMAX <= 8, full tiles (the headline shapes).
//
// One workgroup per token: TPB threads own CH chunks of V channels each and
// exactly cover the token (C == TPB * CH * V), 16-byte aligned rows.  No
// per-stream, per-chunk or per-channel conditions remain; M, a and p are
// wave-uniform scalars.  The grid-stride loop only matters for T > kMaxGrid.
// ---------------------------------------------------------------------------

// MHC_FWD_WPE > 0 (a build-time tuning knob) caps the registers of the
// full-tile forward at that many waves per SIMD.
#ifndef MHC_FWD_WPE
#define MHC_FWD_WPE 0
#endif
#if MHC_FWD_WPE > 0
#define MHC_FWD_FULL_ATTR __attribute__((amdgpu_waves_per_eu(MHC_FWD_WPE)))
#else
#define MHC_FWD_FULL_ATTR
#endif

// Channels per chunk of the full-tile kernel: 16 bytes per lane of the wider
// of x and out (8 channels for 16-bit I/O, 4 with an fp32 side), so every
// load and store is one coalesced access of at most 16 bytes per lane.
template <typename XT, typename OT>
constexpr int full_vec() {
  return 16 / (ElemTraits<XT>::kBytes > ElemTraits<OT>::kBytes ? ElemTraits<XT>::kBytes : ElemTraits<OT>::kBytes);
}

// PIPE (persistent grid): the next token's loads are issued before this
// token's RMS barrier, into a second register set, so they are in flight
// across the barrier and the stores (the barrier waits for LDS only).
template <int NMAX, typename XT, typename OT, int CH, bool RAW, bool SKF = false, bool PIPE = false>
// (n = 8 with two chunks per thread holds 128 fp32 values of x per thread: bounded at 512 threads, so
// 256 VGPRs, where the 1024-thread bound spilled)
__global__ __launch_bounds__(NMAX == 8 && CH == 2 ? 512 : 1024) MHC_FWD_FULL_ATTR
void fused_fwd_full_kernel(FwdArgs A) {
  static_assert(!(PIPE && SKF), "the pipelined forward reads M");
  constexpr int V = full_vec<XT, OT>();
  __shared__ float s_red[2][16];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int C = A.C;
  const int64_t nC = (int64_t)NMAX * C;
  int c0[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) c0[k] = (tid + k * (int)blockDim.x) * V;

  // SKF: the Sinkhorn projection of the layer-wide logits runs in every wave
  // (after the first token's loads are issued); block 0 stores M for the backward.
  float Mk[SKF ? NMAX * NMAX : 1];

  // parameters and the lane's rms weights: per token (PIPE: once, before the first token's loads are waited
  // for, since a load issued after a token's stores would wait for those stores too)
  float Ms[NMAX * NMAX], as[NMAX], ps[NMAX], wv[CH][V];
  auto load_params = [&]() {
#pragma unroll
    for (int i = 0; i < NMAX; ++i) {
      float av = A.hpre[i], pv = A.hpost[i];
      if constexpr (RAW) {
        av = sigmoidf_(av);
        pv = 2.0f * sigmoidf_(pv);
      }
      as[i] = uniform_f(av);
      ps[i] = uniform_f(pv);
#pragma unroll
      for (int j = 0; j < NMAX; ++j) {
        if constexpr (SKF) Ms[i * NMAX + j] = Mk[i * NMAX + j];
        else Ms[i * NMAX + j] = uniform_f(A.M[i * NMAX + j]);
      }
    }
#pragma unroll
    for (int k = 0; k < CH; ++k)
#pragma unroll
      for (int v = 0; v < V; ++v) wv[k][v] = A.w[c0[k] + v];
  };
  Vec<XT, V> xr[CH][NMAX];
  auto load_tok = [&](Vec<XT, V> (&xa)[CH][NMAX], int64_t t) {
    const XT* xt = (const XT*)A.x + t * nC;
#pragma unroll
    for (int k = 0; k < CH; ++k)
#pragma unroll
      for (int i = 0; i < NMAX; ++i) xa[k][i].load(xt + i * C + c0[k]);
  };
  if constexpr (PIPE) {
    if ((int64_t)blockIdx.x < A.T) load_tok(xr, blockIdx.x);
    load_params();
    // enter the loop with no loads pending (else every token's first wait would be as strict as this one)
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
  }

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    // the token's loads go out first; parameters and w are read while they fly
    OT* ot = (OT*)A.out + t * nC;
    if constexpr (!PIPE) load_tok(xr, t);
    if constexpr (SKF) {
      if (it == 0) {
        float mine;
        sk_fwd_wave<NMAX>(A.hres, A.iters, A.eps, lane, Mk, mine);
        if (blockIdx.x == 0 && tid < NMAX * NMAX) A.M_out[tid] = mine;
      }
    }
    if constexpr (!PIPE) load_params();

    float y[CH][V];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
#pragma unroll
      for (int v = 0; v < V; ++v) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < NMAX; ++i) acc = fmaf(as[i], xr[k][i].get(v), acc);
        y[k][v] = acc;
        ss = fmaf(acc, acc, ss);
      }
    }
    ss = wave_sum(ss);
    if (lane == 0) s_red[it & 1][wave] = ss;
    Vec<XT, V> xn[PIPE ? CH : 1][NMAX];
    if constexpr (PIPE) {
      if (t + gridDim.x < A.T) load_tok(xn, t + gridDim.x);
      lds_barrier();
    } else {
      __syncthreads();
    }
    float tot = 0.0f;
    for (int w = 0; w < nwaves; ++w) tot += s_red[it & 1][w];
    const float inv = 1.0f / sqrtf(tot / (float)C + A.eps);
    if (A.inv_rms != nullptr && tid == 0) A.inv_rms[t] = inv;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      float yn[V];
#pragma unroll
      for (int v = 0; v < V; ++v) yn[v] = (y[k][v] * inv) * wv[k][v];
#pragma unroll
      for (int i = 0; i < NMAX; ++i) {
        float o[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
          float acc = 0.0f;
#pragma unroll
          for (int j = 0; j < NMAX; ++j) acc = fmaf(Ms[i * NMAX + j], xr[k][j].get(v), acc);
          o[v] = fmaf(yn[v], ps[i], acc);
        }
        store_vec<OT, V>(ot + i * C + c0[k], o);
      }
    }
    if constexpr (PIPE) {
#pragma unroll
      for (int k = 0; k < CH; ++k)
#pragma unroll
        for (int i = 0; i < NMAX; ++i) xr[k][i] = xn[k][i];
    }
  }
}

// ---------------------------------------------------------------------------
// n == 16, 16-bit x, C a multiple of 128: the stream mix and the aggregate on
// MFMA (config 3 and any 16-stream layer).
//
// At n = 16 the mix is 256 FMAs per channel, more VALU issue time than the
// token's HBM time, so it moves to the matrix cores: per 16 channels
//   out[0..16) = M X,   y = a^T X     (X = 16 streams x 16 channels)
// as v_mfma_f32_16x16x16 with M and a (fp32) each split into three 16-bit
// terms (split3): the products are those of fp32 M and a with the 16-bit
// x, accumulated in fp32.  For y the A operand repeats a in every row, so
// every lane receives y of its column.
//
// Layout: a wave handles slabs of 128 channels; lane (q = lane >> 4,
// r = lane & 15) loads streams 4q .. 4q+3 of channels [8r, 8r + 8) of the
// slab (four 16-byte loads).  For MFMA number v (0..7) the B operand of the
// lane is stream 4q .. 4q+3 of channel 8r + v, and the result D holds out of
// streams 4q .. 4q+3 at that channel: after the eight MFMAs the lane owns
// out for exactly the elements it loaded, stored as 16-byte rows.  One token
// per workgroup of S / SPW waves (S = C / 128 slabs, SPW slabs per wave).
// ---------------------------------------------------------------------------

template <typename XT, typename OT, int SPW, bool PT, bool RAW>
__global__ __launch_bounds__(SPW == 2 ? 512 : 1024) void fused_fwd_mfma16_kernel(FwdArgs A) {
  constexpr int N = 16;
  __shared__ float s_red[2][16];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int C = A.C;
  const int64_t nC = (int64_t)N * C;
  int cb[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) cb[s] = (wave * SPW + s) * 128 + 8 * r;

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const XT* xt = (const XT*)A.x + t * nC;
    OT* ot = (OT*)A.out + t * nC;
    Vec<XT, 8> xr[SPW][4];
#pragma unroll
    for (int s = 0; s < SPW; ++s)
#pragma unroll
      for (int k = 0; k < 4; ++k) xr[s][k].load(xt + (int64_t)(4 * q + k) * C + cb[s]);

    // parameters of this token: M row r, columns 4q..4q+3; a and p of streams 4q..4q+3
    const float4 m4 = *reinterpret_cast<const float4*>(A.M + (PT ? t * 256 : 0) + r * 16 + 4 * q);
    const float4 h4 = *reinterpret_cast<const float4*>(A.hpre + (PT ? t * 16 : 0) + 4 * q);
    const float4 g4 = *reinterpret_cast<const float4*>(A.hpost + (PT ? t * 16 : 0) + 4 * q);
    float av[4] = {h4.x, h4.y, h4.z, h4.w}, pv[4] = {g4.x, g4.y, g4.z, g4.w};
    if constexpr (RAW) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        av[k] = sigmoidf_(av[k]);
        pv[k] = 2.0f * sigmoidf_(pv[k]);
      }
    }
    uint2 am[3], aa[3];
    {
      const float mv[4] = {m4.x, m4.y, m4.z, m4.w};
      split3x4<XT>(mv, am);
      split3x4<XT>(av, aa);
    }

    // rms weight of the lane's channels, in flight with the tile
    float4 wq[SPW][2];
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      wq[s][0] = *reinterpret_cast<const float4*>(A.w + cb[s]);
      wq[s][1] = *reinterpret_cast<const float4*>(A.w + cb[s] + 4);
    }
    f32x4 dmix[SPW][8];
    float y[SPW][8];
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int wd = v >> 1;
        uint2 b;
        if (v & 1) {
          b.x = pack_hi16<XT>(xr[s][0].w[wd], xr[s][1].w[wd]);
          b.y = pack_hi16<XT>(xr[s][2].w[wd], xr[s][3].w[wd]);
        } else {
          b.x = pack_lo16<XT>(xr[s][0].w[wd], xr[s][1].w[wd]);
          b.y = pack_lo16<XT>(xr[s][2].w[wd], xr[s][3].w[wd]);
        }
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        f32x4 accy = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 2; e >= 0; --e) {
          acc = mfma16<XT>(am[e], b, acc);
          accy = mfma16<XT>(aa[e], b, accy);
        }
        dmix[s][v] = acc;
        y[s][v] = accy[0];
        ss = fmaf(accy[0], accy[0], ss);
      }
    }
    // the four lanes of a column hold the same y: count it once
    ss = q == 0 ? ss : 0.0f;
    ss = wave_sum(ss);
    if (lane == 0) s_red[it & 1][wave] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int w = 0; w < nwaves; ++w) tot += s_red[it & 1][w];
    const float inv = 1.0f / sqrtf(tot / (float)C + A.eps);
    if (A.inv_rms != nullptr && tid == 0) A.inv_rms[t] = inv;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      const float4 w0 = wq[s][0], w1 = wq[s][1];
      const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      float yn[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) yn[v] = (y[s][v] * inv) * wv[v];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float o[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) o[v] = fmaf(yn[v], pv[k], dmix[s][v][k]);
        store_vec<OT, 8>(ot + (int64_t)(4 * q + k) * C + cb[s], o);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

namespace {

// MFMA kernel for n == 16 with 16-bit x.  Returns 1 when the shape is not
// covered (the caller then uses fused_fwd_kernel).
template <typename XT, typename OT, bool PT>
int launch_fwd_mfma16(FwdArgs A, hipStream_t stream) {
  if constexpr (std::is_same<XT, float>::value) {
    return 1;
  } else {
    if (A.n != 16 || !A.vec || A.C % 128 != 0) return 1;
    if (!aligned(A.M, 16) || !aligned(A.hpre, 16) || !aligned(A.hpost, 16) || !aligned(A.w, 16)) return 1;
    if (knob(kKnobFwdMfma, 1) == 0) return 1;
    const int S = A.C / 128;
    int spw = knob(kKnobFwdSpw, S % 2 == 0 && S >= 8 ? 2 : 1);
    if (spw != 1 && spw != 2) spw = 1;
    if (S % spw != 0) spw = 1;
    const int waves = S / spw;
    if (waves > (spw == 2 ? 8 : 16)) return 1;
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(A.T, kMaxGrid));
    const dim3 g((unsigned)blocks), b(waves * 64);
    const bool raw = A.h_mode == MHC_H_RAW;
    if (spw == 2) {
      if (raw) hipLaunchKernelGGL((fused_fwd_mfma16_kernel<XT, OT, 2, PT, true>), g, b, 0, stream, A);
      else hipLaunchKernelGGL((fused_fwd_mfma16_kernel<XT, OT, 2, PT, false>), g, b, 0, stream, A);
    } else {
      if (raw) hipLaunchKernelGGL((fused_fwd_mfma16_kernel<XT, OT, 1, PT, true>), g, b, 0, stream, A);
      else hipLaunchKernelGGL((fused_fwd_mfma16_kernel<XT, OT, 1, PT, false>), g, b, 0, stream, A);
    }
    MHC_CHECK_LAUNCH("fused_fwd_mfma16_kernel");
    return MHC_OK;
  }
}

// Full-tile kernel for layer-wide n == NMAX <= 8.  Returns 1 when the shape
// is not covered (the caller then uses fused_fwd_kernel).
template <int NMAX, typename XT, typename OT>
int launch_fwd_full(FwdArgs A, hipStream_t stream) {
  // A.vec (checked for 8-channel chunks) implies the alignment of narrower ones
  constexpr int V = full_vec<XT, OT>();
  if (A.n != NMAX || !A.vec || A.C % V != 0) return 1;
  const int nchunks = A.C / V;
  // Workgroups of at most 512 threads, one chunk per thread where that fits:
  // at 32768 tokens x 4 x 4096, bf16 -> bf16 (8-channel chunks) runs 355 us
  // with one chunk per thread against 380 us with two; bf16 -> fp32
  // (4-channel chunks) 566 us with two against 625 us with one (1024 threads).
  int ch = nchunks <= 512 ? 1 : 2;
  const int ch_pref = knob(kKnobFwdCh, 0);
  if (ch_pref == 1 || ch_pref == 2) ch = ch_pref;
  if (nchunks % (64 * ch) != 0) ch = 1;
  if (nchunks % 64 != 0 || nchunks / ch > (NMAX == 8 && ch == 2 ? 512 : 1024)) return 1;
  const int tpb = nchunks / ch;
  const bool raw = A.h_mode == MHC_H_RAW;
  // n = 4: MHC_FWD_PIPE > 0 takes the pipelined kernel on a persistent grid of that many workgroups per
  // CU.  Alone it ran config 2's forward 7-10 us faster at one workgroup per CU (two to four: slower),
  // but the training step moved by -10, +2.5 and +0.8 us on three boxes, so it is not the default.
  if constexpr (NMAX == 4) {
    const int pipe = knob(kKnobFwdPipe, 0);
    if (pipe > 0 && ch == 1 && raw) {
      // persistent pipelined grid: `pipe` workgroups per CU
      const int64_t pb = std::max<int64_t>(1, std::min<int64_t>(A.T, (int64_t)device_cu_count() * pipe));
      hipLaunchKernelGGL((fused_fwd_full_kernel<NMAX, XT, OT, 1, true, false, true>), dim3((unsigned)pb), dim3(tpb),
                         0, stream, A);
      MHC_CHECK_LAUNCH("fused_fwd_full_kernel");
      return MHC_OK;
    }
  }
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(A.T, kMaxGrid));
  const dim3 g((unsigned)blocks), b(tpb);
  if (ch == 2) {
    if (raw) hipLaunchKernelGGL((fused_fwd_full_kernel<NMAX, XT, OT, 2, true>), g, b, 0, stream, A);
    else hipLaunchKernelGGL((fused_fwd_full_kernel<NMAX, XT, OT, 2, false>), g, b, 0, stream, A);
  } else {
    if (raw) hipLaunchKernelGGL((fused_fwd_full_kernel<NMAX, XT, OT, 1, true>), g, b, 0, stream, A);
    else hipLaunchKernelGGL((fused_fwd_full_kernel<NMAX, XT, OT, 1, false>), g, b, 0, stream, A);
  }
  MHC_CHECK_LAUNCH("fused_fwd_full_kernel");
  return MHC_OK;
}

template <int NMAX, typename XT, typename OT, bool PT>
int launch_fwd(FwdArgs A, hipStream_t stream) {
  constexpr int V = FwdCfg<NMAX>::V;
  constexpr int CH = FwdCfg<NMAX>::CH;
  constexpr int NPAR = NMAX * NMAX + 2 * NMAX;
  if constexpr (!PT && NMAX <= 8) {
    const int rc = launch_fwd_full<NMAX, XT, OT>(A, stream);
    if (rc != 1) return rc;
  }
  if constexpr (NMAX == 16) {
    const int rc = launch_fwd_mfma16<XT, OT, PT>(A, stream);
    if (rc != 1) return rc;
  }
  A.nchunks = (int)ceil_div(A.C, V);
  const ThreadPlan tp = plan_threads(A.nchunks, CH, knob(kKnobFwdTpb, 0), 1024);
  A.ch = tp.ch;
  A.reload = tp.reload;
  const bool par_lds = PT || NMAX > 8;
  const size_t smem = (par_lds ? (size_t)(PT ? 3 : 1) * NPAR * sizeof(float) : 0) +
                      (tp.reload ? 0 : (size_t)CH * V * tp.tpb * sizeof(float));
  const void* kfn = (const void*)fused_fwd_kernel<NMAX, XT, OT, PT>;
  const int occ = occupancy_blocks(kfn, tp.tpb, smem);
  if (occ <= 0)
    return set_error(MHC_ERR_INVALID_ARG, "fused_fwd: no occupancy for %d threads (n=%d C=%d)",
                     tp.tpb, A.n, A.C);
  // Persistent grid (per-token parameters are staged one token ahead).
  const int grid_per_cu = knob(kKnobFwdGrid, 0);
  int64_t blocks = (int64_t)device_cu_count() * (grid_per_cu > 0 ? grid_per_cu : occ);
  blocks = std::max<int64_t>(1, std::min<int64_t>(A.T, blocks));
  hipLaunchKernelGGL((fused_fwd_kernel<NMAX, XT, OT, PT>), dim3((unsigned)blocks), dim3(tp.tpb),
                     smem, stream, A);
  MHC_CHECK_LAUNCH("fused_fwd_kernel");
  return MHC_OK;
}

template <typename XT, typename OT, bool PT>
int dispatch_n(const FwdArgs& A, hipStream_t s) {
  switch (nmax_for(A.n)) {
    case 4: return launch_fwd<4, XT, OT, PT>(A, s);
    case 8: return launch_fwd<8, XT, OT, PT>(A, s);
    default: return launch_fwd<16, XT, OT, PT>(A, s);
  }
}

template <bool PT>
int dispatch_types(const FwdArgs& A, int xd, int od, hipStream_t s) {
  if (xd == MHC_DTYPE_F32 && od == MHC_DTYPE_F32) return dispatch_n<float, float, PT>(A, s);
  if (xd == MHC_DTYPE_BF16 && od == MHC_DTYPE_F32) return dispatch_n<__bf16, float, PT>(A, s);
  if (xd == MHC_DTYPE_BF16 && od == MHC_DTYPE_BF16) return dispatch_n<__bf16, __bf16, PT>(A, s);
  if (xd == MHC_DTYPE_F16 && od == MHC_DTYPE_F32) return dispatch_n<_Float16, float, PT>(A, s);
  if (xd == MHC_DTYPE_F16 && od == MHC_DTYPE_F16) return dispatch_n<_Float16, _Float16, PT>(A, s);
  return set_error(MHC_ERR_INVALID_ARG,
                   "fused_fwd: unsupported (x_dtype=%d, out_dtype=%d); out must be fp32 or x's dtype",
                   xd, od);
}

}  // namespace
}  // namespace mhc

using namespace mhc;

extern "C" int mhc_fused_fwd(const void* x, int x_dtype, const float* M, int64_t M_token_stride,
                             const float* h_pre, const float* h_post, int64_t h_token_stride,
                             int h_mode, const float* rms_weight, void* out, int out_dtype,
                             float* inv_rms, int64_t T, int n, int C, float eps, void* stream) {
  clear_error();
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
  if (T == 0) return MHC_OK;
  MHC_CHECK_ARG(x && M && h_pre && h_post && rms_weight && out, "null pointer argument");
  FwdArgs A{};
  A.x = x; A.out = out; A.inv_rms = inv_rms; A.M = M; A.hpre = h_pre; A.hpost = h_post;
  A.w = rms_weight; A.T = T; A.M_ts = (int)M_token_stride; A.h_ts = (int)h_token_stride; A.n = n; A.C = C;
  A.h_mode = h_mode; A.eps = eps;
  const int xb = dtype_bytes(x_dtype), ob = dtype_bytes(out_dtype);
  MHC_CHECK_ARG(xb > 0 && ob > 0, "unknown dtype code");
  MHC_CHECK_ARG(out_dtype == MHC_DTYPE_F32 || out_dtype == x_dtype,
                "out_dtype (%d) must be fp32 or x_dtype (%d)", out_dtype, x_dtype);
  if (nmax_for(n) == 0) {
    Mf32Args F{};
    F.x = x; F.out = out; F.inv_rms = inv_rms; F.M = M; F.hpre = h_pre; F.hpost = h_post; F.w = rms_weight;
    F.T = T; F.M_ts = M_token_stride; F.h_ts = h_token_stride; F.n = n; F.C = C; F.h_mode = h_mode; F.eps = eps;
    const int rc = mf32_fused_fwd(F, x_dtype, out_dtype, (hipStream_t)stream);
    if (rc != 1) return rc;
    GenArgs G{};
    G.x = x; G.out = out; G.M = M; G.hpre = h_pre; G.hpost = h_post; G.w = rms_weight;
    G.inv_rms = inv_rms; G.T = T; G.M_ts = M_token_stride; G.h_ts = h_token_stride; G.n = n;
    G.C = C; G.h_mode = h_mode; G.eps = eps;
    return gen_fused_fwd(G, x_dtype, out_dtype, (hipStream_t)stream);
  }
  const int V = fwd_vec_width(nmax_for(n));
  const int align_x = std::min(16, V * xb), align_o = std::min(16, V * ob);
  A.vec = (C % V == 0) && aligned(x, align_x) && aligned(out, align_o) &&
          ((int64_t)C * xb) % align_x == 0 && ((int64_t)C * ob) % align_o == 0 ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  return M_token_stride ? dispatch_types<true>(A, x_dtype, out_dtype, s)
                        : dispatch_types<false>(A, x_dtype, out_dtype, s);
}

namespace mhc {
namespace {

// One launch for the layer-wide forward at n == NMAX <= 8 with few tokens
// (at most one per CU): the Sinkhorn projection runs in the forward kernel
// instead of a launch of its own.  Returns 1 when the shape is not covered.
template <int NMAX, typename XT, typename OT>
int launch_fwd_full_skf(FwdArgs A, hipStream_t stream) {
  constexpr int V = full_vec<XT, OT>();
  if (A.n != NMAX || !A.vec || A.C % V != 0) return 1;
  const int nchunks = A.C / V;
  if (nchunks % 64 != 0 || nchunks > 1024) return 1;
  hipLaunchKernelGGL((fused_fwd_full_kernel<NMAX, XT, OT, 1, true, true>), dim3((unsigned)A.T), dim3(nchunks), 0,
                     stream, A);
  MHC_CHECK_LAUNCH("fused_fwd_full_kernel");
  return MHC_OK;
}

int layer_fwd_single_launch(const FwdArgs& A, int xd, int od, hipStream_t s) {
  if (knob(kKnobFwdSkf, 1) == 0 || A.T < 1 || A.T > device_cu_count()) return 1;
  if (xd == MHC_DTYPE_BF16 && od == MHC_DTYPE_BF16) {
    if (A.n == 4) return launch_fwd_full_skf<4, __bf16, __bf16>(A, s);
    if (A.n == 8) return launch_fwd_full_skf<8, __bf16, __bf16>(A, s);
  } else if (xd == MHC_DTYPE_BF16 && od == MHC_DTYPE_F32) {
    if (A.n == 4) return launch_fwd_full_skf<4, __bf16, float>(A, s);
    if (A.n == 8) return launch_fwd_full_skf<8, __bf16, float>(A, s);
  } else if (xd == MHC_DTYPE_F32 && od == MHC_DTYPE_F32) {
    if (A.n == 4) return launch_fwd_full_skf<4, float, float>(A, s);
    if (A.n == 8) return launch_fwd_full_skf<8, float, float>(A, s);
  } else if (xd == MHC_DTYPE_F16 && od == MHC_DTYPE_F16) {
    if (A.n == 4) return launch_fwd_full_skf<4, _Float16, _Float16>(A, s);
    if (A.n == 8) return launch_fwd_full_skf<8, _Float16, _Float16>(A, s);
  } else if (xd == MHC_DTYPE_F16 && od == MHC_DTYPE_F32) {
    if (A.n == 4) return launch_fwd_full_skf<4, _Float16, float>(A, s);
    if (A.n == 8) return launch_fwd_full_skf<8, _Float16, float>(A, s);
  }
  return 1;
}

}  // namespace
}  // namespace mhc

extern "C" int mhc_layer_fwd(const void* x, int x_dtype, const float* h_pre_raw, const float* h_post_raw,
                             const float* h_res_raw, const float* rms_weight, void* out, int out_dtype,
                             float* M_out, int64_t T, int n, int C, int per_token, int iters, float eps,
                             void* stream) {
  clear_error();
  MHC_CHECK_ARG(T >= 0, "T=%lld must be >= 0", (long long)T);
  MHC_CHECK_ARG(M_out != nullptr && h_res_raw != nullptr, "null pointer argument");
  if (!per_token && (n == 4 || n == 8) && T >= 1 && iters >= 0 && x && h_pre_raw && h_post_raw && rms_weight &&
      out && dtype_bytes(x_dtype) && dtype_bytes(out_dtype)) {
    FwdArgs A{};
    A.x = x; A.out = out; A.M = M_out; A.hpre = h_pre_raw; A.hpost = h_post_raw; A.w = rms_weight; A.T = T;
    A.n = n; A.C = C; A.h_mode = MHC_H_RAW; A.eps = eps; A.hres = h_res_raw; A.M_out = M_out; A.iters = iters;
    const int V = fwd_vec_width(nmax_for(n));
    const int xb = dtype_bytes(x_dtype), ob = dtype_bytes(out_dtype);
    const int align_x = std::min(16, V * xb), align_o = std::min(16, V * ob);
    A.vec = (C >= 1 && C % V == 0) && aligned(x, align_x) && aligned(out, align_o) &&
            ((int64_t)C * xb) % align_x == 0 && ((int64_t)C * ob) % align_o == 0 ? 1 : 0;
    const int rc = layer_fwd_single_launch(A, x_dtype, out_dtype, (hipStream_t)stream);
    if (rc != 1) return rc;
  }
  if (!per_token && n > 16 && n <= 32 && T >= 1 && iters >= 0 && x && h_pre_raw && h_post_raw && rms_weight &&
      out && (out_dtype == MHC_DTYPE_F32 || out_dtype == x_dtype) && dtype_bytes(x_dtype) == 2) {
    Mf32Args F{};
    F.x = x; F.out = out; F.M = M_out; F.hpre = h_pre_raw; F.hpost = h_post_raw; F.w = rms_weight; F.T = T;
    F.n = n; F.C = C; F.h_mode = MHC_H_RAW; F.eps = eps; F.hres = h_res_raw; F.M_out = M_out; F.iters = iters;
    const int rc = mf32_layer_fwd_single_launch(F, x_dtype, out_dtype, (hipStream_t)stream);
    if (rc != 1) return rc;
  }
  const int64_t batch = per_token ? T : 1;
  if (batch > 0) {
    const int rc = mhc_sinkhorn_fwd(h_res_raw, M_out, batch, n, iters, eps, stream);
    if (rc != MHC_OK) return rc;
  }
  return mhc_fused_fwd(x, x_dtype, M_out, per_token ? (int64_t)n * n : 0, h_pre_raw, h_post_raw,
                       per_token ? n : 0, MHC_H_RAW, rms_weight, out, out_dtype, nullptr, T, n, C, eps, stream);
}
