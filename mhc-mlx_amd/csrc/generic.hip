// Kernels for 16 < n <= 64 (the reference allows n up to 64: metal.py:71),
// templated on NMAX = 32 or 64 register slots per channel with runtime n.
// A persistent workgroup walks tokens; threads own channels, keep a
// channel's n values in registers and mix them against rows of M broadcast
// from LDS; parameter-gradient sums are 4 x 4 outer-product blocks, one per
// wavefront.  The kernels in fused_fwd.hip / fused_bwd.hip / stream_mix.hip
// cover n <= 16.
#include <type_traits>

#include "mhc_device.hpp"
#include "mhc_generic.hpp"
#include "mhc_host.hpp"
#include "mhc_plan.hpp"
#include "mhc_reduce.hpp"

namespace mhc {

namespace {

constexpr int kGenThreads = 256;
// The layer backward takes its parameter sums one 4 x 4 block per wavefront;
// at n <= 32 its registers allow 512-thread workgroups (at most 256 VGPRs),
// which measured 4.7 -> 3.0 ms at n = 32.  The post-combine VJP measured
// slower with 1024 threads (0.97 -> 1.24 ms) and keeps kGenThreads.
constexpr int gen_bwd_threads(int nmax) { return nmax <= 32 ? 512 : 256; }
constexpr int kGenMaxWaves = 8;
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

// Forward.  A thread owns channels c = tid, tid + blockDim.x, ...; in the
// second pass the n values of its channel sit in registers (NMAX = 32 or 64
// slots, the unused ones zero) and the n x n mix runs from them against rows
// of M broadcast from LDS as float4s (row stride NMAX, zero-padded), so x is
// read once per pass instead of once per output stream.
template <typename XT, typename OT, int NMAX>
__global__ __launch_bounds__(kGenThreads) void gen_fwd_kernel(GenArgs A) {
  __shared__ float s_par[kGenMaxPar];
  __shared__ __align__(16) float s_M[NMAX * NMAX];
  __shared__ float s_red[2][kGenThreads / 64];
  const int n = A.n, C = A.C, nn = n * n;
  const XT* X = (const XT*)A.x;
  OT* O = (OT*)A.out;
  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    __syncthreads();  // previous token done with s_par / s_M
    gen_stage(s_par, A.M + t * A.M_ts, A.hpre + t * A.h_ts, A.hpost + t * A.h_ts, n, A.h_mode);
    const float* Mt = A.M + t * A.M_ts;
    for (int k = threadIdx.x; k < NMAX * NMAX; k += blockDim.x) {
      const int i = k / NMAX, j = k % NMAX;
      s_M[k] = (i < n && j < n) ? Mt[i * n + j] : 0.0f;
    }
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
      float xv[NMAX];
#pragma unroll
      for (int j = 0; j < NMAX; ++j) xv[j] = j < n ? load1<XT>(xt + (int64_t)j * C + c) : 0.0f;
      float y = 0.0f;
#pragma unroll
      for (int j = 0; j < NMAX; ++j) y = fmaf(j < n ? s_par[nn + j] : 0.0f, xv[j], y);
      const float yn = (y * inv) * A.w[c];
      for (int i = 0; i < n; ++i) {
        const float4* Mi = reinterpret_cast<const float4*>(s_M + i * NMAX);
        float acc = 0.0f;
#pragma unroll
        for (int j4 = 0; j4 < NMAX / 4; ++j4) {
          const float4 m = Mi[j4];
          acc = fmaf(m.x, xv[4 * j4], acc);
          acc = fmaf(m.y, xv[4 * j4 + 1], acc);
          acc = fmaf(m.z, xv[4 * j4 + 2], acc);
          acc = fmaf(m.w, xv[4 * j4 + 3], acc);
        }
        store1<OT>(ot + (int64_t)i * C + c, fmaf(yn, s_par[nn + n + i], acc));
      }
    }
  }
}

// Backward.  Per token:
//  pass 1: y = a.x and d = p.g per channel give sum y^2 and sum d y w;
//  pass 2: the n values of g of a channel sit in registers (NMAX slots, the
//          unused ones zero); dx_j = sum_i M_ij g_i + a_j dy runs against rows
//          of M^T broadcast from LDS as float4s; dy and yn = y inv w go to
//          this workgroup's scratch rows and dw to its partial row;
//  pass 3: the parameter gradients are the sums over channels of an
//          (n+1) x (n+1) outer product -- rows g_0..g_{n-1}, dy; columns
//          x_0..x_{n-1}, yn: dM_ij = sum g_i x_j, dA_j = sum dy x_j,
//          dP_i = sum g_i yn.  A wavefront takes one 4 x 4 block at a time,
//          its lanes over consecutive channels (coalesced loads), and adds
//          the wave sums into the block's entries: in LDS across tokens for
//          layer-wide parameters, or straight to the per-token outputs.
//          Each entry belongs to one wavefront, so the order is fixed.
// 16 x 16 x 32 MFMA of 16-bit operands (eight elements per lane), fp32 accumulation.
typedef __bf16 gen_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 gen_f16x8 __attribute__((ext_vector_type(8)));
template <typename T>
MHC_DEV f32x4 gen_mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (std::is_same<T, __bf16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(gen_bf16x8, a), __builtin_bit_cast(gen_bf16x8, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(gen_f16x8, a), __builtin_bit_cast(gen_f16x8, b), c,
                                                  0, 0, 0);
}

// MF (16-bit x and dout of one dtype, C a multiple of 32, 16-byte aligned
// rows): pass 3's dM = G X^T runs on MFMA in 16 x 16 blocks of (stream i,
// stream j), each block owned by one wavefront for the whole kernel (at most
// kGenMfBlk per wave), K = 32 channels per v_mfma_f32_16x16x32: lane
// (q = lane >> 4, r = lane & 15) reads channels 32k + 8q .. + 7 of g row
// 16I + r and of x row 16J + r (rows past n as zero) and holds dM entries
// (16I + 4q + e, 16J + r).  The rows were just read by passes 1 and 2, so
// these reads come from the caches.  dA and dP (the extended row and column
// of the outer product) are dot products over the channels, one wavefront
// each.  Every sum has one owner, so the order is fixed.
template <int NMAX>
constexpr int gen_mf_blocks() {
  return ((NMAX / 16) * (NMAX / 16) + gen_bwd_threads(NMAX) / 64 - 1) / (gen_bwd_threads(NMAX) / 64);
}

template <typename XT, typename GT, int NMAX, bool MF = false>
__global__ __launch_bounds__(gen_bwd_threads(NMAX)) void gen_bwd_kernel(GenArgs A) {
  static_assert(!MF || (std::is_same<XT, GT>::value && sizeof(XT) == 2), "MFMA pass 3 takes 16-bit x == dout");
  constexpr int kMfBlk = gen_mf_blocks<NMAX>();
  f32x4 dmb[MF ? kMfBlk : 1];
#pragma unroll
  for (int b = 0; b < (MF ? kMfBlk : 1); ++b) dmb[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int NE = NMAX + 1;  // extended rows / columns
  __shared__ float s_par[kGenMaxPar];
  __shared__ __align__(16) float s_MT[NMAX * NMAX];
  __shared__ float s_acc[NE * NE];
  __shared__ float s_red[2][2][kGenMaxWaves];
  const int n = A.n, C = A.C, nn = n * n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int nb = (n + 1 + 3) / 4;  // 4-wide blocks of the n + 1 rows (and columns)
  const XT* X = (const XT*)A.x;
  const GT* Gd = (const GT*)A.g;
  XT* DX = (XT*)A.out;
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  float* sdy = A.scratch + (int64_t)blockIdx.x * 2 * A.C;
  float* syn = sdy + A.C;
  for (int c = threadIdx.x; c < A.P; c += blockDim.x) prow[c] = 0.0f;
  for (int k = threadIdx.x; k < NE * NE; k += blockDim.x) s_acc[k] = 0.0f;
  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    __syncthreads();  // previous token done with s_par / s_MT
    gen_stage(s_par, A.M + t * A.M_ts, A.hpre + t * A.h_ts, A.hpost + t * A.h_ts, n, A.h_mode);
    const float* Mt = A.M + t * A.M_ts;
    for (int k = threadIdx.x; k < NMAX * NMAX; k += blockDim.x) {
      const int j = k / NMAX, i = k % NMAX;  // s_MT[j][i] = M_ij
      s_MT[k] = (i < n && j < n) ? Mt[i * n + j] : 0.0f;
    }
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
      float gv[NMAX];
#pragma unroll
      for (int i = 0; i < NMAX; ++i) gv[i] = i < n ? load1<GT>(gt + (int64_t)i * C + c) : 0.0f;
      float y = 0.0f, d = 0.0f;
      for (int i = 0; i < n; ++i) y = fmaf(s_par[nn + i], load1<XT>(xt + (int64_t)i * C + c), y);
#pragma unroll
      for (int i = 0; i < NMAX; ++i) d = fmaf(i < n ? s_par[nn + n + i] : 0.0f, gv[i], d);
      const float wc = A.w[c];
      const float yi = y * inv;
      const float dy = d * inv * wc - kf * y;
      sdy[c] = dy;
      syn[c] = yi * wc;
      prow[c] = fmaf(d, yi, prow[c]);
      for (int j = 0; j < n; ++j) {
        const float4* Mj = reinterpret_cast<const float4*>(s_MT + j * NMAX);
        float acc = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < NMAX / 4; ++i4) {
          const float4 m = Mj[i4];
          acc = fmaf(m.x, gv[4 * i4], acc);
          acc = fmaf(m.y, gv[4 * i4 + 1], acc);
          acc = fmaf(m.z, gv[4 * i4 + 2], acc);
          acc = fmaf(m.w, gv[4 * i4 + 3], acc);
        }
        store1<XT>(dxt + (int64_t)j * C + c, fmaf(s_par[nn + j], dy, acc));
      }
    }
    __syncthreads();  // sdy / syn visible to the workgroup
    if constexpr (MF) {
      const int q = lane >> 4, r = lane & 15;
      const int nbk = (n + 15) / 16;
#pragma unroll
      for (int b = 0; b < kMfBlk; ++b) {
        const int blk = wave + b * nwaves;
        if (blk >= nbk * nbk) break;
        const int I = blk / nbk, J = blk % nbk;
        const int gi = 16 * I + r, xj = 16 * J + r;
        const XT* grow = (const XT*)gt + (int64_t)(gi < n ? gi : 0) * C + 8 * q;
        const XT* xrow = xt + (int64_t)(xj < n ? xj : 0) * C + 8 * q;
        f32x4 acc = A.M_ts ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : dmb[b];
        for (int k = 0; k < C; k += 32) {
          const u32x4 zero = {0u, 0u, 0u, 0u};
          const u32x4 ga = gi < n ? *reinterpret_cast<const u32x4*>(grow + k) : zero;
          const u32x4 xb = xj < n ? *reinterpret_cast<const u32x4*>(xrow + k) : zero;
          acc = gen_mfma<XT>(ga, xb, acc);
        }
        if (A.M_ts) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int i = 16 * I + 4 * q + e, j = 16 * J + r;
            if (i < n && j < n) A.dM_tok[t * nn + i * n + j] = acc[e];
          }
        } else {
          dmb[b] = acc;
        }
      }
      // dA_j = sum dy x_j (e < n), dP_i = sum g_i yn (e >= n): one wavefront per dot product
      for (int e = wave; e < 2 * n; e += nwaves) {
        const bool da = e < n;
        const int j = da ? e : e - n;
        float acc = 0.0f;
        for (int c = lane; c < C; c += 64)
          acc = da ? fmaf(sdy[c], load1<XT>(xt + (int64_t)j * C + c), acc)
                   : fmaf(load1<GT>(gt + (int64_t)j * C + c), syn[c], acc);
        const float v = wave_sum(acc);
        if (lane != 0) continue;
        if (A.M_ts) {
          if (da) {
            const float av = s_par[nn + j];
            A.dpre_tok[t * n + j] = A.h_mode == MHC_H_RAW ? v * av * (1.0f - av) : v;
          } else {
            const float pq = s_par[nn + n + j];
            A.dpost_tok[t * n + j] = A.h_mode == MHC_H_RAW ? v * pq * (1.0f - 0.5f * pq) : v;
          }
        } else if (da) {
          s_acc[n * NE + j] += v;
        } else {
          s_acc[j * NE + n] += v;
        }
      }
      continue;
    }
    for (int blk = wave; blk < nb * nb; blk += nwaves) {
      const int r0 = (blk / nb) * 4, c0 = (blk % nb) * 4;
      float acc[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
      for (int c = lane; c < C; c += 64) {
        float rv[4], cv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int ri = r0 + e, cj = c0 + e;
          rv[e] = ri < n ? load1<GT>(gt + (int64_t)ri * C + c) : (ri == n ? sdy[c] : 0.0f);
          cv[e] = cj < n ? load1<XT>(xt + (int64_t)cj * C + c) : (cj == n ? syn[c] : 0.0f);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = fmaf(rv[e >> 2], cv[e & 3], acc[e]);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float v = wave_sum(acc[e]);
        const int i = r0 + (e >> 2), j = c0 + (e & 3);
        if (lane != 0 || i > n || j > n || (i == n && j == n)) continue;
        if (A.M_ts) {
          if (i < n && j < n) {
            A.dM_tok[t * nn + i * n + j] = v;
          } else if (i == n) {  // dA_j
            const float av = s_par[nn + j];
            A.dpre_tok[t * n + j] = A.h_mode == MHC_H_RAW ? v * av * (1.0f - av) : v;
          } else {  // dP_i
            const float pq = s_par[nn + n + i];
            A.dpost_tok[t * n + i] = A.h_mode == MHC_H_RAW ? v * pq * (1.0f - 0.5f * pq) : v;
          }
        } else {
          s_acc[i * NE + j] += v;
        }
      }
    }
  }
  if constexpr (MF) {
    // the blocks of dM into s_acc (each entry written by its one owner)
    if (!A.M_ts) {
      const int q = lane >> 4, r = lane & 15;
      const int nbk = (n + 15) / 16;
#pragma unroll
      for (int b = 0; b < kMfBlk; ++b) {
        const int blk = wave + b * nwaves;
        if (blk >= nbk * nbk) break;
        const int I = blk / nbk, J = blk % nbk;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 16 * I + 4 * q + e, j = 16 * J + r;
          if (i < n && j < n) s_acc[i * NE + j] = dmb[b][e];
        }
      }
    }
  }
  __syncthreads();
  if (!A.M_ts) {
    // [Cp | dM n*n | dA n | dP n]
    for (int k = threadIdx.x; k < nn + 2 * n; k += blockDim.x) {
      float v;
      if (k < nn) v = s_acc[(k / n) * NE + (k % n)];
      else if (k < nn + n) v = s_acc[n * NE + (k - nn)];
      else v = s_acc[(k - nn - n) * NE + n];
      prow[A.Cp + k] = v;
    }
  }
}

// post-combine / stream_mix_add forward: out_i = p_i (y_i + sum_j M_ij a_j x_j).
// The n values of x at a (token, channel) item sit in registers (NMAX slots,
// the unused ones zero) against float4 rows of Mf_ij = M_ij a_j in LDS.
template <typename XT, typename YT, typename OT, int NMAX>
__global__ __launch_bounds__(kGenThreads) void gen_mix_fwd_kernel(GenArgs A) {
  __shared__ float s_par[kGenMaxPar];
  __shared__ __align__(16) float s_Mf[NMAX * NMAX];
  const int n = A.n, C = A.C, nn = n * n;
  gen_stage(s_par, A.M, A.hpre, A.hpost, n, A.h_mode);
  __syncthreads();
  for (int k = threadIdx.x; k < NMAX * NMAX; k += blockDim.x) {
    const int i = k / NMAX, j = k % NMAX;
    s_Mf[k] = (i < n && j < n) ? s_par[i * n + j] * s_par[nn + j] : 0.0f;
  }
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
    float xv[NMAX];
#pragma unroll
    for (int j = 0; j < NMAX; ++j) xv[j] = j < n ? load1<XT>(X + base + (int64_t)j * C) : 0.0f;
    for (int i = 0; i < n; ++i) {
      const float4* Mi = reinterpret_cast<const float4*>(s_Mf + i * NMAX);
      float acc = 0.0f;
#pragma unroll
      for (int j4 = 0; j4 < NMAX / 4; ++j4) {
        const float4 m = Mi[j4];
        acc = fmaf(m.x, xv[4 * j4], acc);
        acc = fmaf(m.y, xv[4 * j4 + 1], acc);
        acc = fmaf(m.z, xv[4 * j4 + 2], acc);
        acc = fmaf(m.w, xv[4 * j4 + 3], acc);
      }
      const float yv = Y ? load1<YT>(Y + base + (int64_t)i * C) : 0.0f;
      store1<OT>(O + base + (int64_t)i * C, s_par[nn + n + i] * (yv + acc));
    }
  }
}

// post-combine VJP: dx_j = a_j sum_i M_ij p_i g_i, dy_i = p_i g_i and the
// sums S_ij = sum g_i x_j, Yd_i = sum g_i y_i (one partial row per workgroup).
// dx runs from g in registers against rows of (M^T p) a in LDS.  S and Yd
// are taken per token in 4 x 4 blocks of rows g_i and columns x_j (column n:
// y_i of the same row), one block per wavefront at a time with the lanes
// over consecutive channels; each entry belongs to one wavefront, so the
// LDS sums have a fixed order.
// Eight floats as three packed 16-bit operands whose sum is the fp32 value (split3).
template <typename T>
MHC_DEV void gen_split3x8(const float (&v)[8], u32x4 (&out)[3]) {
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    float a = v[2 * h], b = v[2 * h + 1];
#pragma unroll
    for (int e = 0; e < 3; ++e) {
      const uint32_t wd = pack2<T>(a, b);
      a -= lo16<T>(wd);
      b -= hi16<T>(wd);
      out[e][h] = wd;
    }
  }
}

// MF (16-bit x, dout of x's dtype or fp32, C a multiple of 32, 16-byte
// aligned rows): the sums S = G X^T run on MFMA in 16 x 16 blocks owned by
// the waves for the whole kernel (as in gen_bwd_kernel), an fp32 dout split
// into three 16-bit terms per element (three MFMAs, fp32-accurate products);
// Yd_i = sum G_i Y_i is a dot product per row, one wavefront each, over
// 16-byte pieces.
template <typename XT, typename YT, typename GT, int NMAX, bool MF = false>
__global__ __launch_bounds__(kGenThreads) void gen_mix_bwd_kernel(GenArgs A) {
  static_assert(!MF || (sizeof(XT) == 2 && (std::is_same<GT, XT>::value || std::is_same<GT, float>::value)),
                "MFMA sums take 16-bit x and dout of x's dtype or fp32");
  constexpr int kMfBlk = ((NMAX / 16) * (NMAX / 16) + kGenThreads / 64 - 1) / (kGenThreads / 64);
  f32x4 smb[MF ? kMfBlk : 1];
#pragma unroll
  for (int b = 0; b < (MF ? kMfBlk : 1); ++b) smb[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  constexpr int NE = NMAX + 1;
  __shared__ float s_par[kGenMaxPar];
  __shared__ __align__(16) float s_W[NMAX * NMAX];  // s_W[j][i] = a_j M_ij p_i
  __shared__ float s_acc[NMAX * NE];
  const int n = A.n, C = A.C, nn = n * n, K = nn + n;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  gen_stage(s_par, A.M, A.hpre, A.hpost, n, A.h_mode);
  for (int k = threadIdx.x; k < NMAX * NE; k += blockDim.x) s_acc[k] = 0.0f;
  __syncthreads();
  for (int k = threadIdx.x; k < NMAX * NMAX; k += blockDim.x) {
    const int j = k / NMAX, i = k % NMAX;
    s_W[k] = (i < n && j < n) ? s_par[nn + j] * s_par[i * n + j] * s_par[nn + n + i] : 0.0f;
  }
  __syncthreads();
  const XT* X = (const XT*)A.x;
  const YT* Y = (const YT*)A.y;
  const GT* Gd = (const GT*)A.g;
  XT* DX = (XT*)A.out;
  YT* DY = (YT*)A.dy;
  const int nbr = (n + 3) / 4, nbc = (n + 1 + 3) / 4;  // row blocks, column blocks (column n: y)
  // tokens in groups of tpi (several per pass when C is below the workgroup size, so every thread has a
  // channel of the dx pass); the sums then take the group's tokens in order
  const int tpi = MF && C < (int)blockDim.x ? (int)blockDim.x / C : 1;
  for (int64_t t0 = blockIdx.x; t0 < A.T; t0 += (int64_t)gridDim.x * tpi) {
    for (int idx = threadIdx.x; idx < tpi * C; idx += blockDim.x) {
      const int u = idx / C, c = idx - u * C;
      const int64_t t = t0 + (int64_t)u * gridDim.x;
      if (t >= A.T) continue;
      const int64_t tb = t * n * C;
      float gv[NMAX];
#pragma unroll
      for (int i = 0; i < NMAX; ++i) gv[i] = i < n ? load1<GT>(Gd + tb + (int64_t)i * C + c) : 0.0f;
      for (int j = 0; j < n; ++j) {
        const float4* Wj = reinterpret_cast<const float4*>(s_W + j * NMAX);
        float acc = 0.0f;
#pragma unroll
        for (int i4 = 0; i4 < NMAX / 4; ++i4) {
          const float4 m = Wj[i4];
          acc = fmaf(m.x, gv[4 * i4], acc);
          acc = fmaf(m.y, gv[4 * i4 + 1], acc);
          acc = fmaf(m.z, gv[4 * i4 + 2], acc);
          acc = fmaf(m.w, gv[4 * i4 + 3], acc);
        }
        store1<XT>(DX + tb + (int64_t)j * C + c, acc);
      }
      if (DY) {
#pragma unroll
        for (int i = 0; i < NMAX; ++i)
          if (i < n) store1<YT>(DY + tb + (int64_t)i * C + c, s_par[nn + n + i] * gv[i]);
      }
    }
    for (int u = 0; u < tpi; ++u) {
      const int64_t t = t0 + (int64_t)u * gridDim.x;
      if (t >= A.T) break;
      const int64_t tb = t * n * C;
      if constexpr (MF) {
        const int q = lane >> 4, r = lane & 15;
        const int nbk = (n + 15) / 16;
#pragma unroll
        for (int b = 0; b < kMfBlk; ++b) {
          const int blk = wave + b * nwaves;
          if (blk >= nbk * nbk) break;
          const int I = blk / nbk, J = blk % nbk;
          const int gi = 16 * I + r, xj = 16 * J + r;
          const GT* grow = Gd + tb + (int64_t)(gi < n ? gi : 0) * C + 8 * q;
          const XT* xrow = X + tb + (int64_t)(xj < n ? xj : 0) * C + 8 * q;
          f32x4 acc = smb[b];
          for (int k = 0; k < C; k += 32) {
            const u32x4 zero = {0u, 0u, 0u, 0u};
            const u32x4 xb = xj < n ? *reinterpret_cast<const u32x4*>(xrow + k) : zero;
            if constexpr (std::is_same<GT, XT>::value) {
              const u32x4 ga = gi < n ? *reinterpret_cast<const u32x4*>(grow + k) : zero;
              acc = gen_mfma<XT>(ga, xb, acc);
            } else {
              float gv8[8];
              if (gi < n) {
                const float4 g0 = *reinterpret_cast<const float4*>(grow + k);
                const float4 g1 = *reinterpret_cast<const float4*>(grow + k + 4);
                gv8[0] = g0.x; gv8[1] = g0.y; gv8[2] = g0.z; gv8[3] = g0.w;
                gv8[4] = g1.x; gv8[5] = g1.y; gv8[6] = g1.z; gv8[7] = g1.w;
              } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) gv8[e] = 0.0f;
              }
              u32x4 ga[3];
              gen_split3x8<XT>(gv8, ga);
#pragma unroll
              for (int e = 2; e >= 0; --e) acc = gen_mfma<XT>(ga[e], xb, acc);
            }
          }
          smb[b] = acc;
        }
        // Yd_i = sum G_i Y_i: one wavefront per row, 8 channels per lane
        if (Y) {
          for (int i = wave; i < n; i += nwaves) {
            const GT* grow = Gd + tb + (int64_t)i * C;
            const YT* yrow = Y + tb + (int64_t)i * C;
            float acc = 0.0f;
            for (int c = 8 * lane; c < C; c += 512) {
              Vec<GT, 8> gv;
              Vec<YT, 8> yv;
              gv.load(grow + c);
              yv.load(yrow + c);
#pragma unroll
              for (int v = 0; v < 8; ++v) acc = fmaf(gv.get(v), yv.get(v), acc);
            }
            acc = wave_sum(acc);
            if (lane == 0) s_acc[i * NE + n] += acc;
          }
        }
        continue;
      }
      for (int blk = wave; blk < nbr * nbc; blk += nwaves) {
        const int r0 = (blk / nbc) * 4, c0 = (blk % nbc) * 4;
        float acc[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
        for (int c = lane; c < C; c += 64) {
          float rv[4], cv[4], yv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int ri = r0 + e, cj = c0 + e;
            rv[e] = ri < n ? load1<GT>(Gd + tb + (int64_t)ri * C + c) : 0.0f;
            cv[e] = cj < n ? load1<XT>(X + tb + (int64_t)cj * C + c) : 0.0f;
            yv[e] = (Y && c0 + 3 >= n && ri < n) ? load1<YT>(Y + tb + (int64_t)ri * C + c) : 0.0f;
          }
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int f = e & 3;
            const float col = (c0 + f == n) ? yv[e >> 2] : cv[f];
            acc[e] = fmaf(rv[e >> 2], col, acc[e]);
          }
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float v = wave_sum(acc[e]);
          const int i = r0 + (e >> 2), j = c0 + (e & 3);
          if (lane == 0 && i < n && j <= n) s_acc[i * NE + j] += v;
        }
      }

    }
  }
  if constexpr (MF) {
    const int q = lane >> 4, r = lane & 15;
    const int nbk = (n + 15) / 16;
#pragma unroll
    for (int b = 0; b < kMfBlk; ++b) {
      const int blk = wave + b * nwaves;
      if (blk >= nbk * nbk) break;
      const int I = blk / nbk, J = blk % nbk;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * I + 4 * q + e, j = 16 * J + r;
        if (i < n && j < n) s_acc[i * NE + j] = smb[b][e];
      }
    }
  }
  __syncthreads();
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  // [S n*n | Yd n], then zero padding
  for (int k = threadIdx.x; k < A.P; k += blockDim.x) {
    float v = 0.0f;
    if (k < nn) v = s_acc[(k / n) * NE + (k % n)];
    else if (k < K) v = s_acc[(k - nn) * NE + n];
    prow[k] = v;
  }
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
      if (A.n <= 32)
        hipLaunchKernelGGL((gen_fwd_kernel<XT, OT, 32>), dim3((unsigned)blocks), dim3(kGenThreads), 0, s, A);
      else
        hipLaunchKernelGGL((gen_fwd_kernel<XT, OT, 64>), dim3((unsigned)blocks), dim3(kGenThreads), 0, s, A);
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
      // pass 3 on MFMA: 16-bit x == dout, C a multiple of 32, 16-byte aligned rows
      bool mf = false;
      if constexpr (std::is_same<XT, GT>::value && sizeof(XT) == 2)
        mf = knob(kKnobGenMfma, 1) != 0 && A.C % 32 == 0 && aligned(A.x, 16) && aligned(A.g, 16);
      if (A.n <= 32) {
        if constexpr (std::is_same<XT, GT>::value && sizeof(XT) == 2) {
          if (mf) {
            hipLaunchKernelGGL((gen_bwd_kernel<XT, GT, 32, true>), dim3((unsigned)blocks), dim3(gen_bwd_threads(32)),
                               0, s, A);
            MHC_CHECK_LAUNCH("gen_bwd_kernel");
            return MHC_OK;
          }
        }
        hipLaunchKernelGGL((gen_bwd_kernel<XT, GT, 32>), dim3((unsigned)blocks), dim3(gen_bwd_threads(32)), 0, s,
                           A);
      } else {
        if constexpr (std::is_same<XT, GT>::value && sizeof(XT) == 2) {
          if (mf) {
            hipLaunchKernelGGL((gen_bwd_kernel<XT, GT, 64, true>), dim3((unsigned)blocks), dim3(gen_bwd_threads(64)),
                               0, s, A);
            MHC_CHECK_LAUNCH("gen_bwd_kernel");
            return MHC_OK;
          }
        }
        hipLaunchKernelGGL((gen_bwd_kernel<XT, GT, 64>), dim3((unsigned)blocks), dim3(gen_bwd_threads(64)), 0, s,
                           A);
      }
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
        if (A.n <= 32)
          hipLaunchKernelGGL((gen_mix_fwd_kernel<XT, YT, OT, 32>), dim3((unsigned)blocks), dim3(kGenThreads), 0,
                             s, A);
        else
          hipLaunchKernelGGL((gen_mix_fwd_kernel<XT, YT, OT, 64>), dim3((unsigned)blocks), dim3(kGenThreads), 0,
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
        if constexpr (sizeof(XT) == 2 && (std::is_same<GT, XT>::value || std::is_same<GT, float>::value)) {
          // the sums on MFMA: C a multiple of 32, 16-byte aligned rows (Y's 8-channel pieces too)
          if (knob(kKnobGenMfma, 1) != 0 && A.C % 32 == 0 && aligned(A.x, 16) && aligned(A.g, 16) &&
              (A.y == nullptr || aligned(A.y, 16))) {
            if (A.n <= 32)
              hipLaunchKernelGGL((gen_mix_bwd_kernel<XT, YT, GT, 32, true>), dim3((unsigned)blocks),
                                 dim3(kGenThreads), 0, s, A);
            else
              hipLaunchKernelGGL((gen_mix_bwd_kernel<XT, YT, GT, 64, true>), dim3((unsigned)blocks),
                                 dim3(kGenThreads), 0, s, A);
            MHC_CHECK_LAUNCH("gen_mix_bwd_kernel");
            return MHC_OK;
          }
        }
        if (A.n <= 32)
          hipLaunchKernelGGL((gen_mix_bwd_kernel<XT, YT, GT, 32>), dim3((unsigned)blocks), dim3(kGenThreads), 0,
                             s, A);
        else
          hipLaunchKernelGGL((gen_mix_bwd_kernel<XT, YT, GT, 64>), dim3((unsigned)blocks), dim3(kGenThreads), 0,
                             s, A);
        MHC_CHECK_LAUNCH("gen_mix_bwd_kernel");
        return MHC_OK;
      });
    });
  });
}

}  // namespace mhc
