// Fused mHC forward and backward for 16 < n <= 32 on MFMA (gfx950
// v_mfma_f32_16x16x32, bf16 / fp16: exact 16-bit products, fp32 sums).
//
// At n = 32 the stream mix is 1024 FMAs per channel, far more VALU issue
// time than the channel's HBM time, so every contraction over streams runs on
// the matrix cores with the fp32 parameters split into three 16-bit terms
// (split3: for bf16 they sum exactly to the fp32 value, so the MFMA forms the
// products of the fp32 parameters with the 16-bit data):
//   forward   y = a^T X,  out = M X + p (y inv w)
//   backward  y = a^T X,  dyn = p^T G,  dx = M^T G + a dy,  dM = G X^T
// n is padded to 32 with zero parameters; streams >= n are neither loaded
// nor stored.
//
// Lane layout (q = lane >> 4, r = lane & 15).  A wave owns 128-channel
// slabs; in a slab the lane loads streams 8q .. 8q+7 of channels
// [8r, 8r + 8) (eight 16-byte loads).  Transposed in registers, channel v of
// that range gives the B operand "streams 8q .. 8q+7 of column r", i.e. the K
// index of the MFMA runs over (q, element) = stream, and the columns are the
// 16 channels 8r + v of the 16 lanes r.  The A operand of lane (q, r) is row
// r of a 16-row block of the parameter matrix at the same streams, and D
// holds rows 4q .. 4q+3 of column r: out (or dx) of streams 16I + 4q + k at
// channel 8r + v.  Over v = 0..7 the lane so collects 8 contiguous channels
// of 8 output streams, stored as 16-byte rows.
//
// dM = G X^T contracts over channels instead: each wave stages its slab of x
// and g in LDS as one row per stream, and A (rows of g) and B (rows of x)
// are read back as 16-byte row pieces, 32 channels per MFMA.
#include "mhc_device.hpp"
#include "mhc_host.hpp"
#include "mhc_mfma32.hpp"
#include "mhc_plan.hpp"
#include "mhc_sinkhorn.hpp"

namespace mhc {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// D += A B for one 16 x 16 x 32 block; operands are eight 16-bit elements,
// element e of word m at half (e & 1) of word e >> 1.
template <typename T>
MHC_DEV f32x4 mfma32k(u32x4 a, u32x4 b, f32x4 c);
template <>
MHC_DEV f32x4 mfma32k<__bf16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
template <>
MHC_DEV f32x4 mfma32k<_Float16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                0, 0);
}

// split3 of eight values as three packed operands (term e of v[0..7]).
template <typename T>
MHC_DEV void split3x8(const float (&v)[8], u32x4 (&out)[3]) {
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

// Eight streams x eight channels (stream e in rows[e], channel v at element
// v) -> per channel v the operand "streams 0..7 of channel v".
template <typename T>
MHC_DEV void transpose8(const Vec<T, 8> (&rows)[8], u32x4 (&b)[8]) {
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    const int wd = v >> 1;
#pragma unroll
    for (int m = 0; m < 4; ++m)
      b[v][m] = (v & 1) ? pack_hi16<T>(rows[2 * m].w[wd], rows[2 * m + 1].w[wd])
                        : pack_lo16<T>(rows[2 * m].w[wd], rows[2 * m + 1].w[wd]);
  }
}

// One channel of eight stream rows: the operand "streams 0..7 of channel v".
template <typename T>
MHC_DEV u32x4 column8(const Vec<T, 8> (&rows)[8], int v) {
  const int wd = v >> 1;
  u32x4 b;
#pragma unroll
  for (int m = 0; m < 4; ++m)
    b[m] = (v & 1) ? pack_hi16<T>(rows[2 * m].w[wd], rows[2 * m + 1].w[wd])
                   : pack_lo16<T>(rows[2 * m].w[wd], rows[2 * m + 1].w[wd]);
  return b;
}

// D = sum_e A_e B over the three split terms, smallest first.
template <typename T>
MHC_DEV f32x4 mfma_split3(const u32x4 (&a)[3], u32x4 b, f32x4 acc) {
#pragma unroll
  for (int e = 2; e >= 0; --e) acc = mfma32k<T>(a[e], b, acc);
  return acc;
}

// Token rows through buffer resources: one lane offset serves every row and
// slab, the row and slab parts go in as uniform offsets.
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor word 3 (raw, 32-bit data)
constexpr int kBufNt = 2;               // buffer access cache policy: non-temporal

template <typename T>
MHC_DEV __amdgpu_buffer_rsrc_t rows_rsrc(const T* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), 0, (int)bytes, kRsrcWord3);
}

template <int AUX, typename T>
MHC_DEV void buf_load(Vec<T, 8>& v, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, AUX);
  v.w[0] = u.x; v.w[1] = u.y; v.w[2] = u.z; v.w[3] = u.w;
}

// v, passed through an empty asm the compiler cannot see through: offsets
// formed from the result are formed where they are used, instead of being
// hoisted out of the token loop and held in registers for all of it (with the
// row part in the lane offset, n < 64, that is one register per row).
MHC_DEV uint32_t opaque_u32(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Four output rows of eight channels, filled a channel pair (p = 0..3) at a
// time: 16-bit rows as packed words (one conversion per pair), fp32 rows as
// the values themselves; stored as 16-byte pieces.
template <typename OT>
struct OutRows {
  static constexpr bool kHalf = ElemTraits<OT>::kBytes == 2;
  uint32_t w[4][kHalf ? 4 : 8];
  MHC_DEV void put(int p, f32x4 even, f32x4 odd) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if constexpr (kHalf) {
        w[k][p] = pack2<OT>(even[k], odd[k]);
      } else {
        // through scalars: a bit_cast of an ext-vector element reads element 0
        const float e0 = even[k], e1 = odd[k];
        w[k][2 * p] = __builtin_bit_cast(uint32_t, e0);
        w[k][2 * p + 1] = __builtin_bit_cast(uint32_t, e1);
      }
    }
  }
  MHC_DEV void store(int k, OT* dst) const {
    uint32_t* d = reinterpret_cast<uint32_t*>(dst);
    if constexpr (kHalf) {
      st_nt(d, w[k][0], w[k][1], w[k][2], w[k][3]);
    } else {
      st16<false>(d, w[k][0], w[k][1], w[k][2], w[k][3]);
      st16<false>(d + 4, w[k][4], w[k][5], w[k][6], w[k][7]);
    }
  }
  // row k through a buffer resource (lane offset voff, uniform offset soff)
  MHC_DEV void store_buf(int k, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) const {
    if constexpr (kHalf) {
      buf_store_b128<kBufNt>(u32x4{w[k][0], w[k][1], w[k][2], w[k][3]}, rs, voff, soff);
    } else {
      buf_store_b128<0>(u32x4{w[k][0], w[k][1], w[k][2], w[k][3]}, rs, voff, soff);
      buf_store_b128<0>(u32x4{w[k][4], w[k][5], w[k][6], w[k][7]}, rs, voff, soff + 16);
    }
  }
};

template <bool RAW>
MHC_DEV float act_pre(float h) { return RAW ? sigmoid_fast(h) : h; }
template <bool RAW>
MHC_DEV float act_post(float h) { return RAW ? 2.0f * sigmoid_fast(h) : h; }

// Eight consecutive RMS weights.
MHC_DEV void load_w8(const float* p, float (&wv)[8]) {
  const float4 w0 = *reinterpret_cast<const float4*>(p);
  const float4 w1 = *reinterpret_cast<const float4*>(p + 4);
  wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
  wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
}

// The layer-wide projection inside a forward workgroup: wave 0 runs the
// block Sinkhorn (sk_fwd_blk, the arithmetic of mhc_sinkhorn_fwd's kernel
// for one matrix, so M is bitwise the same) into s_M ([n][n], LDS); after the
// barrier every wave reads its parameters from there, and workgroup 0 also
// writes M for the caller (kept for the backward).
MHC_DEV void mf32_project_into_lds(const Mf32Args& A, float* s_M, int n, int wave, int lane) {
  if (wave == 0) sk_fwd_blk<32, false>(A.hres, s_M, n, A.iters, A.eps, lane, nullptr);
  __syncthreads();
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < n * n; i += blockDim.x) A.M_out[i] = s_M[i];
}

// ---------------------------------------------------------------------------
// Forward.  One token at a time per workgroup of S / SPW waves (S = C / 128
// slabs); the grid strides over tokens, so layer-wide parameters are split
// once per workgroup.  Before the RMS barrier only y = a^T X runs; the mix
// runs after it, slab by slab, straight into the output rows.
// ---------------------------------------------------------------------------

// v[2 grp + k] for a lane-dependent grp in 0..3, as bit selects (a select
// chain on these values was turned into branches)
MHC_DEV float pick_pair(const float (&v)[8], int grp, int k) {
  const uint32_t m1 = 0u - (uint32_t)(grp & 1), m2 = 0u - (uint32_t)((grp >> 1) & 1);
  const uint32_t a = __builtin_bit_cast(uint32_t, v[k]), b = __builtin_bit_cast(uint32_t, v[2 + k]);
  const uint32_t c = __builtin_bit_cast(uint32_t, v[4 + k]), d = __builtin_bit_cast(uint32_t, v[6 + k]);
  const uint32_t lo = (a & ~m1) | (b & m1), hi = (c & ~m1) | (d & m1);
  return __builtin_bit_cast(float, (lo & ~m2) | (hi & m2));
}

// FULL: n == 32, so no stream index is ever out of range (no per-stream
// branches in the load, store and parameter code).
// RELOAD (C above 2048: SPW = C / 1024 slabs per wave): the transposed
// slabs do not stay in registers across the RMS barrier; the lane reads its
// x again for the mix (from the caches: the token was read just before).
// Of y only channels 8r + 2q, 8r + 2q + 1 stay with lane group q (the four
// groups hold the same values), gathered back after the barrier.
// SKF (layer-wide, raw logits): the Sinkhorn projection runs in the kernel
// (mf32_project_into_lds) instead of a launch of its own.
template <typename XT, typename OT, int SPW, bool PT, bool RAW, bool FULL, bool RELOAD = false, bool SKF = false>
__global__ __launch_bounds__(512) void mf32_fwd_kernel(Mf32Args A) {
  static_assert(!SKF || (!PT && RAW), "the in-kernel projection takes layer-wide raw logits");
  __shared__ float s_red[2][16];
  __shared__ float s_M[SKF ? 32 * 32 : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 32 : A.n;
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  int cb[SPW];
#pragma unroll
  for (int s = 0; s < SPW; ++s) cb[s] = (wave * SPW + s) * 128 + 8 * r;

  // a of streams 8q+e (the A operand of y), M rows 16I + r at streams 8q+e
  // (the A operands of the mix), p of the output rows 16I + 4q + k
  u32x4 aa[3], am[2][3];
  float pv[2][4];
  auto load_params = [&](int64_t t) {
    const float* M = SKF ? s_M : A.M + t * A.M_ts;
    const float* hp = A.hpre + t * A.h_ts;
    const float* hq = A.hpost + t * A.h_ts;
    float av[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) av[e] = 8 * q + e < n ? act_pre<RAW>(hp[8 * q + e]) : 0.0f;
    split3x8<XT>(av, aa);
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      const int row = 16 * I + r;
      float mv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) mv[e] = (row < n && 8 * q + e < n) ? M[row * n + 8 * q + e] : 0.0f;
      split3x8<XT>(mv, am[I]);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int o = 16 * I + 4 * q + k;
        pv[I][k] = o < n ? act_post<RAW>(hq[o]) : 0.0f;
      }
    }
  };
  if constexpr (SKF) mf32_project_into_lds(A, s_M, n, wave, lane);
  if constexpr (!PT) load_params(0);

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const XT* xt = (const XT*)A.x + t * nC;
    OT* ot = (OT*)A.out + t * nC;
    // one slab of x (streams 8q .. 8q+7), transposed into the B operands
    auto load_slab = [&](int s, u32x4 (&b)[8]) {
      Vec<XT, 8> xr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (8 * q + e < n) xr[e].load(xt + (int64_t)(8 * q + e) * C + cb[s]);
        else xr[e].zero();
      }
      transpose8<XT>(xr, b);
    };
    u32x4 bx[RELOAD ? 1 : SPW][8];
    float y[RELOAD ? 1 : SPW][8];
    // RELOAD: y of channels 8r + 2q, 8r + 2q + 1 kept by lane group q
    float yk[RELOAD ? SPW : 1][2];
    float ss = 0.0f;
    if constexpr (!RELOAD) {
      Vec<XT, 8> xr[SPW][8];
#pragma unroll
      for (int s = 0; s < SPW; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (8 * q + e < n) xr[s][e].load(xt + (int64_t)(8 * q + e) * C + cb[s]);
          else xr[s][e].zero();
        }
      if constexpr (PT) load_params(t);
#pragma unroll
      for (int s = 0; s < SPW; ++s) transpose8<XT>(xr[s], bx[s]);
    } else {
      if constexpr (PT) load_params(t);
    }
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      if constexpr (RELOAD) load_slab(s, bx[0]);
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const f32x4 acc = mfma_split3<XT>(aa, bx[RELOAD ? 0 : s][v], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        y[RELOAD ? 0 : s][v] = acc[0];
        ss = fmaf(acc[0], acc[0], ss);
      }
      if constexpr (RELOAD) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          yk[s][k] = pick_pair(y[0], q, k);
          // selected here, not at the uses after the barrier
          asm volatile("" : "+v"(yk[s][k]));
        }
      }
    }
    // the four lane groups q hold the same y: count it once
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
      // RELOAD: x of the slab read again; y of the lane's eight channels
      // gathered back from the four lane groups
      if constexpr (RELOAD) {
        load_slab(s, bx[0]);
#pragma unroll
        for (int v = 0; v < 8; ++v) y[0][v] = __shfl(yk[s][v & 1], 16 * (v >> 1) + r);
      }
      const float4 w0 = *reinterpret_cast<const float4*>(A.w + cb[s]);
      const float4 w1 = *reinterpret_cast<const float4*>(A.w + cb[s] + 4);
      const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      float yn[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) yn[v] = (y[RELOAD ? 0 : s][v] * inv) * wv[v];
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        // four output rows of this lane, converted a channel pair at a time
        OutRows<OT> rows;
        f32x4 even;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          f32x4 acc = mfma_split3<XT>(am[I], bx[RELOAD ? 0 : s][v], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
          for (int k = 0; k < 4; ++k) acc[k] = fmaf(yn[v], pv[I][k], acc[k]);
          if (v & 1) rows.put(v >> 1, even, acc);
          else even = acc;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int row = 16 * I + 4 * q + k;
          if (row < n) rows.store(k, ot + (int64_t)row * C + cb[s]);
        }
      }
    }
  }
}

// Largest C of the forward: the loop variant's y buffer (512 bytes per slab)
// stays within 64 KiB of LDS.
constexpr int kMf32FwdMaxC = 16384;

// Forward above C = 2048 (LOOP): W waves per workgroup walk SPW = S / W slabs
// each in a runtime loop, one slab in registers at a time, so the kernel
// needs the registers of the one-slab variant whatever C is and several
// workgroups share a CU.  Before the RMS barrier the lane loads its slab for
// y = a^T X and the token's sum of y^2, and lane group 0 writes the slab's y
// to LDS (512 bytes per slab); after it the lane loads the slab again (from
// the caches: the token was read just before) and reads its channels' y
// back for the mix.  Each wave reads back only the y it wrote itself.
template <typename XT, typename OT, bool PT, bool RAW, bool FULL, bool SKF = false>
__global__ __launch_bounds__(512) void mf32_fwd_loop_kernel(Mf32Args A, int spw) {
  static_assert(!SKF || (!PT && RAW), "the in-kernel projection takes layer-wide raw logits");
  extern __shared__ float4 s_y4[];  // [S][16 r][8 channels]
  float* const s_y = reinterpret_cast<float*>(s_y4);
  __shared__ float s_red[2][16];
  __shared__ float s_M[SKF ? 32 * 32 : 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 32 : A.n;
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  // token rows through buffer resources: a 32-bit lane offset for the lane's
  // first row, the row and slab parts as uniform offsets (n < 32: the row part
  // in the lane offset, so rows past n fall outside the resource, which reads
  // them as zero and drops their stores)
  constexpr uint32_t kEs = sizeof(XT), kOs = sizeof(OT);
  const uint32_t rowb = (uint32_t)C * kEs, orowb = (uint32_t)C * kOs;
  const uint32_t lane_in = (uint32_t)(8 * q * C + 8 * r) * kEs;   // stream 8q (+ e rows)
  const uint32_t lane_out = (uint32_t)(4 * q * C + 8 * r) * kOs;  // stream 4q (+ 16 I + k rows)
  const uint32_t tokb = (uint32_t)(nC * kEs), otokb = (uint32_t)(nC * kOs);

  u32x4 aa[3], am[2][3];
  float pv[2][4];
  auto load_params = [&](int64_t t) {
    const float* M = SKF ? s_M : A.M + t * A.M_ts;
    const float* hp = A.hpre + t * A.h_ts;
    const float* hq = A.hpost + t * A.h_ts;
    float av[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) av[e] = 8 * q + e < n ? act_pre<RAW>(hp[8 * q + e]) : 0.0f;
    split3x8<XT>(av, aa);
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      const int row = 16 * I + r;
      float mv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) mv[e] = (row < n && 8 * q + e < n) ? M[row * n + 8 * q + e] : 0.0f;
      split3x8<XT>(mv, am[I]);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int o = 16 * I + 4 * q + k;
        pv[I][k] = o < n ? act_post<RAW>(hq[o]) : 0.0f;
      }
    }
  };
  // layer-wide: the split operands (36 words per lane, the same for every
  // wave) are staged in LDS once and read back at each use, which keeps
  // the kernel at two 8-wave workgroups per CU
  __shared__ u32x4 s_aa[3][64], s_am[2][3][64];
  if constexpr (SKF) mf32_project_into_lds(A, s_M, n, wave, lane);
  if constexpr (!PT) {
    load_params(0);
    if (wave == 0) {
#pragma unroll
      for (int e = 0; e < 3; ++e) {
        s_aa[e][lane] = aa[e];
        s_am[0][e][lane] = am[0][e];
        s_am[1][e][lane] = am[1][e];
      }
    }
    __syncthreads();
  }

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const auto rx = rows_rsrc((const XT*)A.x + t * nC, tokb);
    const auto ro = rows_rsrc((OT*)A.out + t * nC, otokb);
    // streams 8q .. 8q+7 of the slab's channels 8r .. 8r+7, transposed into
    // the B operands (the first read cached, the second non-temporal)
    auto load_slab = [&](auto aux, int slab, u32x4 (&b)[8]) {
      const uint32_t sb = (uint32_t)slab * 128 * kEs;
      Vec<XT, 8> xr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        buf_load<decltype(aux)::value>(xr[e], rx, FULL ? lane_in : lane_in + (uint32_t)e * rowb,
                                       FULL ? sb + (uint32_t)e * rowb : sb);
      transpose8<XT>(xr, b);
    };
    if constexpr (PT) load_params(t);
    float ss = 0.0f;
    for (int s = 0; s < spw; ++s) {
      const int slab = wave * spw + s;
      u32x4 bx[8];
      load_slab(std::integral_constant<int, 0>{}, slab, bx);
      if constexpr (!PT) {
        asm volatile("" ::: "memory");  // read at each use, not held in registers across the loop
#pragma unroll
        for (int e = 0; e < 3; ++e) aa[e] = s_aa[e][lane];
      }
      float y[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const f32x4 acc = mfma_split3<XT>(aa, bx[v], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        y[v] = acc[0];
        ss = fmaf(acc[0], acc[0], ss);
      }
      // the four lane groups q hold the same y: group 0 keeps it
      if (q == 0) {
        float4* dst = reinterpret_cast<float4*>(s_y + (slab * 16 + r) * 8);
        dst[0] = make_float4(y[0], y[1], y[2], y[3]);
        dst[1] = make_float4(y[4], y[5], y[6], y[7]);
      }
    }
    ss = q == 0 ? ss : 0.0f;
    ss = wave_sum(ss);
    if (lane == 0) s_red[it & 1][wave] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int w = 0; w < nwaves; ++w) tot += s_red[it & 1][w];
    const float inv = 1.0f / sqrtf(tot / (float)C + A.eps);
    if (A.inv_rms != nullptr && tid == 0) A.inv_rms[t] = inv;
    for (int s = 0; s < spw; ++s) {
      const int slab = wave * spw + s;
      u32x4 bx[8];
      load_slab(std::integral_constant<int, kBufNt>{}, slab, bx);
      const float4* src = reinterpret_cast<const float4*>(s_y + (slab * 16 + r) * 8);
      const float4 y0 = src[0], y1 = src[1];
      const float y[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
      float wv[8];
      load_w8(A.w + slab * 128 + 8 * r, wv);
      float yn[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) yn[v] = (y[v] * inv) * wv[v];
      const uint32_t sob = (uint32_t)slab * 128 * kOs;
      if constexpr (!PT) asm volatile("" ::: "memory");
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        if constexpr (!PT) {
#pragma unroll
          for (int e = 0; e < 3; ++e) am[I][e] = s_am[I][e][lane];
        }
        OutRows<OT> rows;
        f32x4 even;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          f32x4 acc = mfma_split3<XT>(am[I], bx[v], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
          for (int k = 0; k < 4; ++k) acc[k] = fmaf(yn[v], pv[I][k], acc[k]);
          if (v & 1) rows.put(v >> 1, even, acc);
          else even = acc;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t ro_row = (uint32_t)(16 * I + k) * orowb;
          rows.store_buf(k, ro, FULL ? lane_out : lane_out + ro_row, FULL ? sob + ro_row : sob);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Forward for 32 < n <= 64, layer-wide or per-token parameters: the loop
// kernel above with the streams in two halves of 32.  Per slab the lane loads streams
// 32h + 8q .. 32h + 8q + 7 (h = 0, 1) of channels 8r .. 8r + 7 and
// transposes each half into B operands, so every contraction over streams
// is two chained MFMAs (K = 32 each): y = a^T X as before, and the mix in
// four 16-row blocks of M (rows 16I + r as the A operand, output rows
// 16I + 4q + k in D).  The split operands of a, M (two halves, four row
// blocks: 30 words of 16 bytes per lane) live in LDS and are read at each
// use.  Per-token parameters (PT): each lane splits the token's a into its
// own operands before the slab pass, and the workgroup splits the token's M
// (512 tasks of 8 values) and p into LDS buffers of the token's parity,
// read after the RMS barrier; a buffer is written again two tokens later,
// after every wave has passed the next token's barrier.  For n < 64 the row part of each stream's offset is in the lane
// offset, so rows past n read as zero and their stores are dropped.
// ---------------------------------------------------------------------------
template <typename XT, typename OT, bool RAW, bool FULL, bool PT>
__global__ __launch_bounds__(512) void mf64_fwd_loop_kernel(Mf32Args A, int spw) {
  extern __shared__ float4 s_y4[];  // [S][16 r][8 channels]
  float* const s_y = reinterpret_cast<float*>(s_y4);
  __shared__ float s_red[2][16];
  __shared__ u32x4 s_aa[PT ? 1 : 2][3][64], s_am[PT ? 2 : 1][4][2][3][64];
  __shared__ float s_pv[PT ? 2 : 1][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 64 : A.n;
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  constexpr uint32_t kEs = sizeof(XT), kOs = sizeof(OT);
  const uint32_t rowb = (uint32_t)C * kEs, orowb = (uint32_t)C * kOs;
  const uint32_t lane_in = (uint32_t)(8 * q * C + 8 * r) * kEs;   // stream 8q (+ 32 h + e rows)
  const uint32_t lane_out = (uint32_t)(4 * q * C + 8 * r) * kOs;  // stream 4q (+ 16 I + k rows)
  const uint32_t tokb = (uint32_t)(nC * kEs), otokb = (uint32_t)(nC * kOs);

  // split operands, written by wave 0 (one (h) or (I, h) block at a time)
  if (!PT && wave == 0) {
    u32x4 sp[3];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float av[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = 32 * h + 8 * q + e;
        av[e] = j < n ? act_pre<RAW>(A.hpre[j]) : 0.0f;
      }
      split3x8<XT>(av, sp);
#pragma unroll
      for (int e = 0; e < 3; ++e) s_aa[PT ? 0 : h][e][lane] = sp[e];
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const int row = 16 * I + r;
        float mv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = 32 * h + 8 * q + e;
          mv[e] = (row < n && j < n) ? A.M[row * n + j] : 0.0f;
        }
        split3x8<XT>(mv, sp);
#pragma unroll
        for (int e = 0; e < 3; ++e) s_am[0][I][h][e][lane] = sp[e];
      }
    }
    s_pv[0][lane] = lane < n ? act_post<RAW>(A.hpost[lane]) : 0.0f;
  }
  __syncthreads();

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const auto rx = rows_rsrc((const XT*)A.x + t * nC, tokb);
    const auto ro = rows_rsrc((OT*)A.out + t * nC, otokb);
    // half h of the slab: streams 32h + 8q .. + 7 of channels 8r .. 8r+7, transposed into B operands
    auto load_half = [&](auto aux, int slab, int h, u32x4 (&b)[8]) {
      const uint32_t sb = (uint32_t)slab * 128 * kEs;
      const uint32_t hb = (uint32_t)(32 * h) * rowb;
      Vec<XT, 8> xr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        buf_load<decltype(aux)::value>(xr[e], rx, FULL ? lane_in : lane_in + hb + (uint32_t)e * rowb,
                                       FULL ? sb + hb + (uint32_t)e * rowb : sb);
      transpose8<XT>(xr, b);
    };
    const int pb = PT ? (it & 1) : 0;
    u32x4 ta[2][3];  // PT: the token's a, split per lane
    if constexpr (PT) {
      const float* Mt = A.M + t * A.M_ts;
      const float* hp = A.hpre + t * A.h_ts;
      const float* hq = A.hpost + t * A.h_ts;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float av[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = 32 * h + 8 * q + e;
          av[e] = j < n ? act_pre<RAW>(hp[j]) : 0.0f;
        }
        split3x8<XT>(av, ta[h]);
      }
      for (int task = tid; task < 4 * 2 * 64; task += blockDim.x) {
        const int I = task >> 7, h = (task >> 6) & 1, l = task & 63;
        const int row = 16 * I + (l & 15), j0 = 32 * h + 8 * (l >> 4);
        float mv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) mv[e] = (row < n && j0 + e < n) ? Mt[row * n + j0 + e] : 0.0f;
        u32x4 sp[3];
        split3x8<XT>(mv, sp);
#pragma unroll
        for (int e = 0; e < 3; ++e) s_am[pb][I][h][e][l] = sp[e];
      }
      if (tid < 64) s_pv[pb][tid] = tid < n ? act_post<RAW>(hq[tid]) : 0.0f;
    }
    float ss = 0.0f;
    for (int s = 0; s < spw; ++s) {
      const int slab = wave * spw + s;
      u32x4 bx[2][8];
      load_half(std::integral_constant<int, 0>{}, slab, 0, bx[0]);
      load_half(std::integral_constant<int, 0>{}, slab, 1, bx[1]);
      asm volatile("" ::: "memory");  // split operands read at each use
      u32x4 aa[2][3];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 3; ++e) aa[h][e] = PT ? ta[h][e] : s_aa[PT ? 0 : h][e][lane];
      float y[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        f32x4 acc = mfma_split3<XT>(aa[0], bx[0][v], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        acc = mfma_split3<XT>(aa[1], bx[1][v], acc);
        y[v] = acc[0];
        ss = fmaf(acc[0], acc[0], ss);
      }
      if (q == 0) {
        float4* dst = reinterpret_cast<float4*>(s_y + (slab * 16 + r) * 8);
        dst[0] = make_float4(y[0], y[1], y[2], y[3]);
        dst[1] = make_float4(y[4], y[5], y[6], y[7]);
      }
    }
    ss = q == 0 ? ss : 0.0f;
    ss = wave_sum(ss);
    if (lane == 0) s_red[it & 1][wave] = ss;
    __syncthreads();
    float tot = 0.0f;
    for (int w = 0; w < nwaves; ++w) tot += s_red[it & 1][w];
    const float inv = 1.0f / sqrtf(tot / (float)C + A.eps);
    if (A.inv_rms != nullptr && tid == 0) A.inv_rms[t] = inv;
    for (int s = 0; s < spw; ++s) {
      const int slab = wave * spw + s;
      u32x4 bx[2][8];
      load_half(std::integral_constant<int, kBufNt>{}, slab, 0, bx[0]);
      load_half(std::integral_constant<int, kBufNt>{}, slab, 1, bx[1]);
      const float4* src = reinterpret_cast<const float4*>(s_y + (slab * 16 + r) * 8);
      const float4 y0 = src[0], y1 = src[1];
      const float y[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
      float wv[8];
      load_w8(A.w + slab * 128 + 8 * r, wv);
      float yn[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) yn[v] = (y[v] * inv) * wv[v];
      const uint32_t sob = (uint32_t)slab * 128 * kOs;
      asm volatile("" ::: "memory");
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        u32x4 am[2][3];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 3; ++e) am[h][e] = s_am[pb][I][h][e][lane];
        float pv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) pv[k] = s_pv[pb][16 * I + 4 * q + k];
        OutRows<OT> rows;
        f32x4 even;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          f32x4 acc = mfma_split3<XT>(am[0], bx[0][v], f32x4{0.0f, 0.0f, 0.0f, 0.0f});
          acc = mfma_split3<XT>(am[1], bx[1][v], acc);
#pragma unroll
          for (int k = 0; k < 4; ++k) acc[k] = fmaf(yn[v], pv[k], acc[k]);
          if (v & 1) rows.put(v >> 1, even, acc);
          else even = acc;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t ro_row = (uint32_t)(16 * I + k) * orowb;
          rows.store_buf(k, ro, FULL ? lane_out : lane_out + ro_row, FULL ? sob + ro_row : sob);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward, layer-wide parameters.  A persistent workgroup of C / 128 waves
// walks tokens t = b, b + G, ...; per token and slab:
//   before the RMS barrier: y = a^T X, dyn = p^T G (MFMA), the two per-token
//     sums, and dM += G X^T over the slab staged in LDS (MFMA);
//   after it: dy, yn and the dw contribution per channel; dx = M^T G + a dy
//     (MFMA, a dy as the accumulator input) stored as 16-byte rows; dA and
//     dP as lane partials from x and g read back from the staged slab.
// dM, dA, dP and dw stay in registers across the workgroup's tokens and end
// in its partial row, the waves' parts added in wave order.
// ---------------------------------------------------------------------------

constexpr int kMf32Row = 128 + 8;                 // LDS row: 16-bit elements (68 dwords, 4 mod 64 banks)
constexpr int kMf32Slab = 2 * 32 * kMf32Row;      // x rows then g rows
constexpr int kMf32MaxWaves = 8;                  // C <= 1024
constexpr int kMf32Par = 32 * 32 + 2 * 32;

// The backward's parameters, split once (by wave 0) into LDS: a, p of streams
// 8q+e (the A operands of y, dyn; per lane group q), column 16J + r of M at
// rows 8q+e (the A operand of M^T, per lane) and a of the dx rows
// 16J + 4q + k (per lane group q).
struct Mf32BwdPar {
  u32x4 amt[2][3][64];
  float4 a4[2][4];
  u32x4 aa[3][4], ap[3][4];
};

template <typename XT, bool RAW>
MHC_DEV void mf32_bwd_params(const float* __restrict__ M, const float* __restrict__ hpre,
                             const float* __restrict__ hpost, int n, Mf32BwdPar& P) {
  const int lane = threadIdx.x & 63;
  const int q = lane >> 4, r = lane & 15;
  if (r == 0) {
    float av[8], pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = 8 * q + e;
      av[e] = i < n ? act_pre<RAW>(hpre[i]) : 0.0f;
      pv[e] = i < n ? act_post<RAW>(hpost[i]) : 0.0f;
    }
    u32x4 aa[3], ap[3];
    split3x8<XT>(av, aa);
    split3x8<XT>(pv, ap);
#pragma unroll
    for (int e = 0; e < 3; ++e) {
      P.aa[e][q] = aa[e];
      P.ap[e][q] = ap[e];
    }
  }
#pragma unroll
  for (int J = 0; J < 2; ++J) {
    const int col = 16 * J + r;
    float mv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) mv[e] = (col < n && 8 * q + e < n) ? M[(8 * q + e) * n + col] : 0.0f;
    u32x4 amt[3];
    split3x8<XT>(mv, amt);
#pragma unroll
    for (int e = 0; e < 3; ++e) P.amt[J][e][lane] = amt[e];
    if (r == 0) {
      float a4[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = 16 * J + 4 * q + k;
        a4[k] = j < n ? act_pre<RAW>(hpre[j]) : 0.0f;
      }
      P.a4[J][q] = make_float4(a4[0], a4[1], a4[2], a4[3]);
    }
  }
}

// The workgroup's dM, dA and dP after its partial row's dw slice: dA and dP
// summed over the 16 lanes of a group, then every wave's part added in wave
// order through LDS (the staged slabs are no longer read by then).
MHC_DEV void mf32_bwd_param_sums(const Mf32Args& A, float* prow, uint16_t* lds, int n, const f32x4 (&dm)[2][2],
                                 float (&dA)[8], float (&dP)[8]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  // dA, dP: sums over the 16 lanes of a group, then the waves in order
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    dA[e] = group_sum<16>(dA[e]);
    dP[e] = group_sum<16>(dP[e]);
  }
  __syncthreads();  // every wave is done with its slab: reuse the LDS for the cross-wave sums
  float* s_fin = reinterpret_cast<float*>(lds);  // [wave][kMf32Par]
  float* mine = s_fin + wave * kMf32Par;
#pragma unroll
  for (int I = 0; I < 2; ++I)
#pragma unroll
    for (int J = 0; J < 2; ++J)
#pragma unroll
      for (int k = 0; k < 4; ++k) mine[(16 * I + 4 * q + k) * 32 + 16 * J + r] = dm[I][J][k];
  if (r == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      mine[1024 + 8 * q + e] = dA[e];
      mine[1024 + 32 + 8 * q + e] = dP[e];
    }
  }
  __syncthreads();
  const int nn = n * n;
  for (int k = tid; k < nn + 2 * n; k += blockDim.x) {
    int src;
    if (k < nn) src = (k / n) * 32 + (k % n);
    else if (k < nn + n) src = 1024 + (k - nn);
    else src = 1024 + 32 + (k - nn - n);
    float sum = 0.0f;
    for (int w = 0; w < nwaves; ++w) sum += s_fin[w * kMf32Par + src];
    prow[A.Cp + k] = sum;
  }
  if (tid == 0)
    for (int c = A.Cp + nn + 2 * n; c < A.P; ++c) prow[c] = 0.0f;
}

template <typename XT, bool RAW, bool FULL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void mf32_bwd_kernel(Mf32Args A) {
  extern __shared__ __align__(16) uint16_t mf32_lds[];
  __shared__ float s_red[2][2][kMf32MaxWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 32 : A.n;
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  uint16_t* xs = mf32_lds + (size_t)wave * kMf32Slab;
  uint16_t* gs = xs + 32 * kMf32Row;
  const int cb = wave * 128 + 8 * r;

  // parameters, split once by wave 0 into LDS and read per token (registers
  // are kept for the next token's loads)
  __shared__ Mf32BwdPar s_par;
  if (wave == 0) mf32_bwd_params<XT, RAW>(A.M, A.hpre, A.hpost, n, s_par);
  __syncthreads();
  float wv[8];
  {
    const float4 w0 = *reinterpret_cast<const float4*>(A.w + cb);
    const float4 w1 = *reinterpret_cast<const float4*>(A.w + cb + 4);
    wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
    wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
  }
  f32x4 dm[2][2];
#pragma unroll
  for (int I = 0; I < 2; ++I)
#pragma unroll
    for (int J = 0; J < 2; ++J) dm[I][J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float dA[8], dP[8], dwv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dA[e] = dP[e] = dwv[e] = 0.0f;

  // The token's x and g rows are loaded one token ahead: the next token's
  // loads are issued as soon as this token's registers are staged, so they
  // are in flight during the dM, barrier and dx phases and go out before this
  // token's dx stores (a wait for them then never waits for those stores).
  Vec<XT, 8> xr[8], gr[8];
  auto load_token = [&](int64_t t) {
    const XT* xt = (const XT*)A.x + t * nC;
    const XT* gt = (const XT*)A.g + t * nC;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (8 * q + e < n) {
        xr[e].load(xt + (int64_t)(8 * q + e) * C + cb);
        gr[e].load(gt + (int64_t)(8 * q + e) * C + cb);
      } else {
        xr[e].zero();
        gr[e].zero();
      }
    }
  };
  // (n < 32: loads at the top of each token instead; the per-stream
  // branches leave no registers for the next token's rows)
  if constexpr (FULL) {
    if ((int64_t)blockIdx.x < A.T) load_token(blockIdx.x);
    // the first token's loads are waited for before the loop: pending at the
    // loop entry (with no stores after them) they would make every token's
    // loop-top wait also wait for the previous token's dx stores
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
  }

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    float y[8], dyn[8];
    float ss = 0.0f, sr = 0.0f;
    if constexpr (!FULL) load_token(t);
    {
      // stage the slab (one LDS row per stream; zero rows for streams >= n)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        *reinterpret_cast<u32x4*>(&xs[(8 * q + e) * kMf32Row + 8 * r]) =
            u32x4{xr[e].w[0], xr[e].w[1], xr[e].w[2], xr[e].w[3]};
        *reinterpret_cast<u32x4*>(&gs[(8 * q + e) * kMf32Row + 8 * r]) =
            u32x4{gr[e].w[0], gr[e].w[1], gr[e].w[2], gr[e].w[3]};
      }
      const u32x4 aa[3] = {s_par.aa[0][q], s_par.aa[1][q], s_par.aa[2][q]};
      const u32x4 ap[3] = {s_par.ap[0][q], s_par.ap[1][q], s_par.ap[2][q]};
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const f32x4 ay = mfma_split3<XT>(aa, column8<XT>(xr, v), f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        const f32x4 ad = mfma_split3<XT>(ap, column8<XT>(gr, v), f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        y[v] = ay[0];
        dyn[v] = ad[0];
        ss = fmaf(ay[0], ay[0], ss);
        sr = fmaf(ad[0] * ay[0], wv[v], sr);
      }
      if constexpr (FULL) {
        if (t + gridDim.x < A.T) load_token(t + gridDim.x);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // dM over the slab: A = g rows 16I + r, B = x rows 16J + r, 32 channels per step
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4 ga[2], xb[2];
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        ga[I] = *reinterpret_cast<const u32x4*>(&gs[(16 * I + r) * kMf32Row + 32 * kk + 8 * q]);
        xb[I] = *reinterpret_cast<const u32x4*>(&xs[(16 * I + r) * kMf32Row + 32 * kk + 8 * q]);
      }
#pragma unroll
      for (int I = 0; I < 2; ++I)
#pragma unroll
        for (int J = 0; J < 2; ++J) dm[I][J] = mfma32k<XT>(ga[I], xb[J], dm[I][J]);
    }
    // the four lane groups q hold the same y and dyn: count them once
    ss = q == 0 ? ss : 0.0f;
    sr = q == 0 ? sr : 0.0f;
    ss = wave_sum(ss);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_red[it & 1][0][wave] = ss;
      s_red[it & 1][1][wave] = sr;
    }
    lds_barrier();
    float tss = 0.0f, tsr = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
      tss += s_red[it & 1][0][w];
      tsr += s_red[it & 1][1][w];
    }
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;

    float dyv[8], ynv[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float yi = y[v] * inv;
      dyv[v] = dyn[v] * inv * wv[v] - kf * y[v];
      ynv[v] = yi * wv[v];
      dwv[v] = fmaf(dyn[v], yi, dwv[v]);
    }
    XT* dxt = (XT*)A.out + t * nC;
    __builtin_amdgcn_sched_barrier(0);
    {
      // g back from the slab: dx = M^T g + a dy, and dP
      Vec<XT, 8> gr2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const u32x4 u = *reinterpret_cast<const u32x4*>(&gs[(8 * q + e) * kMf32Row + 8 * r]);
        gr2[e].w[0] = u[0]; gr2[e].w[1] = u[1]; gr2[e].w[2] = u[2]; gr2[e].w[3] = u[3];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int v = 0; v < 8; ++v) dP[e] = fmaf(gr2[e].get(v), ynv[v], dP[e]);
#pragma unroll
      for (int J = 0; J < 2; ++J) {
        // one 16-row half of dx at a time: the scheduler would otherwise overlap the halves'
        // operands and spill
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 amt[3] = {s_par.amt[J][0][lane], s_par.amt[J][1][lane], s_par.amt[J][2][lane]};
        const float4 a4 = s_par.a4[J][q];
        uint32_t ow[4][4];
        f32x4 even;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const u32x4 bg = column8<XT>(gr2, v);
          f32x4 acc = {a4.x * dyv[v], a4.y * dyv[v], a4.z * dyv[v], a4.w * dyv[v]};
          acc = mfma_split3<XT>(amt, bg, acc);
          if (v & 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) ow[k][v >> 1] = pack2<XT>(even[k], acc[k]);
          } else {
            even = acc;
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int j = 16 * J + 4 * q + k;
          if (j < n)
            st_nt(reinterpret_cast<uint32_t*>(dxt + (int64_t)j * C + cb), ow[k][0], ow[k][1], ow[k][2], ow[k][3]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    {
      // x back from the slab: dA
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Vec<XT, 8> xv;
        const u32x4 u = *reinterpret_cast<const u32x4*>(&xs[(8 * q + e) * kMf32Row + 8 * r]);
        xv.w[0] = u[0]; xv.w[1] = u[1]; xv.w[2] = u[2]; xv.w[3] = u[3];
#pragma unroll
        for (int v = 0; v < 8; ++v) dA[e] = fmaf(dyv[v], xv.get(v), dA[e]);
      }
    }
  }

  // ---- the workgroup's partial row [dw C | 0 .. Cp | dM n*n | dA n | dP n | 0 .. P]
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  // the channel base again from the thread index (opaque to the optimiser): kept from before the
  // token loop, it was the one value the loop spilled
  int tid2 = tid;
  asm volatile("" : "+v"(tid2));
  const int cb2 = (tid2 >> 6) * 128 + 8 * (tid2 & 15);
  if (q == 0) {
    *reinterpret_cast<float4*>(prow + cb2) = make_float4(dwv[0], dwv[1], dwv[2], dwv[3]);
    *reinterpret_cast<float4*>(prow + cb2 + 4) = make_float4(dwv[4], dwv[5], dwv[6], dwv[7]);
  }
  if (tid == 0)
    for (int c = C; c < A.Cp; ++c) prow[c] = 0.0f;
  mf32_bwd_param_sums(A, prow, mf32_lds, n, dm, dA, dP);
}

// ---------------------------------------------------------------------------
// Backward for 16 < n <= 32 with per-token parameters, 16-bit x == dout, C a
// multiple of 128 up to 1024: mf32_bwd_kernel's per-slab work (one slab per
// wave, staged in the wave's LDS slab buffer) with the token's own M, a, p:
//   - wave 0 splits the next token's parameters (as mf32_bwd_params does the
//     layer's) into one of two LDS blocks by token parity, after its dx pass;
//     the block's readers, two tokens back, are past this token's RMS
//     barrier by then, and the barrier after the parts below publishes it;
//   - after the dx pass each wave writes its dM, dA, dP over its slab into
//     its own slab buffer (free by then), a barrier, one thread per output
//     adds the waves' parts in wave order and writes the token's dM, dh_pre,
//     dh_post (with the activation chain), and a barrier before the next
//     token's slabs overwrite the parts.
// dw stays in registers across the workgroup's tokens and ends in its
// partial row.
// ---------------------------------------------------------------------------
template <typename XT, bool RAW, bool FULL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void mf32_bwd_pt_kernel(Mf32Args A) {
  extern __shared__ __align__(16) uint16_t mf32_lds[];
  __shared__ float s_red[2][2][kMf32MaxWaves];
  __shared__ Mf32BwdPar s_par[2];
  __shared__ float s_act[2][64];  // activated a [32], p [32] of the token, by parity
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 32 : A.n;
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  uint16_t* xs = mf32_lds + (size_t)wave * kMf32Slab;
  uint16_t* gs = xs + 32 * kMf32Row;
  const int cb = wave * 128 + 8 * r;

  auto params = [&](int64_t t, int par) {
    mf32_bwd_params<XT, RAW>(A.M + t * A.M_ts, A.hpre + t * A.h_ts, A.hpost + t * A.h_ts, n, s_par[par]);
    if (lane < 32) {
      s_act[par][lane] = lane < n ? act_pre<RAW>(A.hpre[t * A.h_ts + lane]) : 0.0f;
      s_act[par][32 + lane] = lane < n ? act_post<RAW>(A.hpost[t * A.h_ts + lane]) : 0.0f;
    }
  };
  if (wave == 0 && (int64_t)blockIdx.x < A.T) params(blockIdx.x, 0);
  __syncthreads();
  float wv[8];
  {
    const float4 w0 = *reinterpret_cast<const float4*>(A.w + cb);
    const float4 w1 = *reinterpret_cast<const float4*>(A.w + cb + 4);
    wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w;
    wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
  }
  float dwv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dwv[e] = 0.0f;

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const Mf32BwdPar& P = s_par[it & 1];
    const XT* xt = (const XT*)A.x + t * nC;
    const XT* gt = (const XT*)A.g + t * nC;
    // rows past n (n < 32) are loaded from row n - 1 and zeroed by a select: no per-row branch
    Vec<XT, 8> xr[8], gr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int row = FULL ? 8 * q + e : min(8 * q + e, n - 1);
      xr[e].load(xt + (int64_t)row * C + cb);
      gr[e].load(gt + (int64_t)row * C + cb);
    }
    if constexpr (!FULL) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool in = 8 * q + e < n;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          xr[e].w[m] = in ? xr[e].w[m] : 0u;
          gr[e].w[m] = in ? gr[e].w[m] : 0u;
        }
      }
    }
    f32x4 dm[2][2];
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int J = 0; J < 2; ++J) dm[I][J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    float dA[8], dP[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) dA[e] = dP[e] = 0.0f;
    float y[8], dyn[8];
    float ss = 0.0f, sr = 0.0f;
    {
      // stage the slab (one LDS row per stream; zero rows for streams >= n)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        *reinterpret_cast<u32x4*>(&xs[(8 * q + e) * kMf32Row + 8 * r]) =
            u32x4{xr[e].w[0], xr[e].w[1], xr[e].w[2], xr[e].w[3]};
        *reinterpret_cast<u32x4*>(&gs[(8 * q + e) * kMf32Row + 8 * r]) =
            u32x4{gr[e].w[0], gr[e].w[1], gr[e].w[2], gr[e].w[3]};
      }
      const u32x4 aa[3] = {P.aa[0][q], P.aa[1][q], P.aa[2][q]};
      const u32x4 ap[3] = {P.ap[0][q], P.ap[1][q], P.ap[2][q]};
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const f32x4 ay = mfma_split3<XT>(aa, column8<XT>(xr, v), f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        const f32x4 ad = mfma_split3<XT>(ap, column8<XT>(gr, v), f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        y[v] = ay[0];
        dyn[v] = ad[0];
        ss = fmaf(ay[0], ay[0], ss);
        sr = fmaf(ad[0] * ay[0], wv[v], sr);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // dM over the slab: A = g rows 16I + r, B = x rows 16J + r, 32 channels per step
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4 ga[2], xb[2];
#pragma unroll
      for (int I = 0; I < 2; ++I) {
        ga[I] = *reinterpret_cast<const u32x4*>(&gs[(16 * I + r) * kMf32Row + 32 * kk + 8 * q]);
        xb[I] = *reinterpret_cast<const u32x4*>(&xs[(16 * I + r) * kMf32Row + 32 * kk + 8 * q]);
      }
#pragma unroll
      for (int I = 0; I < 2; ++I)
#pragma unroll
        for (int J = 0; J < 2; ++J) dm[I][J] = mfma32k<XT>(ga[I], xb[J], dm[I][J]);
    }
    // the four lane groups q hold the same y and dyn: count them once
    ss = q == 0 ? ss : 0.0f;
    sr = q == 0 ? sr : 0.0f;
    ss = wave_sum(ss);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_red[it & 1][0][wave] = ss;
      s_red[it & 1][1][wave] = sr;
    }
    lds_barrier();
    float tss = 0.0f, tsr = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
      tss += s_red[it & 1][0][w];
      tsr += s_red[it & 1][1][w];
    }
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;

    float dyv[8], ynv[8];
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const float yi = y[v] * inv;
      dyv[v] = dyn[v] * inv * wv[v] - kf * y[v];
      ynv[v] = yi * wv[v];
      dwv[v] = fmaf(dyn[v], yi, dwv[v]);
    }
    // dx rows through a buffer resource spanning the token's n rows: the range check drops the stores of
    // rows past n (a per-row branch around the stores made the compiler spill)
    const auto rdx = rows_rsrc((XT*)A.out + t * nC, (uint32_t)(nC * (int64_t)sizeof(XT)));
    __builtin_amdgcn_sched_barrier(0);
    {
      // g back from the slab: dx = M^T g + a dy, and dP
      Vec<XT, 8> gr2[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const u32x4 u = *reinterpret_cast<const u32x4*>(&gs[(8 * q + e) * kMf32Row + 8 * r]);
        gr2[e].w[0] = u[0]; gr2[e].w[1] = u[1]; gr2[e].w[2] = u[2]; gr2[e].w[3] = u[3];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int v = 0; v < 8; ++v) dP[e] = fmaf(gr2[e].get(v), ynv[v], dP[e]);
#pragma unroll
      for (int J = 0; J < 2; ++J) {
        __builtin_amdgcn_sched_barrier(0);
        const u32x4 amt[3] = {P.amt[J][0][lane], P.amt[J][1][lane], P.amt[J][2][lane]};
        const float4 a4 = P.a4[J][q];
        uint32_t ow[4][4];
        f32x4 even;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const u32x4 bg = column8<XT>(gr2, v);
          f32x4 acc = {a4.x * dyv[v], a4.y * dyv[v], a4.z * dyv[v], a4.w * dyv[v]};
          acc = mfma_split3<XT>(amt, bg, acc);
          if (v & 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) ow[k][v >> 1] = pack2<XT>(even[k], acc[k]);
          } else {
            even = acc;
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t vo = (uint32_t)((16 * J + 4 * q + k) * C + cb) * (uint32_t)sizeof(XT);
          buf_store_b128<kBufNt>(u32x4{ow[k][0], ow[k][1], ow[k][2], ow[k][3]}, rdx, vo, 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    {
      // x back from the slab: dA
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Vec<XT, 8> xv;
        const u32x4 u = *reinterpret_cast<const u32x4*>(&xs[(8 * q + e) * kMf32Row + 8 * r]);
        xv.w[0] = u[0]; xv.w[1] = u[1]; xv.w[2] = u[2]; xv.w[3] = u[3];
#pragma unroll
        for (int v = 0; v < 8; ++v) dA[e] = fmaf(dyv[v], xv.get(v), dA[e]);
      }
    }
    // this wave's part of the token's dM, dA, dP into its own slab buffer (its reads of the slab above
    // come first in the wave's program order)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dA[e] = group_sum<16>(dA[e]);
      dP[e] = group_sum<16>(dP[e]);
    }
    float* mine = reinterpret_cast<float*>(xs);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int J = 0; J < 2; ++J)
#pragma unroll
        for (int k = 0; k < 4; ++k) mine[(16 * I + 4 * q + k) * 32 + 16 * J + r] = dm[I][J][k];
    if (r == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        mine[1024 + 8 * q + e] = dA[e];
        mine[1024 + 32 + 8 * q + e] = dP[e];
      }
    }
    // the next token's parameters (wave 0, into the other parity block), once the token's own sums are
    // out of its registers
    if (wave == 0 && t + gridDim.x < A.T) params(t + gridDim.x, (it + 1) & 1);
    lds_barrier();
    const int nn = n * n;
    for (int k = tid; k < nn + 2 * n; k += blockDim.x) {
      int src;
      if (k < nn) src = (k / n) * 32 + (k % n);
      else if (k < nn + n) src = 1024 + (k - nn);
      else src = 1024 + 32 + (k - nn - n);
      float sum = 0.0f;
      for (int w = 0; w < nwaves; ++w) sum += reinterpret_cast<const float*>(mf32_lds + (size_t)w * kMf32Slab)[src];
      if (k < nn) {
        A.dM_tok[t * nn + k] = sum;
      } else if (k < nn + n) {
        const int j = k - nn;
        if constexpr (RAW) {
          const float av = s_act[it & 1][j];
          sum *= av * (1.0f - av);
        }
        A.dpre_tok[t * n + j] = sum;
      } else {
        const int i = k - nn - n;
        if constexpr (RAW) {
          const float pv = s_act[it & 1][32 + i];
          sum *= pv * (1.0f - 0.5f * pv);
        }
        A.dpost_tok[t * n + i] = sum;
      }
    }
    lds_barrier();  // the parts are read before the next token's slabs are staged over them
  }

  // ---- the workgroup's partial row [dw C | 0 .. Cp]
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  if (q == 0) {
    *reinterpret_cast<float4*>(prow + cb) = make_float4(dwv[0], dwv[1], dwv[2], dwv[3]);
    *reinterpret_cast<float4*>(prow + cb + 4) = make_float4(dwv[4], dwv[5], dwv[6], dwv[7]);
  }
  if (tid == 0)
    for (int c = C; c < A.Cp; ++c) prow[c] = 0.0f;
}

// ---------------------------------------------------------------------------
// Backward for 32 < n <= 64, layer-wide parameters, 16-bit x == dout, C a
// multiple of 128 up to 8192.  A persistent workgroup of W waves walks
// tokens; each wave takes SPW slabs of 128 channels.  With
// dy = dyn inv w - kf y and yn = y inv w (inv and kf the token's RMS
// scalars), dA_i = sum dy x_i = inv sum x_i dyn w - kf sum x_i y and
// dP_i = sum g_i yn = inv sum g_i y w: every parameter sum can be formed
// before the token's RMS sums are known, so only dx needs the token after
// the barrier.  Per token:
//   Before the barrier, per slab and 32-channel chunk, x and g rows in the
//     A-operand layout (rows 16 I + r, channels 32 k + 8 q .. + 7, one
//     16-byte piece per lane and 16-row block): y = a^T X and dyn = p^T G
//     per channel (the lane's four rows, then a sum over the 16 lanes r);
//     the slab's part of dM = G X^T on MFMA (four 16-row blocks of G as A
//     operands, four of X as B operands, each used by four MFMAs); the lane
//     partials of sum x_i dyn w, sum x_i y and sum g_i y w; the token sums
//     sum y^2 and sum dyn y w; y and dyn to LDS.  G of the wave's last slab
//     is also read in the B-operand layout (two 32-stream halves,
//     transposed) and kept in registers (GL: see below).
//   RMS barrier.
//   After it: dA, dP partials += the token's partials times inv and kf;
//     per slab (the last first), dy per channel and the dw term (the
//     workgroup's dw is in LDS), then dx = M^T G + a dy on MFMA in four
//     16-row blocks, stored as 16-byte rows; slabs other than the last read
//     G again.
// With one slab per wave and at least two waves (GL), G does not go through
// HBM twice: the row pieces are also written to the wave's LDS channel-major
// (16 KB), where the B operands are 16-byte reads after the barrier; the
// M^T operands are then split per lane at each use (their 24 KB of LDS
// would leave one workgroup per CU).
//   The dM blocks (in registers) and the dA, dP partials are the wave's over
//   its slabs and every token; they are added in wave order at the end.
// Every LDS value a wave reads after the RMS barrier is one it wrote itself,
// so the RMS barrier is the token's only one.  Every sum has one owner and a
// fixed order.  Row offsets go in the lane offset (at n = 64 too: uniform
// row offsets are loop-invariant, and held in SGPRs across the token loop
// they spill), so rows past n (n < 64) read as zero and their stores are
// dropped by the buffer range check.
// ---------------------------------------------------------------------------
constexpr int kMf64BwdMaxC = 8192;  // y, dyn and dw of a token in LDS: 96 KB

template <typename XT, bool RAW, bool FULL, bool GL, int NB>
__global__ __launch_bounds__(512) void mf64_bwd_kernel(Mf32Args A, int spw) {
  constexpr int NH = NB / 2;  // 32-stream halves
  // [S][16 r][8] y, then dyn; dw [C]; with GL (one slab per wave) then each wave's G, [128 channels][64 streams]
  extern __shared__ float4 s_yd4[];
  float* const s_y = reinterpret_cast<float*>(s_yd4);
  __shared__ float s_red[2][2][16];
  __shared__ u32x4 s_amt[GL ? 1 : 4][2][3][64];
  __shared__ float s_a[64], s_p[64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 64 : A.n;
  const int C = A.C;
  const int S = C / 128;
  float* const s_d = s_y + S * 128;
  float* const s_dw = s_d + S * 128;  // the workgroup's dw, one owner lane per channel
  uint16_t* const s_g0 = reinterpret_cast<uint16_t*>(s_dw + C);
  uint16_t* const s_g = s_g0 + (size_t)wave * 128 * 64;  // GL: the wave's G, channel-major
  const int64_t nC = (int64_t)n * C;
  constexpr uint32_t kEs = sizeof(XT);
  const uint32_t rowb = (uint32_t)C * kEs;
  const uint32_t lane_in = (uint32_t)(8 * q * C + 8 * r) * kEs;   // stream 8q (+ 32 h + e rows)
  const uint32_t lane_out = (uint32_t)(4 * q * C + 8 * r) * kEs;  // stream 4q (+ 16 J + k rows)
  const uint32_t tokb = (uint32_t)(nC * kEs);
  float* prow = A.part + (int64_t)blockIdx.x * A.P;

  // parameters: M^T split once by wave 0 into A operands (GL: per lane at each use); a and p
  if (wave == 0) {
    u32x4 sp[3];
#pragma unroll
    for (int h = 0; h < (GL ? 0 : NH); ++h) {
#pragma unroll
      for (int J = 0; J < NB; ++J) {
        const int j = 16 * J + r;
        float mv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 32 * h + 8 * q + e;
          mv[e] = (i < n && j < n) ? A.M[i * n + j] : 0.0f;
        }
        split3x8<XT>(mv, sp);
#pragma unroll
        for (int e = 0; e < 3; ++e) s_amt[GL ? 0 : J][h][e][lane] = sp[e];
      }
    }
    s_a[lane] = lane < n ? act_pre<RAW>(A.hpre[lane]) : 0.0f;
    s_p[lane] = lane < n ? act_post<RAW>(A.hpost[lane]) : 0.0f;
  }
  for (int c = tid; c < C; c += blockDim.x) s_dw[c] = 0.0f;
  __syncthreads();

  // phase C sums of the wave's slabs over every token: dM blocks [I][J] (rows 16 I + 4 q + k, column
  // 16 J + r), dA of streams 16 J + r and dP of streams 16 I + r over the lane's channels
  f32x4 dmb[NB][NB];
  float dAp[NB], dPp[NB];
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    dAp[I] = dPp[I] = 0.0f;
#pragma unroll
    for (int J = 0; J < NB; ++J) dmb[I][J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const uint32_t lane_c = (uint32_t)(r * C + 8 * q) * kEs;  // stream r (+ 16 I rows), channel 8q of a chunk
  float a_r[NB], p_r[NB];  // a and p of the lane's rows 16 I + r
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    a_r[I] = s_a[16 * I + r];
    p_r[I] = s_p[16 * I + r];
  }

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const XT* xt = (const XT*)A.x + t * nC;
    const XT* gt = (const XT*)A.g + t * nC;
    const auto rx = rows_rsrc(xt, tokb);
    const auto rg = rows_rsrc(gt, tokb);
    const auto rdx = rows_rsrc((XT*)A.out + t * nC, tokb);
    auto load_half = [&](auto aux, const __amdgpu_buffer_rsrc_t& rs, int slab, int h, u32x4 (&b)[8]) {
      const uint32_t sb = (uint32_t)slab * 128 * kEs;
      const uint32_t hb = (uint32_t)(32 * h) * rowb;
      const uint32_t li = opaque_u32(lane_in);
      Vec<XT, 8> xr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        buf_load<decltype(aux)::value>(xr[e], rs, li + hb + (uint32_t)e * rowb, sb);
      transpose8<XT>(xr, b);
    };
    // ---- before the RMS barrier, per slab and 32-channel chunk: x and g rows 16 I + r at channels
    // 32 k + 8 q .. + 7 (A-operand layout); y = a^T X and dyn = p^T G per channel (the lane's four rows,
    // then a sum over the 16 lanes r); the slab's part of dM = G X^T on MFMA (four 16-row blocks of G as
    // A operands, four of X as B operands, each used by four MFMAs); the lane partials of
    // sum x_i dyn w, sum x_i y and sum g_i y w.  G of the wave's last slab is also read in the B-operand
    // layout (two 32-stream halves, transposed) and kept for the dx pass.
    float ss = 0.0f, sr = 0.0f;
    float ua[NB], va[NB], wa[NB];
#pragma unroll
    for (int I = 0; I < NB; ++I) ua[I] = va[I] = wa[I] = 0.0f;
    u32x4 bg[NH][8];
    for (int s = 0; s < spw; ++s) {
      const int slab = wave * spw + s;
      const uint32_t sob = (uint32_t)slab * 128 * kEs;
      if (!GL && s == spw - 1) {
#pragma unroll
        for (int h = 0; h < NH; ++h) load_half(std::integral_constant<int, 0>{}, rg, slab, h, bg[h]);
      }
#pragma unroll 1  // unrolled, the chunks' rows and sums spill
      for (int k = 0; k < 4; ++k) {
        const uint32_t cb = sob + (uint32_t)(32 * k) * kEs;
        const uint32_t lc = opaque_u32(lane_c);
        Vec<XT, 8> ga[NB], xb[NB];
#pragma unroll
        for (int I = 0; I < NB; ++I) {
          const uint32_t row = (uint32_t)(16 * I) * rowb;
          buf_load<0>(xb[I], rx, lc + row, cb);
          buf_load<0>(ga[I], rg, lc + row, cb);
        }
        float wc[8];
        load_w8(A.w + slab * 128 + 32 * k + 8 * q, wc);
        float yc[8], dc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float ys = 0.0f, ds = 0.0f;
#pragma unroll
          for (int I = 0; I < NB; ++I) {
            ys = fmaf(a_r[I], xb[I].get(e), ys);
            ds = fmaf(p_r[I], ga[I].get(e), ds);
          }
          yc[e] = strided_sum<1, 16>(ys);
          dc[e] = strided_sum<1, 16>(ds);
        }
#pragma unroll
        for (int I = 0; I < NB; ++I) {
          const u32x4 a = {ga[I].w[0], ga[I].w[1], ga[I].w[2], ga[I].w[3]};
#pragma unroll
          for (int J = 0; J < NB; ++J) {
            const u32x4 b = {xb[J].w[0], xb[J].w[1], xb[J].w[2], xb[J].w[3]};
            dmb[I][J] = mfma32k<XT>(a, b, dmb[I][J]);
          }
        }
        if constexpr (GL) {
          // G to the wave's LDS, channel-major: element e of the piece is channel 32 k + 8 q + e of
          // stream 16 I + r (the B-operand reads after the barrier take 8 streams of a channel at once)
#pragma unroll
          for (int I = 0; I < NB; ++I)
#pragma unroll
            for (int e = 0; e < 8; ++e)
              s_g[(32 * k + 8 * q + e) * 64 + 16 * I + r] = (uint16_t)(ga[I].w[e >> 1] >> (16 * (e & 1)));
        }
        // the rows are converted again below rather than kept as 64 floats
#pragma unroll
        for (int I = 0; I < NB; ++I)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            xb[I].w[e] = opaque_u32(xb[I].w[e]);
            ga[I].w[e] = opaque_u32(ga[I].w[e]);
          }
        float dw8[8], yw8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dw8[e] = dc[e] * wc[e];
          yw8[e] = yc[e] * wc[e];
          // the 16 lanes r hold the same y and dyn: lane r = 0 counts them
          ss = fmaf(yc[e], yc[e], ss);
          sr = fmaf(dw8[e], yc[e], sr);
        }
#pragma unroll
        for (int I = 0; I < NB; ++I) {
          float su = 0.0f, sv = 0.0f, sw = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float xe = xb[I].get(e);
            su = fmaf(dw8[e], xe, su);
            sv = fmaf(yc[e], xe, sv);
            sw = fmaf(yw8[e], ga[I].get(e), sw);
          }
          ua[I] += su;
          va[I] += sv;
          wa[I] += sw;
        }
        if (r == 0) {
          float4* y4 = reinterpret_cast<float4*>(s_y + slab * 128 + 32 * k + 8 * q);
          float4* d4 = reinterpret_cast<float4*>(s_d + slab * 128 + 32 * k + 8 * q);
          y4[0] = make_float4(yc[0], yc[1], yc[2], yc[3]);
          y4[1] = make_float4(yc[4], yc[5], yc[6], yc[7]);
          d4[0] = make_float4(dc[0], dc[1], dc[2], dc[3]);
          d4[1] = make_float4(dc[4], dc[5], dc[6], dc[7]);
        }
      }
    }
    ss = r == 0 ? ss : 0.0f;
    sr = r == 0 ? sr : 0.0f;
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
    // dy = dyn inv w - kf y and yn = y inv w: dA_i = inv sum x_i dyn w - kf sum x_i y, dP_i = inv sum g_i y w
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      dAp[I] += inv * ua[I] - kf * va[I];
      dPp[I] += inv * wa[I];
    }
    // ---- after it, per slab (the last first: its G is in registers): dy and dw, then
    // dx = M^T G + a dy on MFMA in four 16-row blocks, stored as 16-byte rows
    for (int s = spw - 1; s >= 0; --s) {
      const int slab = wave * spw + s;
      const float* yp = s_y + (slab * 16 + r) * 8;
      const float* dp = s_d + (slab * 16 + r) * 8;
      const float4 y0 = reinterpret_cast<const float4*>(yp)[0], y1 = reinterpret_cast<const float4*>(yp)[1];
      const float4 d0 = reinterpret_cast<const float4*>(dp)[0], d1 = reinterpret_cast<const float4*>(dp)[1];
      const float y[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
      const float dyn[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
      float wv[8];
      load_w8(A.w + slab * 128 + 8 * r, wv);
      float dy[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) dy[v] = dyn[v] * inv * wv[v] - kf * y[v];
      if (q == 0) {
        float* pw = s_dw + slab * 128 + 8 * r;
#pragma unroll
        for (int v = 0; v < 8; ++v) pw[v] = fmaf(dyn[v], y[v] * inv, pw[v]);
      }
      if constexpr (GL) {
        // streams 32 h + 8 q .. + 7 of channel 8 r + v: the B operands, from the wave's LDS
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
          for (int v = 0; v < 8; ++v)
            bg[h][v] = *reinterpret_cast<const u32x4*>(s_g + (8 * r + v) * 64 + 32 * h + 8 * q);
      } else if (s != spw - 1) {
#pragma unroll
        for (int h = 0; h < NH; ++h) load_half(std::integral_constant<int, kBufNt>{}, rg, slab, h, bg[h]);
        asm volatile("" ::: "memory");
      }
      const uint32_t sob = (uint32_t)slab * 128 * kEs;
#pragma unroll 1
      for (int J = 0; J < NB; ++J) {
        u32x4 amt[NH][3];
        if constexpr (GL) {
#pragma unroll
          for (int h = 0; h < NH; ++h) {
            const int j = 16 * J + r;
            float mv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int i = 32 * h + 8 * q + e;
              mv[e] = (i < n && j < n) ? A.M[i * n + j] : 0.0f;
            }
            split3x8<XT>(mv, amt[h]);
          }
        } else {
#pragma unroll
          for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int e = 0; e < 3; ++e) amt[h][e] = s_amt[J][h][e][lane];
        }
        float a4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) a4[k] = s_a[16 * J + 4 * q + k];
        OutRows<XT> rows;
        f32x4 even;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          f32x4 acc = {a4[0] * dy[v], a4[1] * dy[v], a4[2] * dy[v], a4[3] * dy[v]};
#pragma unroll
          for (int h = 0; h < NH; ++h) acc = mfma_split3<XT>(amt[h], bg[h][v], acc);
          if (v & 1) rows.put(v >> 1, even, acc);
          else even = acc;
        }
        const uint32_t lo = opaque_u32(lane_out);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t row = (uint32_t)(16 * J + k) * rowb;
          rows.store_buf(k, rdx, lo + row, sob);
        }
      }
    }
  }

  // ---- partial row: [dw C | 0 .. Cp | dM n*n | dA n | dP n | 0 .. P].  The waves' sums are added in
  // wave order in LDS (in the parameter operands' space, free once every wave is past its last token).
#pragma unroll
  for (int I = 0; I < NB; ++I) {
    dAp[I] += shfl_xor(dAp[I], 16);
    dAp[I] += shfl_xor(dAp[I], 32);
    dPp[I] += shfl_xor(dPp[I], 16);
    dPp[I] += shfl_xor(dPp[I], 32);
  }
  __syncthreads();
  // dM [64][64], dA [64], dP [64]: in the parameter operands' space, or (GL) the waves' G buffers
  float* const s_acc = GL ? reinterpret_cast<float*>(s_g0) : reinterpret_cast<float*>(&s_amt[0][0][0][0]);
  static_assert(GL || sizeof(s_amt) >= (64 * 64 + 128) * sizeof(float), "LDS for the wave-order sums");
  for (int w = 0; w < nwaves; ++w) {
    if (wave == w) {
#pragma unroll
      for (int I = 0; I < NB; ++I)
#pragma unroll
        for (int J = 0; J < NB; ++J)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            float* d = s_acc + (16 * I + 4 * q + k) * 64 + 16 * J + r;
            *d = w == 0 ? dmb[I][J][k] : *d + dmb[I][J][k];
          }
      if (q == 0) {
#pragma unroll
        for (int I = 0; I < NB; ++I) {
          float* da = s_acc + 4096 + 16 * I + r;
          float* dp = s_acc + 4096 + 64 + 16 * I + r;
          *da = w == 0 ? dAp[I] : *da + dAp[I];
          *dp = w == 0 ? dPp[I] : *dp + dPp[I];
        }
      }
    }
    __syncthreads();
  }
  for (int c = tid; c < A.Cp; c += blockDim.x) prow[c] = c < C ? s_dw[c] : 0.0f;
  for (int e = tid; e < A.P - A.Cp; e += blockDim.x) {
    float v = 0.0f;
    if (e < n * n) v = s_acc[(e / n) * 64 + e % n];
    else if (e < n * n + 2 * n) v = s_acc[4096 + (e < n * n + n ? e - n * n : 64 + e - n * n - n)];
    prow[A.Cp + e] = v;
  }
}

// ---------------------------------------------------------------------------
// Backward for 16 < n <= 64 with per-token parameters, 16-bit x == dout, C a
// multiple of 128 up to 4096; NB 16-row blocks of streams (4, or 2 for
// n <= 32).  Each wave takes whole tokens (the wave's
// global index, then steps of the total wave count), so a token's RMS sums
// and its dM, dh_pre and dh_post are the wave's own: no barrier and no sum
// across waves per token.  Per token: a and p of the lane's rows 16 I + r;
// per slab and 32-channel chunk the pass of the layer-wide kernel before its
// barrier (x and g rows in the A-operand layout, y and dyn on the VALU with a
// sum over the 16 lanes r, dM = G X^T on MFMA, the lane partials of
// sum x_i dyn w, sum x_i y and sum g_i y w, y and dyn to the wave's LDS);
// the RMS scalars from two wave sums; the token's dM (the wave's 64
// accumulator registers), dh_pre and dh_post (lane partials summed over the
// lane groups q, with the activation chain) written out; then per slab, dy
// and the wave's dw term (its dw is in its LDS), g read in the B-operand
// layout and dx = M^T G + a dy on MFMA, the token's M^T split per lane for
// each 16-row block.  At the end the waves' dw are added in wave order into
// the workgroup's partial row [dw C | 0 .. Cp].
// ---------------------------------------------------------------------------
constexpr int kMf64BwdPtMaxC = 4096;  // y, dyn, dw, a and p of a token per wave in LDS: 48.5 KB

template <typename XT, bool RAW, bool FULL, int NB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void mf64_bwd_pt_kernel(Mf32Args A) {
  constexpr int NH = NB / 2;  // 32-stream halves
  extern __shared__ float s_pt[];  // per wave [y C][dyn C][dw C][a 64][p 64]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 64 : A.n;
  const int C = A.C;
  const int S = C / 128;
  float* const s_y = s_pt + (size_t)wave * (3 * C + 128);
  float* const s_d = s_y + C;
  float* const s_dw = s_d + C;
  float* const s_ap = s_dw + C;  // the token's a and p
  const int64_t nC = (int64_t)n * C;
  constexpr uint32_t kEs = sizeof(XT);
  const uint32_t rowb = (uint32_t)C * kEs;
  const uint32_t lane_in = (uint32_t)(8 * q * C + 8 * r) * kEs;   // stream 8q (+ 32 h + e rows)
  const uint32_t lane_out = (uint32_t)(4 * q * C + 8 * r) * kEs;  // stream 4q (+ 16 J + k rows)
  const uint32_t lane_c = (uint32_t)(r * C + 8 * q) * kEs;      // stream r (+ 16 I rows), channel 8q of a chunk
  const uint32_t tokb = (uint32_t)(nC * kEs);
  for (int c = lane; c < C; c += 64) s_dw[c] = 0.0f;

  const int64_t nw = (int64_t)gridDim.x * nwaves;
  for (int64_t t = (int64_t)blockIdx.x * nwaves + wave; t < A.T; t += nw) {
    const float* Mt = A.M + t * A.M_ts;
    const float* hp = A.hpre + t * A.h_ts;
    const float* hq = A.hpost + t * A.h_ts;
    s_ap[lane] = lane < n ? act_pre<RAW>(hp[lane]) : 0.0f;
    s_ap[64 + lane] = lane < n ? act_post<RAW>(hq[lane]) : 0.0f;
    const auto rx = rows_rsrc((const XT*)A.x + t * nC, tokb);
    const auto rg = rows_rsrc((const XT*)A.g + t * nC, tokb);
    const auto rdx = rows_rsrc((XT*)A.out + t * nC, tokb);
    f32x4 dmb[NB][NB];
    float ua[NB], va[NB], wa[NB];
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      ua[I] = va[I] = wa[I] = 0.0f;
#pragma unroll
      for (int J = 0; J < NB; ++J) dmb[I][J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    float ss = 0.0f, sr = 0.0f;
    for (int slab = 0; slab < S; ++slab) {
      const uint32_t sob = (uint32_t)slab * 128 * kEs;
#pragma unroll 1  // unrolled, the chunks' rows and sums spill
      for (int k = 0; k < 4; ++k) {
        const uint32_t cb = sob + (uint32_t)(32 * k) * kEs;
        const uint32_t lc = opaque_u32(lane_c);
        Vec<XT, 8> ga[NB], xb[NB];
#pragma unroll
        for (int I = 0; I < NB; ++I) {
          const uint32_t row = (uint32_t)(16 * I) * rowb;
          buf_load<0>(xb[I], rx, lc + row, cb);
          buf_load<0>(ga[I], rg, lc + row, cb);
        }
        float wc[8];
        load_w8(A.w + slab * 128 + 32 * k + 8 * q, wc);
        float a_r[NB], p_r[NB];  // a and p of the lane's rows 16 I + r
#pragma unroll
        for (int I = 0; I < NB; ++I) {
          a_r[I] = s_ap[16 * I + r];
          p_r[I] = s_ap[64 + 16 * I + r];
        }
        float yc[8], dc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float ys = 0.0f, ds = 0.0f;
#pragma unroll
          for (int I = 0; I < NB; ++I) {
            ys = fmaf(a_r[I], xb[I].get(e), ys);
            ds = fmaf(p_r[I], ga[I].get(e), ds);
          }
          yc[e] = strided_sum<1, 16>(ys);
          dc[e] = strided_sum<1, 16>(ds);
        }
#pragma unroll
        for (int I = 0; I < NB; ++I) {
          const u32x4 a = {ga[I].w[0], ga[I].w[1], ga[I].w[2], ga[I].w[3]};
#pragma unroll
          for (int J = 0; J < NB; ++J) {
            const u32x4 b = {xb[J].w[0], xb[J].w[1], xb[J].w[2], xb[J].w[3]};
            dmb[I][J] = mfma32k<XT>(a, b, dmb[I][J]);
          }
        }
        // the rows are converted again below rather than kept as 64 floats
#pragma unroll
        for (int I = 0; I < NB; ++I)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            xb[I].w[e] = opaque_u32(xb[I].w[e]);
            ga[I].w[e] = opaque_u32(ga[I].w[e]);
          }
        float dw8[8], yw8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dw8[e] = dc[e] * wc[e];
          yw8[e] = yc[e] * wc[e];
          // the 16 lanes r hold the same y and dyn: lane r = 0 counts them
          ss = fmaf(yc[e], yc[e], ss);
          sr = fmaf(dw8[e], yc[e], sr);
        }
#pragma unroll
        for (int I = 0; I < NB; ++I) {
          float su = 0.0f, sv = 0.0f, sw = 0.0f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float xe = xb[I].get(e);
            su = fmaf(dw8[e], xe, su);
            sv = fmaf(yc[e], xe, sv);
            sw = fmaf(yw8[e], ga[I].get(e), sw);
          }
          ua[I] += su;
          va[I] += sv;
          wa[I] += sw;
        }
        if (r == 0) {
          float4* y4 = reinterpret_cast<float4*>(s_y + slab * 128 + 32 * k + 8 * q);
          float4* d4 = reinterpret_cast<float4*>(s_d + slab * 128 + 32 * k + 8 * q);
          y4[0] = make_float4(yc[0], yc[1], yc[2], yc[3]);
          y4[1] = make_float4(yc[4], yc[5], yc[6], yc[7]);
          d4[0] = make_float4(dc[0], dc[1], dc[2], dc[3]);
          d4[1] = make_float4(dc[4], dc[5], dc[6], dc[7]);
        }
      }
    }
    ss = wave_sum(r == 0 ? ss : 0.0f);
    sr = wave_sum(r == 0 ? sr : 0.0f);
    const float inv = 1.0f / sqrtf(ss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * sr;
    // the token's dh_pre and dh_post (dA_i = inv sum x_i dyn w - kf sum x_i y, dP_i = inv sum g_i y w) and dM
#pragma unroll
    for (int I = 0; I < NB; ++I) {
      float da = inv * ua[I] - kf * va[I], dp = inv * wa[I];
      da += shfl_xor(da, 16);
      da += shfl_xor(da, 32);
      dp += shfl_xor(dp, 16);
      dp += shfl_xor(dp, 32);
      const int i = 16 * I + r;
      if (q == 0 && i < n) {
        if constexpr (RAW) {
          const float av = s_ap[i], pv = s_ap[64 + i];
          da *= av * (1.0f - av);
          dp *= pv * (1.0f - 0.5f * pv);
        }
        A.dpre_tok[t * n + i] = da;
        A.dpost_tok[t * n + i] = dp;
      }
    }
    // dM through a buffer resource of the token's n * n values: entries past n get an offset beyond it
    // (dropped by the range check) rather than a branch each
    const auto rdm = rows_rsrc(A.dM_tok + t * (int64_t)n * n, (uint32_t)(n * n * sizeof(float)));
#pragma unroll
    for (int I = 0; I < NB; ++I)
#pragma unroll
      for (int J = 0; J < NB; ++J)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int row = 16 * I + 4 * q + k, col = 16 * J + r;
          const uint32_t off = (row < n && col < n) ? (uint32_t)(row * n + col) * 4u : 0x80000000u;
          // the element as a scalar first: __builtin_bit_cast of a vector element compiled to a cast of
          // the vector's first element
          const float v = dmb[I][J][k];
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rdm, off, 0, 0);
        }
    // dx = M^T G + a dy per slab, in four 16-row blocks
    for (int slab = 0; slab < S; ++slab) {
      const float* yp = s_y + (slab * 16 + r) * 8;
      const float* dp = s_d + (slab * 16 + r) * 8;
      const float4 y0 = reinterpret_cast<const float4*>(yp)[0], y1 = reinterpret_cast<const float4*>(yp)[1];
      const float4 d0 = reinterpret_cast<const float4*>(dp)[0], d1 = reinterpret_cast<const float4*>(dp)[1];
      const float y[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
      const float dyn[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
      float wv[8];
      load_w8(A.w + slab * 128 + 8 * r, wv);
      float dy[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) dy[v] = dyn[v] * inv * wv[v] - kf * y[v];
      if (q == 0) {
        float* pw = s_dw + slab * 128 + 8 * r;
#pragma unroll
        for (int v = 0; v < 8; ++v) pw[v] = fmaf(dyn[v], y[v] * inv, pw[v]);
      }
      // streams 32h + 8q .. + 7 of channels 8r .. 8r + 7, transposed into B operands
      u32x4 bg[NH][8];
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const uint32_t li = opaque_u32(lane_in);
        Vec<XT, 8> xr[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          buf_load<kBufNt>(xr[e], rg, li + (uint32_t)(32 * h + e) * rowb, (uint32_t)slab * 128 * kEs);
        transpose8<XT>(xr, bg[h]);
      }
      const uint32_t sob = (uint32_t)slab * 128 * kEs;
#pragma unroll 1
      for (int J = 0; J < NB; ++J) {
        u32x4 amt[NH][3];
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const int j = 16 * J + r;
          float mv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int i = 32 * h + 8 * q + e;
            mv[e] = (i < n && j < n) ? Mt[i * n + j] : 0.0f;
          }
          split3x8<XT>(mv, amt[h]);
        }
        float a4[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) a4[k] = s_ap[16 * J + 4 * q + k];
        OutRows<XT> rows;
        f32x4 even;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          f32x4 acc = {a4[0] * dy[v], a4[1] * dy[v], a4[2] * dy[v], a4[3] * dy[v]};
#pragma unroll
          for (int h = 0; h < NH; ++h) acc = mfma_split3<XT>(amt[h], bg[h][v], acc);
          if (v & 1) rows.put(v >> 1, even, acc);
          else even = acc;
        }
        const uint32_t lo = opaque_u32(lane_out);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t row = (uint32_t)(16 * J + k) * rowb;
          rows.store_buf(k, rdx, lo + row, sob);
        }
      }
    }
  }

  // ---- the workgroup's partial row [dw C | 0 .. Cp]: the waves' dw in wave order
  __syncthreads();
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  for (int c = tid; c < A.Cp; c += blockDim.x) {
    float v = 0.0f;
    if (c < C)
      for (int w = 0; w < nwaves; ++w) v += s_pt[(size_t)w * (3 * C + 128) + 2 * C + c];
    prow[c] = v;
  }
}

// ---------------------------------------------------------------------------
// Backward for 16 < n <= 32 above C = 1024 (layer-wide): SPW slabs per wave,
// up to 8 waves.  A token's slabs do not fit in registers across the
// RMS barrier, so the work splits around it:
//   before: per slab, y and dyn (MFMA), the two per-token sums and
//     dM += G X^T over the slab staged in LDS;
//   after: per slab, last first, x and g are read again (from the caches:
//     the token was just read, and those first reads leave it cached) for
//     dx = M^T G + a dy (MFMA), dA and dP.
// Of y and dyn only the pair of channels 8r + 2q, 8r + 2q + 1 stays with
// lane group q across the barrier (the four groups hold the same values);
// the lane's eight are gathered back from the groups afterwards.  dw of those
// two channels is kept by the same group.
// n < 32 (!FULL): a row's offset goes in the lane offset, which the buffer
// range check covers, so rows beyond n load as zero and their stores are
// dropped (the resource spans the token's n rows); at n = 32 the row part is
// a uniform offset.
// ---------------------------------------------------------------------------
template <typename XT, bool RAW, int SPW, bool FULL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void mf32_bwd_wide_kernel(Mf32Args A) {
  extern __shared__ __align__(16) uint16_t mf32_lds[];
  __shared__ float s_red[2][2][kMf32MaxWaves];
  __shared__ Mf32BwdPar s_par;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 32 : A.n;
  constexpr uint32_t kEs = sizeof(XT);
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  uint16_t* xs = mf32_lds + (size_t)wave * kMf32Slab;
  uint16_t* gs = xs + 32 * kMf32Row;
  const int slab0 = wave * SPW * 128;
  const uint32_t rowb = (uint32_t)C * kEs;                      // one stream row
  const uint32_t slabb = (uint32_t)slab0 * kEs;                 // the wave's first slab
  const uint32_t lane_in = (uint32_t)(8 * q * C + 8 * r) * kEs;  // stream 8q (+ e rows)
  const uint32_t lane_dx = (uint32_t)(4 * q * C + 8 * r) * kEs;  // stream 4q (+ 16 J + k rows)
  const uint32_t tokb = (uint32_t)(nC * kEs);

  if (wave == 0) mf32_bwd_params<XT, RAW>(A.M, A.hpre, A.hpost, n, s_par);
  __syncthreads();
  f32x4 dm[2][2];
#pragma unroll
  for (int I = 0; I < 2; ++I)
#pragma unroll
    for (int J = 0; J < 2; ++J) dm[I][J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float dA[8], dP[8], dwv[SPW][2];
#pragma unroll
  for (int e = 0; e < 8; ++e) dA[e] = dP[e] = 0.0f;
#pragma unroll
  for (int s = 0; s < SPW; ++s) dwv[s][0] = dwv[s][1] = 0.0f;

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    const auto rx = rows_rsrc((const XT*)A.x + t * nC, tokb);
    const auto rg = rows_rsrc((const XT*)A.g + t * nC, tokb);
    float yk[SPW][2], dk[SPW][2];
    float ss = 0.0f, sr = 0.0f;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t sb = slabb + (uint32_t)s * 128 * kEs;
      Vec<XT, 8> xr[8], gr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        buf_load<0>(xr[e], rx, FULL ? lane_in : lane_in + (uint32_t)e * rowb, FULL ? sb + (uint32_t)e * rowb : sb);
        buf_load<0>(gr[e], rg, FULL ? lane_in : lane_in + (uint32_t)e * rowb, FULL ? sb + (uint32_t)e * rowb : sb);
      }
      float wv[8];
      load_w8(A.w + slab0 + s * 128 + 8 * r, wv);
      // stage the slab for dM (the previous slab's reads of the buffer were
      // issued first, and one wave's LDS accesses complete in order)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        *reinterpret_cast<u32x4*>(&xs[(8 * q + e) * kMf32Row + 8 * r]) =
            u32x4{xr[e].w[0], xr[e].w[1], xr[e].w[2], xr[e].w[3]};
        *reinterpret_cast<u32x4*>(&gs[(8 * q + e) * kMf32Row + 8 * r]) =
            u32x4{gr[e].w[0], gr[e].w[1], gr[e].w[2], gr[e].w[3]};
      }
      const u32x4 aa[3] = {s_par.aa[0][q], s_par.aa[1][q], s_par.aa[2][q]};
      const u32x4 ap[3] = {s_par.ap[0][q], s_par.ap[1][q], s_par.ap[2][q]};
      float y[8], dyn[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const f32x4 ay = mfma_split3<XT>(aa, column8<XT>(xr, v), f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        const f32x4 ad = mfma_split3<XT>(ap, column8<XT>(gr, v), f32x4{0.0f, 0.0f, 0.0f, 0.0f});
        y[v] = ay[0];
        dyn[v] = ad[0];
        ss = fmaf(ay[0], ay[0], ss);
        sr = fmaf(ad[0] * ay[0], wv[v], sr);
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        yk[s][k] = pick_pair(y, q, k);
        dk[s][k] = pick_pair(dyn, q, k);
        // selected here, not at the uses after the barrier (sunk there, the
        // selects would keep all eight values of every slab live across it)
        asm volatile("" : "+v"(yk[s][k]), "+v"(dk[s][k]));
      }
      // dM over the slab: A = g rows 16I + r, B = x rows 16J + r, 32 channels per step
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        u32x4 ga[2], xb[2];
#pragma unroll
        for (int I = 0; I < 2; ++I) {
          ga[I] = *reinterpret_cast<const u32x4*>(&gs[(16 * I + r) * kMf32Row + 32 * kk + 8 * q]);
          xb[I] = *reinterpret_cast<const u32x4*>(&xs[(16 * I + r) * kMf32Row + 32 * kk + 8 * q]);
        }
#pragma unroll
        for (int I = 0; I < 2; ++I)
#pragma unroll
          for (int J = 0; J < 2; ++J) dm[I][J] = mfma32k<XT>(ga[I], xb[J], dm[I][J]);
      }
    }
    // the four lane groups q hold the same y and dyn: count them once
    ss = q == 0 ? ss : 0.0f;
    sr = q == 0 ? sr : 0.0f;
    ss = wave_sum(ss);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_red[it & 1][0][wave] = ss;
      s_red[it & 1][1][wave] = sr;
    }
    lds_barrier();
    float tss = 0.0f, tsr = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
      tss += s_red[it & 1][0][w];
      tsr += s_red[it & 1][1][w];
    }
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;

    const auto rdx = rows_rsrc((const XT*)A.out + t * nC, tokb);
#pragma unroll
    for (int s = SPW - 1; s >= 0; --s) {
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t sb = slabb + (uint32_t)s * 128 * kEs;
      Vec<XT, 8> gr[8], xr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) buf_load<kBufNt>(gr[e], rg, FULL ? lane_in : lane_in + (uint32_t)e * rowb, FULL ? sb + (uint32_t)e * rowb : sb);
#pragma unroll
      for (int e = 0; e < 8; ++e) buf_load<kBufNt>(xr[e], rx, FULL ? lane_in : lane_in + (uint32_t)e * rowb, FULL ? sb + (uint32_t)e * rowb : sb);
      float wv[8];
      load_w8(A.w + slab0 + s * 128 + 8 * r, wv);
      // y and dyn of the lane's 8 channels back from the four lane groups
      float dyv[8], ynv[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int src = 16 * (v >> 1) + r;
        const float yv = __shfl(yk[s][v & 1], src);
        const float dn = __shfl(dk[s][v & 1], src);
        dyv[v] = dn * inv * wv[v] - kf * yv;
        ynv[v] = (yv * inv) * wv[v];
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) dwv[s][k] = fmaf(dk[s][k], yk[s][k] * inv, dwv[s][k]);
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int v = 0; v < 8; ++v) dP[e] = fmaf(gr[e].get(v), ynv[v], dP[e]);
#pragma unroll
      for (int J = 0; J < 2; ++J) {
        const u32x4 amt[3] = {s_par.amt[J][0][lane], s_par.amt[J][1][lane], s_par.amt[J][2][lane]};
        const float4 a4 = s_par.a4[J][q];
        uint32_t ow[4][4];
        f32x4 even;
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          const u32x4 bg = column8<XT>(gr, v);
          f32x4 acc = {a4.x * dyv[v], a4.y * dyv[v], a4.z * dyv[v], a4.w * dyv[v]};
          acc = mfma_split3<XT>(amt, bg, acc);
          if (v & 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) ow[k][v >> 1] = pack2<XT>(even[k], acc[k]);
          } else {
            even = acc;
          }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
          buf_store_b128<kBufNt>(u32x4{ow[k][0], ow[k][1], ow[k][2], ow[k][3]}, rdx,
                                 FULL ? lane_dx : lane_dx + (uint32_t)(16 * J + k) * rowb,
                                 FULL ? sb + (uint32_t)(16 * J + k) * rowb : sb);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int v = 0; v < 8; ++v) dA[e] = fmaf(dyv[v], xr[e].get(v), dA[e]);
    }
  }

  // ---- the workgroup's partial row [dw C | 0 .. Cp | dM n*n | dA n | dP n | 0 .. P]
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
#pragma unroll
  for (int s = 0; s < SPW; ++s)
    *reinterpret_cast<float2*>(prow + slab0 + s * 128 + 8 * r + 2 * q) = make_float2(dwv[s][0], dwv[s][1]);
  if (tid == 0)
    for (int c = C; c < A.Cp; ++c) prow[c] = 0.0f;
  mf32_bwd_param_sums(A, prow, mf32_lds, n, dm, dA, dP);
}

// ---------------------------------------------------------------------------
// The same backward with each slab step's x and g loaded one step ahead (the
// default; MHC_BWD_PIPE=0 selects the kernel above).  A step stages its x and
// g registers in the wave's LDS slab buffer, issues the next step's loads
// into the freed registers and computes from the staged copy, so a slab's
// loads are in flight during the previous slab's MFMAs.  Steps per token:
// before the RMS barrier slabs 0 .. SPW-1; after it SPW-1 (still staged from
// the last step before the barrier, so not read again), then SPW-2 .. 0.
// The last step loads the next token's first slab, before its dx stores.
// ---------------------------------------------------------------------------
template <typename XT, bool RAW, int SPW, bool FULL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void mf32_bwd_pipe_kernel(Mf32Args A) {
  extern __shared__ __align__(16) uint16_t mf32_lds[];
  __shared__ float s_red[2][2][kMf32MaxWaves];
  __shared__ Mf32BwdPar s_par;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = blockDim.x >> 6;
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 32 : A.n;
  constexpr uint32_t kEs = sizeof(XT);
  const int C = A.C;
  const int64_t nC = (int64_t)n * C;
  uint16_t* xs = mf32_lds + (size_t)wave * kMf32Slab;
  uint16_t* gs = xs + 32 * kMf32Row;
  const int slab0 = wave * SPW * 128;
  const uint32_t rowb = (uint32_t)C * kEs;                      // one stream row
  const uint32_t slabb = (uint32_t)slab0 * kEs;                 // the wave's first slab
  const uint32_t lane_in = (uint32_t)(8 * q * C + 8 * r) * kEs;  // stream 8q (+ e rows)
  const uint32_t lane_dx = (uint32_t)(4 * q * C + 8 * r) * kEs;  // stream 4q (+ 16 J + k rows)
  const uint32_t tokb = (uint32_t)(nC * kEs);

  if (wave == 0) mf32_bwd_params<XT, RAW>(A.M, A.hpre, A.hpost, n, s_par);
  __syncthreads();
  f32x4 dm[2][2];
#pragma unroll
  for (int I = 0; I < 2; ++I)
#pragma unroll
    for (int J = 0; J < 2; ++J) dm[I][J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float dA[8], dP[8], dwv[SPW][2];
#pragma unroll
  for (int e = 0; e < 8; ++e) dA[e] = dP[e] = 0.0f;
#pragma unroll
  for (int s = 0; s < SPW; ++s) dwv[s][0] = dwv[s][1] = 0.0f;

  // the step's x and g rows (streams 8q + e, channels 8r .. 8r + 7 of a slab)
  Vec<XT, 8> xr[8], gr[8];
  using Cached = std::integral_constant<int, 0>;
  using Stream = std::integral_constant<int, kBufNt>;
  auto load = [&](auto aux, int64_t t, int s) {
    const auto rx = rows_rsrc((const XT*)A.x + t * nC, tokb);
    const auto rg = rows_rsrc((const XT*)A.g + t * nC, tokb);
    const uint32_t sb = slabb + (uint32_t)s * 128 * kEs;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      buf_load<decltype(aux)::value>(xr[e], rx, FULL ? lane_in : lane_in + (uint32_t)e * rowb, FULL ? sb + (uint32_t)e * rowb : sb);
      buf_load<decltype(aux)::value>(gr[e], rg, FULL ? lane_in : lane_in + (uint32_t)e * rowb, FULL ? sb + (uint32_t)e * rowb : sb);
    }
  };
  // one LDS row per stream (the previous step's reads of the buffer were
  // issued first, and one wave's LDS accesses complete in order)
  auto stage = [&]() {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      *reinterpret_cast<u32x4*>(&xs[(8 * q + e) * kMf32Row + 8 * r]) =
          u32x4{xr[e].w[0], xr[e].w[1], xr[e].w[2], xr[e].w[3]};
      *reinterpret_cast<u32x4*>(&gs[(8 * q + e) * kMf32Row + 8 * r]) =
          u32x4{gr[e].w[0], gr[e].w[1], gr[e].w[2], gr[e].w[3]};
    }
  };
  // the lane's own rows back from the staged slab
  auto rows_back = [&](const uint16_t* buf, Vec<XT, 8>(&rows)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const u32x4 u = *reinterpret_cast<const u32x4*>(&buf[(8 * q + e) * kMf32Row + 8 * r]);
      rows[e].w[0] = u[0]; rows[e].w[1] = u[1]; rows[e].w[2] = u[2]; rows[e].w[3] = u[3];
    }
  };

  load(Cached{}, blockIdx.x, 0);
  // the first token's loads are waited for before the loop: pending at the
  // loop entry they would make every token's first wait also wait for the
  // previous token's dx stores
  __builtin_amdgcn_s_waitcnt(kWaitVm0);

  int it = 0;
  for (int64_t t = blockIdx.x; t < A.T; t += gridDim.x, ++it) {
    float yk[SPW][2], dk[SPW][2];
    float ss = 0.0f, sr = 0.0f;
    float wlast[8];  // w of slab SPW - 1, used again right after the barrier
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      __builtin_amdgcn_sched_barrier(0);
      // w first: a wait for a load also waits for every load issued before it
      float wv[8];
      load_w8(A.w + slab0 + s * 128 + 8 * r, wv);
      if (s == SPW - 1) {
#pragma unroll
        for (int v = 0; v < 8; ++v) wlast[v] = wv[v];
      }
      stage();
      // next: slab s + 1; after the last slab, the second step after the barrier (SPW - 2)
      if (s + 1 < SPW) load(Cached{}, t, s + 1);
      else load(Stream{}, t, SPW - 2);
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      __builtin_amdgcn_wave_barrier();
      float y[8], dyn[8];
      {
        Vec<XT, 8> rows[8];
        rows_back(xs, rows);
        const u32x4 aa[3] = {s_par.aa[0][q], s_par.aa[1][q], s_par.aa[2][q]};
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          y[v] = mfma_split3<XT>(aa, column8<XT>(rows, v), f32x4{0.0f, 0.0f, 0.0f, 0.0f})[0];
          ss = fmaf(y[v], y[v], ss);
        }
      }
      {
        Vec<XT, 8> rows[8];
        rows_back(gs, rows);
        const u32x4 ap[3] = {s_par.ap[0][q], s_par.ap[1][q], s_par.ap[2][q]};
#pragma unroll
        for (int v = 0; v < 8; ++v) {
          dyn[v] = mfma_split3<XT>(ap, column8<XT>(rows, v), f32x4{0.0f, 0.0f, 0.0f, 0.0f})[0];
          sr = fmaf(dyn[v] * y[v], wv[v], sr);
        }
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        yk[s][k] = pick_pair(y, q, k);
        dk[s][k] = pick_pair(dyn, q, k);
        // selected here, not at the uses after the barrier (sunk there, the
        // selects would keep all eight values of every slab live across it)
        asm volatile("" : "+v"(yk[s][k]), "+v"(dk[s][k]));
      }
      // dM over the slab: A = g rows 16I + r, B = x rows 16J + r, 32 channels per step
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        u32x4 ga[2], xb[2];
#pragma unroll
        for (int I = 0; I < 2; ++I) {
          ga[I] = *reinterpret_cast<const u32x4*>(&gs[(16 * I + r) * kMf32Row + 32 * kk + 8 * q]);
          xb[I] = *reinterpret_cast<const u32x4*>(&xs[(16 * I + r) * kMf32Row + 32 * kk + 8 * q]);
        }
#pragma unroll
        for (int I = 0; I < 2; ++I)
#pragma unroll
          for (int J = 0; J < 2; ++J) dm[I][J] = mfma32k<XT>(ga[I], xb[J], dm[I][J]);
      }
    }
    // the four lane groups q hold the same y and dyn: count them once
    ss = q == 0 ? ss : 0.0f;
    sr = q == 0 ? sr : 0.0f;
    ss = wave_sum(ss);
    sr = wave_sum(sr);
    if (lane == 0) {
      s_red[it & 1][0][wave] = ss;
      s_red[it & 1][1][wave] = sr;
    }
    lds_barrier();
    float tss = 0.0f, tsr = 0.0f;
    for (int w = 0; w < nwaves; ++w) {
      tss += s_red[it & 1][0][w];
      tsr += s_red[it & 1][1][w];
    }
    const float inv = 1.0f / sqrtf(tss / (float)C + A.eps);
    const float kf = (inv * inv * inv / (float)C) * tsr;

    const auto rdx = rows_rsrc((const XT*)A.out + t * nC, tokb);
    const int64_t tn = t + gridDim.x < A.T ? t + gridDim.x : t;  // the next token (this one again at the end)
#pragma unroll
    for (int s = SPW - 1; s >= 0; --s) {
      __builtin_amdgcn_sched_barrier(0);
      float wv[8];
      if (s == SPW - 1) {
#pragma unroll
        for (int v = 0; v < 8; ++v) wv[v] = wlast[v];
      } else {
        load_w8(A.w + slab0 + s * 128 + 8 * r, wv);
      }
      // slab SPW - 1 is still staged; the others are staged from the registers
      if (s < SPW - 1) {
        stage();
        if (s > 0) load(Stream{}, t, s - 1);
        else load(Cached{}, tn, 0);
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        __builtin_amdgcn_wave_barrier();
      }
      const uint32_t sb = slabb + (uint32_t)s * 128 * kEs;
      // y and dyn of the lane's 8 channels back from the four lane groups
      float dyv[8], ynv[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const int src = 16 * (v >> 1) + r;
        const float yv = __shfl(yk[s][v & 1], src);
        const float dn = __shfl(dk[s][v & 1], src);
        dyv[v] = dn * inv * wv[v] - kf * yv;
        ynv[v] = (yv * inv) * wv[v];
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) dwv[s][k] = fmaf(dk[s][k], yk[s][k] * inv, dwv[s][k]);
      {
        Vec<XT, 8> rows[8];
        rows_back(gs, rows);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int v = 0; v < 8; ++v) dP[e] = fmaf(rows[e].get(v), ynv[v], dP[e]);
#pragma unroll
        for (int J = 0; J < 2; ++J) {
          const u32x4 amt[3] = {s_par.amt[J][0][lane], s_par.amt[J][1][lane], s_par.amt[J][2][lane]};
          const float4 a4 = s_par.a4[J][q];
          uint32_t ow[4][4];
          f32x4 even;
#pragma unroll
          for (int v = 0; v < 8; ++v) {
            f32x4 acc = {a4.x * dyv[v], a4.y * dyv[v], a4.z * dyv[v], a4.w * dyv[v]};
            acc = mfma_split3<XT>(amt, column8<XT>(rows, v), acc);
            if (v & 1) {
#pragma unroll
              for (int k = 0; k < 4; ++k) ow[k][v >> 1] = pack2<XT>(even[k], acc[k]);
            } else {
              even = acc;
            }
          }
#pragma unroll
          for (int k = 0; k < 4; ++k)
            buf_store_b128<kBufNt>(u32x4{ow[k][0], ow[k][1], ow[k][2], ow[k][3]}, rdx,
                                   FULL ? lane_dx : lane_dx + (uint32_t)(16 * J + k) * rowb,
                                   FULL ? sb + (uint32_t)(16 * J + k) * rowb : sb);
        }
      }
      {
        Vec<XT, 8> rows[8];
        rows_back(xs, rows);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int v = 0; v < 8; ++v) dA[e] = fmaf(dyv[v], rows[e].get(v), dA[e]);
      }
    }
  }

  // ---- the workgroup's partial row [dw C | 0 .. Cp | dM n*n | dA n | dP n | 0 .. P]
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
#pragma unroll
  for (int s = 0; s < SPW; ++s)
    *reinterpret_cast<float2*>(prow + slab0 + s * 128 + 8 * r + 2 * q) = make_float2(dwv[s][0], dwv[s][1]);
  if (tid == 0)
    for (int c = C; c < A.Cp; ++c) prow[c] = 0.0f;
  mf32_bwd_param_sums(A, prow, mf32_lds, n, dm, dA, dP);
}

constexpr int kMf32MaxSpw = 8;      // slabs per wave of the wide backward (C <= 8 waves x 8 x 128)
constexpr int kMf32PipeMaxSpw = 5;  // and of its pipelined variant (6 and more spill)
constexpr int kMf32PipeMaxS = 24;   // slabs per token up to which the pipelined variant is used

// f(std::integral_constant<int, spw>) for spw in 2 .. kMf32MaxSpw.
template <typename F>
void with_spw(int spw, F&& f) {
  switch (spw) {
    case 2: f(std::integral_constant<int, 2>{}); break;
    case 3: f(std::integral_constant<int, 3>{}); break;
    case 4: f(std::integral_constant<int, 4>{}); break;
    case 5: f(std::integral_constant<int, 5>{}); break;
    case 6: f(std::integral_constant<int, 6>{}); break;
    case 7: f(std::integral_constant<int, 7>{}); break;
    case 8: f(std::integral_constant<int, 8>{}); break;
    default: break;
  }
}

// f(std::true_type) for n == 32 (no stream beyond n), else f(std::false_type).
template <typename F>
void with_full(bool full, F&& f) {
  if (full) f(std::true_type{});
  else f(std::false_type{});
}

template <typename F>
int by_half(int code, F&& f) {
  if (code == MHC_DTYPE_BF16) return f((__bf16*)nullptr);
  if (code == MHC_DTYPE_F16) return f((_Float16*)nullptr);
  return 1;
}

}  // namespace

int mf32_fused_fwd_loop(const Mf32Args& A, int xd, int od, hipStream_t s, bool skf);

// skf: the single-launch layer forward (A.hres, A.M_out, A.iters; layer-wide raw parameters)
int mf32_fused_fwd_impl(const Mf32Args& A, int xd, int od, hipStream_t s, bool skf) {
  if (A.n <= 16 || A.n > 32 || A.C % 128 != 0 || A.C > kMf32FwdMaxC) return 1;
  if (skf && (A.M_ts != 0 || A.h_mode != MHC_H_RAW || A.hres == nullptr || A.M_out == nullptr)) return 1;
  if (od != MHC_DTYPE_F32 && od != xd) return 1;
  if (!aligned(A.x, 16) || !aligned(A.out, 16) || !aligned(A.w, 16)) return 1;
  if (knob(kKnobFwdMfma, 1) == 0) return 1;
  const int S = A.C / 128;
  // above C = 2048 the runtime slab loop (above C = 4096 the only variant);
  // MHC_MF32_FWD_LOOP=0 keeps the register variants up to C = 4096, 2 takes
  // the loop at every C
  const int loop = knob(kKnobFwdLoop, 1);
  if (S > 32 || (S > 16 && loop != 0) || loop == 2) return mf32_fused_fwd_loop(A, xd, od, s, skf);
  // two slabs per wave up to C = 2048 (in registers across the RMS barrier),
  // four above it (read again after the barrier)
  const int spw = S <= 8 ? 1 : (S <= 16 ? 2 : 4);
  if (S % spw != 0) return 1;
  const int waves = S / spw;
  const bool pt = A.M_ts != 0, raw = A.h_mode == MHC_H_RAW, full = A.n == 32;
  const int per_cu = knob(kKnobFwdGrid, 8);
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(A.T, (int64_t)device_cu_count() * std::max(per_cu, 1)));
  const dim3 g((unsigned)blocks), b(waves * 64);
  return by_half(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    auto go = [&](auto* op) {
      using OT = std::remove_pointer_t<decltype(op)>;
#define MF32_FWD(SPW_, PT_, RAW_)                                                                 \
  do {                                                                                             \
    if (full) hipLaunchKernelGGL((mf32_fwd_kernel<XT, OT, SPW_, PT_, RAW_, true>), g, b, 0, s, A);  \
    else hipLaunchKernelGGL((mf32_fwd_kernel<XT, OT, SPW_, PT_, RAW_, false>), g, b, 0, s, A);      \
  } while (0)
#define MF32_FWD_RELOAD(PT_, RAW_)                                                                 \
  do {                                                                                             \
    if (full) hipLaunchKernelGGL((mf32_fwd_kernel<XT, OT, 4, PT_, RAW_, true, true>), g, b, 0, s, A);  \
    else hipLaunchKernelGGL((mf32_fwd_kernel<XT, OT, 4, PT_, RAW_, false, true>), g, b, 0, s, A);      \
  } while (0)
#define MF32_FWD_SKF(SPW_, RELOAD_)                                                                          \
  do {                                                                                                       \
    if (full) hipLaunchKernelGGL((mf32_fwd_kernel<XT, OT, SPW_, false, true, true, RELOAD_, true>), g, b, 0, s, A); \
    else hipLaunchKernelGGL((mf32_fwd_kernel<XT, OT, SPW_, false, true, false, RELOAD_, true>), g, b, 0, s, A);     \
  } while (0)
      if (skf) {
        if (spw == 1) MF32_FWD_SKF(1, false);
        else if (spw == 2) MF32_FWD_SKF(2, false);
        else MF32_FWD_SKF(4, true);
      } else if (spw == 1) {
        if (pt) { if (raw) MF32_FWD(1, true, true); else MF32_FWD(1, true, false); }
        else { if (raw) MF32_FWD(1, false, true); else MF32_FWD(1, false, false); }
      } else if (spw == 2) {
        if (pt) { if (raw) MF32_FWD(2, true, true); else MF32_FWD(2, true, false); }
        else { if (raw) MF32_FWD(2, false, true); else MF32_FWD(2, false, false); }
      } else {
        if (pt) { if (raw) MF32_FWD_RELOAD(true, true); else MF32_FWD_RELOAD(true, false); }
        else { if (raw) MF32_FWD_RELOAD(false, true); else MF32_FWD_RELOAD(false, false); }
      }
#undef MF32_FWD
#undef MF32_FWD_RELOAD
#undef MF32_FWD_SKF
      MHC_CHECK_LAUNCH("mf32_fwd_kernel");
      return MHC_OK;
    };
    return od == MHC_DTYPE_F32 ? go((float*)nullptr) : go((XT*)nullptr);
  });
}

// The runtime-loop forward: the wave count nearest MHC_MF32_FWD_WAVES (default
// 8) that divides the slab count, one token per workgroup at a time.
int mf32_fused_fwd_loop(const Mf32Args& A, int xd, int od, hipStream_t s, bool skf) {
  const int S = A.C / 128;
  const int target = std::min(kMf32MaxWaves, std::max(1, knob(kKnobMf32FwdWaves, 8)));
  int waves = 1;
  for (int w = 1; w <= kMf32MaxWaves; ++w)
    if (S % w == 0 && std::abs(w - target) < std::abs(waves - target)) waves = w;
  const int spw = S / waves;
  const size_t smem = (size_t)S * 16 * 8 * sizeof(float);
  const bool pt = A.M_ts != 0, raw = A.h_mode == MHC_H_RAW, full = A.n == 32;
  const int per_cu = knob(kKnobFwdGrid, 8);
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(A.T, (int64_t)device_cu_count() * std::max(per_cu, 1)));
  const dim3 g((unsigned)blocks), b(waves * 64);
  return by_half(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    auto go = [&](auto* op) {
      using OT = std::remove_pointer_t<decltype(op)>;
      with_full(full, [&](auto fc) {
        constexpr bool F = decltype(fc)::value;
        if (skf) {
          hipLaunchKernelGGL((mf32_fwd_loop_kernel<XT, OT, false, true, F, true>), g, b, smem, s, A, spw);
        } else if (pt) {
          if (raw) hipLaunchKernelGGL((mf32_fwd_loop_kernel<XT, OT, true, true, F>), g, b, smem, s, A, spw);
          else hipLaunchKernelGGL((mf32_fwd_loop_kernel<XT, OT, true, false, F>), g, b, smem, s, A, spw);
        } else {
          if (raw) hipLaunchKernelGGL((mf32_fwd_loop_kernel<XT, OT, false, true, F>), g, b, smem, s, A, spw);
          else hipLaunchKernelGGL((mf32_fwd_loop_kernel<XT, OT, false, false, F>), g, b, smem, s, A, spw);
        }
      });
      MHC_CHECK_LAUNCH("mf32_fwd_loop_kernel");
      return MHC_OK;
    };
    return od == MHC_DTYPE_F32 ? go((float*)nullptr) : go((XT*)nullptr);
  });
}

// 32 < n <= 64: mf64_fwd_loop_kernel (W waves near MHC_MF32_FWD_WAVES walking the slabs, C a multiple
// of 128 up to 8192: the y buffer and the split operands fit in LDS), layer-wide or per-token parameters.
int mf64_fused_fwd(const Mf32Args& A, int xd, int od, hipStream_t s) {
  if (A.n <= 32 || A.n > 64 || A.C % 128 != 0 || A.C > 8192) return 1;
  if (od != MHC_DTYPE_F32 && od != xd) return 1;
  if (!aligned(A.x, 16) || !aligned(A.out, 16) || !aligned(A.w, 16)) return 1;
  if (knob(kKnobFwdMfma, 1) == 0) return 1;
  const int S = A.C / 128;
  const int target = std::min(kMf32MaxWaves, std::max(1, knob(kKnobMf32FwdWaves, 8)));
  int waves = 1;
  for (int w = 1; w <= kMf32MaxWaves; ++w)
    if (S % w == 0 && std::abs(w - target) < std::abs(waves - target)) waves = w;
  const int spw = S / waves;
  const size_t smem = (size_t)S * 16 * 8 * sizeof(float);
  const bool raw = A.h_mode == MHC_H_RAW, full = A.n == 64, pt = A.M_ts != 0;
  const int per_cu = knob(kKnobFwdGrid, 8);
  const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(A.T, (int64_t)device_cu_count() * std::max(per_cu, 1)));
  const dim3 g((unsigned)blocks), b(waves * 64);
  return by_half(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    auto go = [&](auto* op) {
      using OT = std::remove_pointer_t<decltype(op)>;
      with_full(full, [&](auto fc) {
        constexpr bool F = decltype(fc)::value;
        if (pt) {
          if (raw) hipLaunchKernelGGL((mf64_fwd_loop_kernel<XT, OT, true, F, true>), g, b, smem, s, A, spw);
          else hipLaunchKernelGGL((mf64_fwd_loop_kernel<XT, OT, false, F, true>), g, b, smem, s, A, spw);
        } else {
          if (raw) hipLaunchKernelGGL((mf64_fwd_loop_kernel<XT, OT, true, F, false>), g, b, smem, s, A, spw);
          else hipLaunchKernelGGL((mf64_fwd_loop_kernel<XT, OT, false, F, false>), g, b, smem, s, A, spw);
        }
      });
      MHC_CHECK_LAUNCH("mf64_fwd_loop_kernel");
      return MHC_OK;
    };
    return od == MHC_DTYPE_F32 ? go((float*)nullptr) : go((XT*)nullptr);
  });
}

int mf32_fused_fwd(const Mf32Args& A, int xd, int od, hipStream_t s) {
  if (A.n > 32) return mf64_fused_fwd(A, xd, od, s);
  return mf32_fused_fwd_impl(A, xd, od, s, false);
}

int mf32_layer_fwd_single_launch(const Mf32Args& A, int xd, int od, hipStream_t s) {
  if (knob(kKnobFwdSkf, 1) == 0 || A.T < 1 || A.T > device_cu_count()) return 1;
  return mf32_fused_fwd_impl(A, xd, od, s, true);
}

// 16 < n <= 64 with per-token parameters (mf64_bwd_pt_kernel; the n <= 32 kernel takes C up to 1024): whole
// tokens per wave, up to four waves per
// workgroup as the waves' LDS (12 C + 512 bytes each) allows two workgroups per CU.
int mf64_fused_bwd_pt(const Mf32Args& A, int xd, int gd, int64_t gmax, hipStream_t s, int64_t* num_partials) {
  if (A.n <= 16 || A.n > 64 || A.C % 128 != 0 || A.C > kMf64BwdPtMaxC) return 1;
  if (gd != xd || (xd != MHC_DTYPE_BF16 && xd != MHC_DTYPE_F16)) return 1;
  if (A.P != A.Cp || A.dM_tok == nullptr || A.dpre_tok == nullptr || A.dpost_tok == nullptr) return 1;
  if (!aligned(A.x, 16) || !aligned(A.g, 16) || !aligned(A.out, 16) || !aligned(A.w, 16) || !aligned(A.part, 16))
    return 1;
  if (knob(kKnobBwdMfma, 1) == 0) return 1;
  const size_t per_wave = (size_t)(3 * A.C + 128) * sizeof(float);
  const int waves = (int)std::max<size_t>(1, std::min<size_t>(4, (size_t)(80 * 1024) / per_wave));
  const size_t smem = waves * per_wave;
  const bool raw = A.h_mode == MHC_H_RAW, full = A.n == 64, nb2 = A.n <= 32;
  return by_half(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    const void* kfn = nb2 ? (raw ? (const void*)mf64_bwd_pt_kernel<XT, true, false, 2>
                                 : (const void*)mf64_bwd_pt_kernel<XT, false, false, 2>)
                    : full ? (raw ? (const void*)mf64_bwd_pt_kernel<XT, true, true, 4>
                                  : (const void*)mf64_bwd_pt_kernel<XT, false, true, 4>)
                           : (raw ? (const void*)mf64_bwd_pt_kernel<XT, true, false, 4>
                                  : (const void*)mf64_bwd_pt_kernel<XT, false, false, 4>);
    const int occ = occupancy_blocks(kfn, waves * 64, smem);
    if (occ <= 0) return 1;
    int64_t blocks = std::min<int64_t>(gmax, (int64_t)device_cu_count() * occ);
    const int grid_pref = knob(kKnobBwdGrid, 0);
    if (grid_pref > 0) blocks = std::min<int64_t>(gmax, grid_pref);
    blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, (A.T + waves - 1) / waves));
    const dim3 g((unsigned)blocks), b(waves * 64);
    if (nb2) {
      if (raw) hipLaunchKernelGGL((mf64_bwd_pt_kernel<XT, true, false, 2>), g, b, smem, s, A);
      else hipLaunchKernelGGL((mf64_bwd_pt_kernel<XT, false, false, 2>), g, b, smem, s, A);
    } else {
      with_full(full, [&](auto fc) {
        constexpr bool F = decltype(fc)::value;
        if (raw) hipLaunchKernelGGL((mf64_bwd_pt_kernel<XT, true, F, 4>), g, b, smem, s, A);
        else hipLaunchKernelGGL((mf64_bwd_pt_kernel<XT, false, F, 4>), g, b, smem, s, A);
      });
    }
    MHC_CHECK_LAUNCH("mf64_bwd_pt_kernel");
    *num_partials = blocks;
    return MHC_OK;
  });
}

// 16 < n <= 64 (mf64_bwd_kernel; below n = 32 where the n <= 32 kernels do not reach): the wave count
// nearest MHC_MF32_WAVES (default 8) dividing the slab
// count (below C = 512 one wave per slab), as many workgroups per CU as fit.
int mf64_fused_bwd(const Mf32Args& A, int xd, int gd, int64_t gmax, hipStream_t s, int64_t* num_partials) {
  if (A.M_ts != 0) return mf64_fused_bwd_pt(A, xd, gd, gmax, s, num_partials);
  if (A.n <= 16 || A.n > 64 || A.C % 128 != 0 || A.C > kMf64BwdMaxC) return 1;
  if (gd != xd || (xd != MHC_DTYPE_BF16 && xd != MHC_DTYPE_F16)) return 1;
  if (A.P != A.Cp + round_up(A.n * A.n + 2 * A.n, 4)) return 1;
  if (!aligned(A.x, 16) || !aligned(A.g, 16) || !aligned(A.out, 16) || !aligned(A.w, 16) || !aligned(A.part, 16))
    return 1;
  if (knob(kKnobBwdMfma, 1) == 0) return 1;
  const int S = A.C / 128;
  const int target = std::min(kMf32MaxWaves, std::max(4, knob(kKnobMf32Waves, 8)));
  int waves = 1;
  for (int w = 1; w <= kMf32MaxWaves; ++w)
    if (S % w == 0 && std::abs(w - target) < std::abs(waves - target)) waves = w;
  const int spw = S / waves;
  // one slab per wave and at least two waves: G stays in LDS across the RMS barrier (16 KB per wave)
  const bool gl = spw == 1 && waves >= 2 && knob(kKnobBwdPipe, 1) != 0;
  const size_t smem = (size_t)3 * S * 128 * sizeof(float) + (gl ? (size_t)waves * 128 * 64 * sizeof(uint16_t) : 0);
  const bool raw = A.h_mode == MHC_H_RAW, full = A.n == 64, nb2 = A.n <= 32;
  return by_half(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    const void* kfn;
    if (nb2) kfn = gl ? (raw ? (const void*)mf64_bwd_kernel<XT, true, false, true, 2> : (const void*)mf64_bwd_kernel<XT, false, false, true, 2>)
                      : (raw ? (const void*)mf64_bwd_kernel<XT, true, false, false, 2> : (const void*)mf64_bwd_kernel<XT, false, false, false, 2>);
    else if (gl) kfn = full ? (raw ? (const void*)mf64_bwd_kernel<XT, true, true, true, 4> : (const void*)mf64_bwd_kernel<XT, false, true, true, 4>)
                            : (raw ? (const void*)mf64_bwd_kernel<XT, true, false, true, 4> : (const void*)mf64_bwd_kernel<XT, false, false, true, 4>);
    else kfn = full ? (raw ? (const void*)mf64_bwd_kernel<XT, true, true, false, 4> : (const void*)mf64_bwd_kernel<XT, false, true, false, 4>)
                    : (raw ? (const void*)mf64_bwd_kernel<XT, true, false, false, 4> : (const void*)mf64_bwd_kernel<XT, false, false, false, 4>);
    const int occ = occupancy_blocks(kfn, waves * 64, smem);
    if (occ <= 0) return 1;
    int64_t blocks = std::min<int64_t>(gmax, (int64_t)device_cu_count() * occ);
    const int grid_pref = knob(kKnobBwdGrid, 0);
    if (grid_pref > 0) blocks = std::min<int64_t>(gmax, grid_pref);
    blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, A.T));
    const dim3 g((unsigned)blocks), b(waves * 64);
    if (nb2) {
      if (gl) {
        if (raw) hipLaunchKernelGGL((mf64_bwd_kernel<XT, true, false, true, 2>), g, b, smem, s, A, spw);
        else hipLaunchKernelGGL((mf64_bwd_kernel<XT, false, false, true, 2>), g, b, smem, s, A, spw);
      } else {
        if (raw) hipLaunchKernelGGL((mf64_bwd_kernel<XT, true, false, false, 2>), g, b, smem, s, A, spw);
        else hipLaunchKernelGGL((mf64_bwd_kernel<XT, false, false, false, 2>), g, b, smem, s, A, spw);
      }
    } else {
      with_full(full, [&](auto fc) {
        constexpr bool F = decltype(fc)::value;
        if (gl) {
          if (raw) hipLaunchKernelGGL((mf64_bwd_kernel<XT, true, F, true, 4>), g, b, smem, s, A, spw);
          else hipLaunchKernelGGL((mf64_bwd_kernel<XT, false, F, true, 4>), g, b, smem, s, A, spw);
        } else {
          if (raw) hipLaunchKernelGGL((mf64_bwd_kernel<XT, true, F, false, 4>), g, b, smem, s, A, spw);
          else hipLaunchKernelGGL((mf64_bwd_kernel<XT, false, F, false, 4>), g, b, smem, s, A, spw);
        }
      });
    }
    MHC_CHECK_LAUNCH("mf64_bwd_kernel");
    *num_partials = blocks;
    return MHC_OK;
  });
}

// 16 < n <= 32 with per-token parameters (mf32_bwd_pt_kernel): one slab per wave, so C up to 1024.
int mf32_fused_bwd_pt(const Mf32Args& A, int xd, int gd, int64_t gmax, hipStream_t s, int64_t* num_partials) {
  if (A.n <= 16 || A.n > 32 || A.C % 128 != 0 || A.C / 128 > kMf32MaxWaves) return 1;
  if (gd != xd || (xd != MHC_DTYPE_BF16 && xd != MHC_DTYPE_F16)) return 1;
  if (A.P != A.Cp || A.dM_tok == nullptr || A.dpre_tok == nullptr || A.dpost_tok == nullptr) return 1;
  if (!aligned(A.x, 16) || !aligned(A.g, 16) || !aligned(A.out, 16) || !aligned(A.w, 16) || !aligned(A.part, 16))
    return 1;
  if (knob(kKnobBwdMfma, 1) == 0) return 1;
  const int waves = A.C / 128;
  const size_t smem = (size_t)waves * kMf32Slab * sizeof(uint16_t);
  const bool raw = A.h_mode == MHC_H_RAW, full = A.n == 32;
  return by_half(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    const void* kfn = full ? (raw ? (const void*)mf32_bwd_pt_kernel<XT, true, true>
                                  : (const void*)mf32_bwd_pt_kernel<XT, false, true>)
                           : (raw ? (const void*)mf32_bwd_pt_kernel<XT, true, false>
                                  : (const void*)mf32_bwd_pt_kernel<XT, false, false>);
    const int occ = occupancy_blocks(kfn, waves * 64, smem);
    if (occ <= 0) return 1;
    int64_t blocks = std::min<int64_t>(gmax, (int64_t)device_cu_count() * occ);
    const int grid_pref = knob(kKnobBwdGrid, 0);
    if (grid_pref > 0) blocks = std::min<int64_t>(gmax, grid_pref);
    blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, A.T));
    const dim3 g((unsigned)blocks), b(waves * 64);
    with_full(full, [&](auto fc) {
      constexpr bool F = decltype(fc)::value;
      if (raw) hipLaunchKernelGGL((mf32_bwd_pt_kernel<XT, true, F>), g, b, smem, s, A);
      else hipLaunchKernelGGL((mf32_bwd_pt_kernel<XT, false, F>), g, b, smem, s, A);
    });
    MHC_CHECK_LAUNCH("mf32_bwd_pt_kernel");
    *num_partials = blocks;
    return MHC_OK;
  });
}

static int mf32_fused_bwd_lw(const Mf32Args& A, int xd, int gd, int64_t gmax, hipStream_t s,
                             int64_t* num_partials);

// 16 < n <= 32, layer-wide parameters: the n = 32 kernels, and where they do not reach (above C = 5120
// for n < 32) the 32 < n <= 64 kernel with the rows past n read as zero.  Per-token parameters: whole
// tokens per wave (mf64_bwd_pt_kernel with two 16-row blocks); MHC_BWD_LEGACY=1 takes the workgroup-
// per-token kernel (mf32_bwd_pt_kernel, C up to 1024) first.  Measured, bf16 backward kernel:
// 8192 x 32 x 512 284 -> 222 us, 4096 x 24 x 512 170 -> 95 us, 2048 x 32 x 1024 111 us both.
int mf32_fused_bwd(const Mf32Args& A, int xd, int gd, int64_t gmax, hipStream_t s, int64_t* num_partials) {
  if (A.n > 32) return mf64_fused_bwd(A, xd, gd, gmax, s, num_partials);
  if (A.M_ts != 0) {
    const bool legacy = knob(kKnobBwdLegacy, 0) == 1;
    int rc = legacy ? mf32_fused_bwd_pt(A, xd, gd, gmax, s, num_partials)
                    : mf64_fused_bwd_pt(A, xd, gd, gmax, s, num_partials);
    if (rc == 1) rc = legacy ? mf64_fused_bwd_pt(A, xd, gd, gmax, s, num_partials)
                             : mf32_fused_bwd_pt(A, xd, gd, gmax, s, num_partials);
    return rc;
  }
  const int rc = mf32_fused_bwd_lw(A, xd, gd, gmax, s, num_partials);
  return rc == 1 ? mf64_fused_bwd(A, xd, gd, gmax, s, num_partials) : rc;
}

static int mf32_fused_bwd_lw(const Mf32Args& A, int xd, int gd, int64_t gmax, hipStream_t s,
                             int64_t* num_partials) {
  if (A.n <= 16 || A.n > 32 || A.M_ts != 0 || A.C % 128 != 0) return 1;
  if (gd != xd || (xd != MHC_DTYPE_BF16 && xd != MHC_DTYPE_F16)) return 1;
  if (A.P != A.Cp + round_up(A.n * A.n + 2 * A.n, 4)) return 1;
  if (!aligned(A.x, 16) || !aligned(A.g, 16) || !aligned(A.out, 16) || !aligned(A.w, 16) || !aligned(A.part, 16))
    return 1;
  if (knob(kKnobBwdMfma, 1) == 0) return 1;
  const int S = A.C / 128;
  // one slab per wave up to C = 1024; above it (n == 32 only) SPW = 2 .. 8
  // slabs per wave, with x and g read again after the RMS barrier: the wave
  // count nearest MHC_MF32_WAVES among those that divide S.  Default 8 waves
  // up to C = 3072 and 4 above (two workgroups per CU).  Measured, 2048 tokens
  // (4096 at C = 2048), bf16, pipelined / not: C = 2048 on 8 waves 327 / 354
  // us, on 4 341 us; C = 3072 on 8 waves 252 / 268 us; C = 4096 on 8 waves
  // 423 / 400 us, on 4 (eight slabs, not pipelined) 383 us.
  // (n < 32 up to kMf32PipeMaxSpw slabs per wave: the per-row offsets of the
  // range-checked rows cost registers)
  const bool full = A.n == 32;
  int spw = 1;
  if (S > kMf32MaxWaves) {
    const int target = std::max(1, knob(kKnobMf32Waves, S <= kMf32PipeMaxS ? kMf32MaxWaves : 4));
    const int max_spw = full ? kMf32MaxSpw : kMf32PipeMaxSpw;
    spw = 0;
    for (int c = 2; c <= max_spw; ++c) {
      if (S % c != 0 || S / c > kMf32MaxWaves) continue;
      if (spw == 0 || std::abs(S / c - target) < std::abs(S / spw - target)) spw = c;
    }
    if (spw == 0) return 1;
  }
  const int waves = S / spw;
  const size_t smem = std::max<size_t>((size_t)waves * kMf32Slab * sizeof(uint16_t),
                                       (size_t)waves * kMf32Par * sizeof(float));
  const bool raw = A.h_mode == MHC_H_RAW;
  // the pipelined kernel up to C = 3072 and kMf32PipeMaxSpw slabs per wave
  const bool pipe = full && knob(kKnobBwdPipe, 1) != 0 && spw <= kMf32PipeMaxSpw && S <= kMf32PipeMaxS;
  return by_half(xd, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    const void* kfn = nullptr;
    if (spw == 1) {
      kfn = full ? (raw ? (const void*)mf32_bwd_kernel<XT, true, true> : (const void*)mf32_bwd_kernel<XT, false, true>)
                 : (raw ? (const void*)mf32_bwd_kernel<XT, true, false> : (const void*)mf32_bwd_kernel<XT, false, false>);
    } else {
      with_spw(spw, [&](auto c) {
        constexpr int SPW = decltype(c)::value;
        with_full(full, [&](auto fc) {
          constexpr bool F = decltype(fc)::value;
          if constexpr (F && SPW <= kMf32PipeMaxSpw) {
            if (pipe)
              kfn = raw ? (const void*)mf32_bwd_pipe_kernel<XT, true, SPW, F>
                        : (const void*)mf32_bwd_pipe_kernel<XT, false, SPW, F>;
          }
          if constexpr (F || SPW <= kMf32PipeMaxSpw) {
            if (kfn == nullptr)
              kfn = raw ? (const void*)mf32_bwd_wide_kernel<XT, true, SPW, F>
                        : (const void*)mf32_bwd_wide_kernel<XT, false, SPW, F>;
          }
        });
      });
    }
    const int occ = occupancy_blocks(kfn, waves * 64, smem);
    if (occ <= 0) return 1;
    int64_t blocks = std::min<int64_t>(gmax, (int64_t)device_cu_count() * occ);
    const int grid_pref = knob(kKnobBwdGrid, 0);
    if (grid_pref > 0) blocks = std::min<int64_t>(gmax, grid_pref);
    blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, A.T));
    const dim3 g((unsigned)blocks), b(waves * 64);
    if (spw == 1) {
      if (full) {
        if (raw) hipLaunchKernelGGL((mf32_bwd_kernel<XT, true, true>), g, b, smem, s, A);
        else hipLaunchKernelGGL((mf32_bwd_kernel<XT, false, true>), g, b, smem, s, A);
      } else {
        if (raw) hipLaunchKernelGGL((mf32_bwd_kernel<XT, true, false>), g, b, smem, s, A);
        else hipLaunchKernelGGL((mf32_bwd_kernel<XT, false, false>), g, b, smem, s, A);
      }
    } else {
      with_spw(spw, [&](auto c) {
        constexpr int SPW = decltype(c)::value;
        with_full(full, [&](auto fc) {
          constexpr bool F = decltype(fc)::value;
          bool launched = false;
          if constexpr (F && SPW <= kMf32PipeMaxSpw) {
            if (pipe) {
              if (raw) hipLaunchKernelGGL((mf32_bwd_pipe_kernel<XT, true, SPW, F>), g, b, smem, s, A);
              else hipLaunchKernelGGL((mf32_bwd_pipe_kernel<XT, false, SPW, F>), g, b, smem, s, A);
              launched = true;
            }
          }
          if constexpr (F || SPW <= kMf32PipeMaxSpw) {
            if (!launched) {
              if (raw) hipLaunchKernelGGL((mf32_bwd_wide_kernel<XT, true, SPW, F>), g, b, smem, s, A);
              else hipLaunchKernelGGL((mf32_bwd_wide_kernel<XT, false, SPW, F>), g, b, smem, s, A);
            }
          }
        });
      });
    }
    MHC_CHECK_LAUNCH("mf32_bwd_kernel");
    *num_partials = blocks;
    return MHC_OK;
  });
}

}  // namespace mhc
