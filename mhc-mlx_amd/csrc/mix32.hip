// MHCRewire post-combine (stream_mix_add, mhc_mlx/layer.py:302-337,
// metal.py:954-1014) for 16 < n <= 64 on MFMA (v_mfma_f32_16x16x4_f32):
//   forward   out = Mf X + p Y                   (Mf_ij = p_i M_ij a_j)
//   backward  dx = Mf^T G,  dy = p G,  S = G X^T,  Yd_i = sum_c G_ic Y_ic
// At n = 32 each of Mf X, Mf^T G and G X^T is 1024 FMAs per channel, far
// more VALU issue time than the channel's HBM time; on the fp32 matrix cores
// (fp32 operands, so the products are those of the fp32 parameters with the
// data, whatever its storage type) all three fit under the HBM time.
//
// Work item: one wave, one (token, 64-channel slab).  Lane (q = lane >> 4,
// r = lane & 15).  v_mfma_f32_16x16x4_f32 operands: A row r, k = q; B k = q,
// column r; D rows 4q .. 4q+3 of column r.
//
// Stream contractions (Mf X, Mf^T G): K = streams 4m + q (m = 0..7), the
// columns are the channels 4r + v (v = 0..3) of the slab, so the lane loads
// streams 4m + q, channels [4r, 4r + 4); D of row block I holds streams
// 16I + 4q + k at those four channels.
//
// Channel contraction (S = G X^T): K = channels, rows and columns are
// streams: the lane loads streams 16I + r, channels [32g + 8q, +8) of the
// slab (g = 0, 1), and MFMA (g, e) contracts channel 32g + 8q + e over the
// four lane groups q.  The backward loads G in this layout, stages it in LDS
// (one row per stream) and reads it back in the stream-contraction layout
// for dx.
//
// The backward's S and Yd stay in registers across the wave's items and end
// in one partial row per workgroup, [S n*n | Yd n | pad], the waves added in
// wave order, for the fixed-order row reduction of mhc_stream_mix_add_bwd.
#include "mhc_device.hpp"
#include "mhc_host.hpp"
#include "mhc_mix32.hpp"
#include "mhc_plan.hpp"

namespace mhc {

namespace {

MHC_DEV f32x4 mfma4(float a, float b, f32x4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

constexpr int kMxSlab = 64;          // channels per item
constexpr int kMxWaves = 4;          // waves per workgroup
constexpr int kMxThreads = 64 * kMxWaves;
constexpr int kMxPitch = kMxSlab + 4;  // LDS row of the staged G slab (floats)

// Mf (32 x 32, zero past n) and p (32) into LDS.
MHC_DEV void mx_stage(float* s_mf, float* s_p, const Mix32Args& A) {
  const int n = A.n;
  auto act_a = [&](int j) {
    if (A.h_mode == MHC_H_NONE) return 1.0f;
    return A.h_mode == MHC_H_RAW ? sigmoidf_(A.hpre[j]) : A.hpre[j];
  };
  auto act_p = [&](int i) {
    if (A.h_mode == MHC_H_NONE) return 1.0f;
    return A.h_mode == MHC_H_RAW ? 2.0f * sigmoidf_(A.hpost[i]) : A.hpost[i];
  };
  for (int idx = threadIdx.x; idx < 32 * 32 + 32; idx += blockDim.x) {
    if (idx < 32 * 32) {
      const int i = idx >> 5, j = idx & 31;
      s_mf[idx] = (i < n && j < n) ? act_p(i) * A.M[i * n + j] * act_a(j) : 0.0f;
    } else {
      const int i = idx - 32 * 32;
      s_p[i] = i < n ? act_p(i) : 0.0f;
    }
  }
}

template <typename T, int V>
MHC_DEV void ldv(const T* p, float (&v)[V]) {
  Vec<T, V> u;
  u.load(p);
#pragma unroll
  for (int k = 0; k < V; ++k) v[k] = u.get(k);
}

// base + elems elements, the byte offset formed in 32 bits (a scalar base
// plus a zero-extended 32-bit lane offset: the scalar-base address form)
template <typename T>
MHC_DEV T* at(T* base, uint32_t elems) {
  using B = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return reinterpret_cast<T*>(reinterpret_cast<B*>(base) + (uint64_t)(elems * (uint32_t)sizeof(T)));
}

template <int V>
MHC_DEV void zerov(float (&v)[V]) {
#pragma unroll
  for (int k = 0; k < V; ++k) v[k] = 0.0f;
}

// A wave's grid-stride walk over (token, 64-channel slab) items, tracked
// incrementally (no 64-bit division per item; the walk is wave-uniform and
// lives in scalar registers).  off(): element offset of the item's slab in a
// [T, n, C] tensor.
struct SlabWalk {
  int64_t it, stride, items, t, dt, nC;
  int s, ds, nslabs;
  MHC_DEV SlabWalk(int64_t first, int64_t stride_, int64_t items_, int nslabs_, int64_t nC_)
      : it(first), stride(stride_), items(items_), nC(nC_), nslabs(nslabs_) {
    t = first / nslabs;
    s = (int)(first - t * nslabs);
    dt = stride / nslabs;
    ds = (int)(stride - dt * nslabs);
  }
  MHC_DEV bool valid() const { return it < items; }
  MHC_DEV int64_t off() const { return t * nC + (int64_t)s * kMxSlab; }
  // the next item's offset, or this item's when it is the wave's last (a
  // valid address for loads that are not used)
  MHC_DEV int64_t next_off() const {
    int64_t tn = t + dt;
    int sn = s + ds;
    if (sn >= nslabs) {
      sn -= nslabs;
      ++tn;
    }
    return it + stride < items ? tn * nC + (int64_t)sn * kMxSlab : off();
  }
  MHC_DEV void advance() {
    it += stride;
    t += dt;
    s += ds;
    if (s >= nslabs) {
      s -= nslabs;
      ++t;
    }
  }
};

// ---------------------------------------------------------------------------
// Forward: out = Mf X + p Y.
// ---------------------------------------------------------------------------

// FULL: n == 32 and y present, so no load or store is conditional (a
// conditional memory access makes the compiler's vmcnt waits conservative:
// the wait for this item's operands would also wait for the next item's
// loads).
template <typename XT, typename YT, typename OT, bool FULL>
__global__ __launch_bounds__(kMxThreads) void mix32_fwd_kernel(Mix32Args A) {
  __shared__ float s_mf[32 * 32];
  __shared__ float s_p[32];
  mx_stage(s_mf, s_p, A);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 32 : A.n, C = A.C;
  const int nslabs = C / kMxSlab;
  const int64_t nC = (int64_t)n * C;
  // A operands: Mf row 16I + r at streams 4m + q; p of the output rows 16I + 4q + k
  float am[2][8], pv[2][4];
#pragma unroll
  for (int I = 0; I < 2; ++I) {
#pragma unroll
    for (int m = 0; m < 8; ++m) am[I][m] = s_mf[(16 * I + r) * 32 + 4 * m + q];
#pragma unroll
    for (int k = 0; k < 4; ++k) pv[I][k] = s_p[16 * I + 4 * q + k];
  }
  const XT* X = (const XT*)A.x;
  const YT* Y = (const YT*)A.y;
  OT* O = (OT*)A.out;
  const bool hasy = FULL || Y != nullptr;
  const int64_t items = A.T * nslabs;
  const int64_t stride = (int64_t)gridDim.x * kMxWaves;
  // an item's x (streams 4m + q) and y (streams 16I + 4q + k), packed as stored
  struct In {
    Vec<XT, 4> x[8];
    Vec<YT, 4> y[2][4];
  };
  // addresses: the item's slab (wave-uniform, scalar registers) plus a 32-bit
  // lane offset (n C < 2^31), so the loads and stores take the scalar-base form
  auto load = [&](int64_t slab, In& d) {
    const XT* xs = X + slab;
    const YT* ys = Y + slab;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const int i = 4 * m + q;
      if (FULL || i < n) d.x[m].load(at(xs, (uint32_t)(i * C + 4 * r)));
      else d.x[m].zero();
    }
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = 16 * I + 4 * q + k;
        if (hasy && (FULL || i < n)) d.y[I][k].load(at(ys, (uint32_t)(i * C + 4 * r)));
        else d.y[I][k].zero();
      }
  };
  // The next item's loads go into the same registers once this item's
  // operands are consumed, before this item's stores: a vmcnt wait counts
  // stores too, so loads issued after them would wait for them.  The last
  // item reloads itself (a valid address, no branch around the loads).
  In d;
  SlabWalk w((int64_t)blockIdx.x * kMxWaves + wave, stride, items, nslabs, nC);
  // The first item's loads are waited for here: entering the loop with them
  // pending would make every iteration's waits as strict as the first's (no
  // stores issued after the loads), i.e. wait for the previous item's stores.
  if (w.valid()) load(w.off(), d);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  for (; w.valid(); w.advance()) {
    OT* os = O + w.off();
    float o[2][4][4];
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 8; ++m) acc = mfma4(am[I][m], d.x[m].get(v), acc);
#pragma unroll
        for (int k = 0; k < 4; ++k) o[I][k][v] = fmaf(pv[I][k], d.y[I][k].get(v), acc[k]);
      }
    load(w.next_off(), d);
    issue_fence();
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int i = 16 * I + 4 * q + k;
        if (FULL || i < n) store_vec<OT, 4>(at(os, (uint32_t)(i * C + 4 * r)), o[I][k]);
      }
  }
}

// ---------------------------------------------------------------------------
// Backward: dx = Mf^T G, dy = p G, and the sums S = G X^T, Yd = (G . Y) per
// stream.
// ---------------------------------------------------------------------------

// FULL: n == 32 with y and dy present (no conditional load or store).
template <typename XT, typename YT, typename GT, bool FULL>
__global__ __launch_bounds__(kMxThreads) __attribute__((amdgpu_waves_per_eu(FULL ? 2 : 1)))
void mix32_bwd_kernel(Mix32Args A) {
  __shared__ float s_mf[32 * 32];
  __shared__ float s_p[32];
  __shared__ __align__(16) float s_g[kMxWaves][32 * kMxPitch];
  mx_stage(s_mf, s_p, A);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 32 : A.n, C = A.C;
  const int nslabs = C / kMxSlab;
  const int64_t nC = (int64_t)n * C;
  // A operands of Mf^T: column 16J + r of Mf at rows 4m + q; p of streams 16I + r
  float amt[2][8], pr[2];
#pragma unroll
  for (int J = 0; J < 2; ++J) {
#pragma unroll
    for (int m = 0; m < 8; ++m) amt[J][m] = s_mf[(4 * m + q) * 32 + 16 * J + r];
    pr[J] = s_p[16 * J + r];
  }
  const XT* X = (const XT*)A.x;
  const YT* Y = (const YT*)A.y;
  const GT* G = (const GT*)A.g;
  XT* DX = (XT*)A.out;
  YT* DY = (YT*)A.dy;
  const bool hasy = FULL || Y != nullptr, hasdy = FULL || DY != nullptr;
  float* gs = s_g[wave];

  f32x4 sacc[2][2];
#pragma unroll
  for (int I = 0; I < 2; ++I)
#pragma unroll
    for (int J = 0; J < 2; ++J) sacc[I][J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float yd[2] = {0.0f, 0.0f};

  const int64_t items = A.T * nslabs;
  const int64_t stride = (int64_t)gridDim.x * kMxWaves;
  // an item's G, X and Y in the channel-contraction layout (streams 16I + r,
  // channels 32g + 8q .. +8), packed as stored
  struct In {
    Vec<GT, 8> g[2][2];
    Vec<XT, 8> x[2][2];
    Vec<YT, 8> y[2][2];
  };
  // addresses: the item's slab (wave-uniform, scalar registers) plus a 32-bit
  // lane offset (n C < 2^31), so the loads and stores take the scalar-base form
  auto load = [&](int64_t slab, In& d) {
    const GT* gsb = G + slab;
    const XT* xsb = X + slab;
    const YT* ysb = Y + slab;
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      const int i = 16 * I + r;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const uint32_t lo = (uint32_t)(i * C + 32 * g + 8 * q);
        if (FULL || i < n) {
          d.g[I][g].load(at(gsb, lo));
          d.x[I][g].load(at(xsb, lo));
        } else {
          d.g[I][g].zero();
          d.x[I][g].zero();
        }
        if (hasy && (FULL || i < n)) d.y[I][g].load(at(ysb, lo));
        else d.y[I][g].zero();
      }
    }
  };
  // The next item's loads go into the same registers once this item's G, X
  // and Y are consumed (after S and the LDS staging), before this item's dx
  // stores (a vmcnt wait counts stores too).  The last item reloads itself.
  In d;
  SlabWalk w((int64_t)blockIdx.x * kMxWaves + wave, stride, items, nslabs, nC);
  // the first item's loads are waited for before the loop (see the forward)
  if (w.valid()) load(w.off(), d);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  for (; w.valid(); w.advance()) {
    const int64_t slab = w.off();
    float gv[2][2][8];
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) gv[I][g][e] = d.g[I][g].get(e);
    // Yd partials and dy = p G
#pragma unroll
    for (int I = 0; I < 2; ++I) {
      const int i = 16 * I + r;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
#pragma unroll
        for (int e = 0; e < 8; ++e) yd[I] = fmaf(gv[I][g][e], d.y[I][g].get(e), yd[I]);
        if (hasdy && (FULL || i < n)) {
          float o[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = pr[I] * gv[I][g][e];
          store_vec<YT, 8>(at(DY + slab, (uint32_t)(i * C + 32 * g + 8 * q)), o);
        }
      }
    }
    // S += G X^T: row block I (g rows), column block J (x rows), K = channels
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int I = 0; I < 2; ++I)
#pragma unroll
          for (int J = 0; J < 2; ++J) sacc[I][J] = mfma4(gv[I][g][e], d.x[J][g].get(e), sacc[I][J]);
    // stage G (one LDS row per stream), read back as streams 4m + q, channels 4r .. 4r+3
#pragma unroll
    for (int I = 0; I < 2; ++I)
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        float* dst = gs + (16 * I + r) * kMxPitch + 32 * g + 8 * q;
        *reinterpret_cast<float4*>(dst) = make_float4(gv[I][g][0], gv[I][g][1], gv[I][g][2], gv[I][g][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(gv[I][g][4], gv[I][g][5], gv[I][g][6], gv[I][g][7]);
      }
    load(w.next_off(), d);
    issue_fence();
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __builtin_amdgcn_wave_barrier();
    float gb[8][4];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const float4 u = *reinterpret_cast<const float4*>(gs + (4 * m + q) * kMxPitch + 4 * r);
      gb[m][0] = u.x; gb[m][1] = u.y; gb[m][2] = u.z; gb[m][3] = u.w;
    }
    // dx = Mf^T G: rows 16J + 4q + k, channels 4r + v
#pragma unroll
    for (int J = 0; J < 2; ++J) {
      float o[4][4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 8; ++m) acc = mfma4(amt[J][m], gb[m][v], acc);
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k][v] = acc[k];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = 16 * J + 4 * q + k;
        if (FULL || j < n) store_vec<XT, 4>(at(DX + slab, (uint32_t)(j * C + 4 * r)), o[k]);
      }
    }
    // the next item's LDS writes come after these reads in program order
    __builtin_amdgcn_wave_barrier();
  }

  // ---- the workgroup's partial row: [S n*n | Yd n | zero pad]
  // Yd of stream 16I + r: the four lane groups q hold parts of it
#pragma unroll
  for (int I = 0; I < 2; ++I) yd[I] = strided_sum<16, 64>(yd[I]);
  __syncthreads();
  float* red = &s_g[0][0];  // [wave][32*32 + 32]
  float* mine = red + wave * (32 * 32 + 32);
#pragma unroll
  for (int I = 0; I < 2; ++I)
#pragma unroll
    for (int J = 0; J < 2; ++J)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float v = sacc[I][J][k];
        mine[(16 * I + 4 * q + k) * 32 + 16 * J + r] = v;
      }
  if (q == 0) {
    mine[32 * 32 + r] = yd[0];
    mine[32 * 32 + 16 + r] = yd[1];
  }
  __syncthreads();
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  for (int k = threadIdx.x; k < A.P; k += blockDim.x) {
    int src = -1;
    if (k < n * n) src = (k / n) * 32 + (k % n);
    else if (k < n * n + n) src = 32 * 32 + (k - n * n);
    float s = 0.0f;
    if (src >= 0)
      for (int w = 0; w < kMxWaves; ++w) s += red[w * (32 * 32 + 32) + src];
    prow[k] = s;
  }
}

// ---------------------------------------------------------------------------
// 32 < n <= 64: the same contractions over 64 streams (zero past n).
//
// Forward: per item the lane loads streams 4m + q (m = 0..15) of channels
// [4r, 4r + 4) and the y of its output rows; each of the four 16-row blocks
// I of Mf X is, per channel column v, 16 chained MFMAs whose A operand (Mf
// row 16I + r at streams 4m + q) is read from LDS, staged once per
// workgroup as one float4 per (I, m / 4, lane) so that the wave reads
// consecutive 16 bytes per lane.  Each block's rows are stored before the
// next block is formed.
//
// Backward: per item and 32-channel half g, the lane loads G, X and Y of
// streams 16I + r (I = 0..3), channels 32g + 8q .. +8 (the channel-contraction
// layout of the n <= 32 kernel): Yd, dy = p G and S += G X^T (16 blocks of
// 16 x 16 in registers across the wave's items).  For dx = Mf^T G the lane
// then reads G again in the stream-contraction layout (streams 4m + q,
// channels 4r .. 4r + 3; from the caches, the item was just read) with Mf^T
// staged like the forward's A operand.  At the end the waves' S and Yd are
// added in wave order through LDS into the workgroup's partial row.
// ---------------------------------------------------------------------------

constexpr int kMx64Par = 64 * 64 + 64;

// Mf (row-block layout for the forward, column-block layout for the backward) and p into LDS:
// fw[(I * 4 + j) * 64 + lane] = Mf[16I + r][4(4j + t) + q] (t = 0..3), bw the same with Mf^T.
MHC_DEV void mx64_stage(float4* fw, float4* bw, float* s_p, const Mix32Args& A) {
  const int n = A.n;
  auto act_a = [&](int j) {
    if (A.h_mode == MHC_H_NONE) return 1.0f;
    return A.h_mode == MHC_H_RAW ? sigmoidf_(A.hpre[j]) : A.hpre[j];
  };
  auto act_p = [&](int i) {
    if (A.h_mode == MHC_H_NONE) return 1.0f;
    return A.h_mode == MHC_H_RAW ? 2.0f * sigmoidf_(A.hpost[i]) : A.hpost[i];
  };
  auto mf = [&](int i, int j) { return (i < n && j < n) ? act_p(i) * A.M[i * n + j] * act_a(j) : 0.0f; };
  for (int idx = threadIdx.x; idx < 16 * 64; idx += blockDim.x) {
    const int blk = idx >> 6, ln = idx & 63;  // blk = I * 4 + j
    const int I = blk >> 2, j = blk & 3, q = ln >> 4, r = ln & 15;
    float a[4], b[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int st = 4 * (4 * j + t) + q;
      a[t] = mf(16 * I + r, st);
      b[t] = mf(st, 16 * I + r);
    }
    if (fw != nullptr) fw[idx] = make_float4(a[0], a[1], a[2], a[3]);
    if (bw != nullptr) bw[idx] = make_float4(b[0], b[1], b[2], b[3]);
  }
  for (int i = threadIdx.x; i < 64; i += blockDim.x) s_p[i] = i < n ? act_p(i) : 0.0f;
}

// Token rows through buffer resources (one per tensor and item): the lane's
// 32-bit offset plus a uniform offset per row group.  With n == 64 (FULL)
// the row part goes in the uniform offset; below it the row part goes in the
// lane offset, which the range check covers, so rows past n read as zero and
// their stores are dropped (the resource spans the token's n rows).
constexpr int kMxRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor word 3 (raw, 32-bit data)

template <typename T>
MHC_DEV __amdgpu_buffer_rsrc_t mx_rsrc(const T* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), 0, (int)bytes, kMxRsrcWord3);
}

// four elements (16 or 8 bytes)
template <typename T>
MHC_DEV void mx_bload4(Vec<T, 4>& v, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  if constexpr (ElemTraits<T>::kBytes == 4) {
    const u32x4 u = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0);
    v.w[0] = u.x; v.w[1] = u.y; v.w[2] = u.z; v.w[3] = u.w;
  } else {
    const u32x2 u = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0);
    v.w[0] = u.x; v.w[1] = u.y;
  }
}

template <typename T>
MHC_DEV void mx_bstore4(const float (&o)[4], __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  if constexpr (ElemTraits<T>::kBytes == 4) {
    buf_store_b128<0>(u32x4{__builtin_bit_cast(uint32_t, o[0]), __builtin_bit_cast(uint32_t, o[1]),
                            __builtin_bit_cast(uint32_t, o[2]), __builtin_bit_cast(uint32_t, o[3])},
                      rs, voff, soff);
  } else {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack2<T>(o[0], o[1]), pack2<T>(o[2], o[3])}, rs, voff, soff, 0);
  }
}

// FULL: n == 64 and y present.
template <typename XT, typename YT, typename OT, bool FULL>
__global__ __launch_bounds__(kMxThreads) void mix64_fwd_kernel(Mix32Args A) {
  __shared__ float4 s_fw[16 * 64];
  __shared__ float s_p[64];
  mx64_stage(s_fw, nullptr, s_p, A);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 64 : A.n, C = A.C;
  const int nslabs = C / kMxSlab;
  const int64_t nC = (int64_t)n * C;
  constexpr uint32_t xs = sizeof(XT), ys = sizeof(YT), os = sizeof(OT);
  const bool hasy = FULL || A.y != nullptr;
  const int64_t items = A.T * nslabs;
  const int64_t stride = (int64_t)gridDim.x * kMxWaves;
  for (SlabWalk w((int64_t)blockIdx.x * kMxWaves + wave, stride, items, nslabs, nC); w.valid(); w.advance()) {
    const int64_t tok = w.t * nC;
    const uint32_t ch = (uint32_t)(w.s * kMxSlab);
    const auto rx = mx_rsrc((const XT*)A.x + tok, (uint32_t)(nC * xs));
    const auto ry = mx_rsrc((const YT*)A.y + tok, hasy ? (uint32_t)(nC * ys) : 0u);
    const auto ro = mx_rsrc((OT*)A.out + tok, (uint32_t)(nC * os));
    // x: streams 4m + q, channels ch + 4r .. +4
    Vec<XT, 4> x[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const uint32_t row = (uint32_t)((4 * m + (FULL ? 0 : q)) * C);
      mx_bload4(x[m], rx, (uint32_t)(((FULL ? q * C : 0) + 4 * r) * xs) + (FULL ? 0u : row * xs),
                (ch + (FULL ? row : 0u)) * xs);
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      // y of output rows 16I + 4q + k
      Vec<YT, 4> y[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t row = (uint32_t)((16 * I + (FULL ? 0 : 4 * q) + k) * C);
        if (hasy)
          mx_bload4(y[k], ry, (uint32_t)(((FULL ? 4 * q * C : 0) + 4 * r) * ys) + (FULL ? 0u : row * ys),
                    (ch + (FULL ? row : 0u)) * ys);
        else
          y[k].zero();
      }
      float am[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 u = s_fw[(I * 4 + j) * 64 + lane];
        am[4 * j] = u.x; am[4 * j + 1] = u.y; am[4 * j + 2] = u.z; am[4 * j + 3] = u.w;
      }
      float o[4][4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 16; ++m) acc = mfma4(am[m], x[m].get(v), acc);
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k][v] = fmaf(s_p[16 * I + 4 * q + k], y[k].get(v), acc[k]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t row = (uint32_t)((16 * I + (FULL ? 0 : 4 * q) + k) * C);
        mx_bstore4<OT>(o[k], ro, (uint32_t)(((FULL ? 4 * q * C : 0) + 4 * r) * os) + (FULL ? 0u : row * os),
                       (ch + (FULL ? row : 0u)) * os);
      }
    }
  }
}

// FULL: n == 64 with y and dy present (the only variant launched: below 64 the
// per-row lane offsets take more registers than the kernel has).
template <typename XT, typename YT, typename GT, bool FULL>
__global__ __launch_bounds__(kMxThreads) __attribute__((amdgpu_waves_per_eu(2)))
void mix64_bwd_kernel(Mix32Args A) {
  __shared__ float4 s_bw[16 * 64];
  __shared__ float s_p[64];
  __shared__ float s_red[kMx64Par];
  mx64_stage(nullptr, s_bw, s_p, A);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, r = lane & 15;
  const int n = FULL ? 64 : A.n, C = A.C;
  const int nslabs = C / kMxSlab;
  const int64_t nC = (int64_t)n * C;
  constexpr uint32_t xs = sizeof(XT), ys = sizeof(YT), gs = sizeof(GT);
  const bool hasy = FULL || A.y != nullptr, hasdy = FULL || A.dy != nullptr;
  float pr[4];
#pragma unroll
  for (int I = 0; I < 4; ++I) pr[I] = s_p[16 * I + r];

  f32x4 sacc[4][4];
#pragma unroll
  for (int I = 0; I < 4; ++I)
#pragma unroll
    for (int J = 0; J < 4; ++J) sacc[I][J] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float yd[4] = {0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t items = A.T * nslabs;
  const int64_t stride = (int64_t)gridDim.x * kMxWaves;
  for (SlabWalk w((int64_t)blockIdx.x * kMxWaves + wave, stride, items, nslabs, nC); w.valid(); w.advance()) {
    const int64_t tok = w.t * nC;
    const uint32_t ch = (uint32_t)(w.s * kMxSlab);
    const auto rg = mx_rsrc((const GT*)A.g + tok, (uint32_t)(nC * gs));
    const auto rx = mx_rsrc((const XT*)A.x + tok, (uint32_t)(nC * xs));
    const auto ry = mx_rsrc((const YT*)A.y + tok, hasy ? (uint32_t)(nC * ys) : 0u);
    const auto rdy = mx_rsrc((YT*)A.dy + tok, hasdy ? (uint32_t)(nC * ys) : 0u);
    const auto rdx = mx_rsrc((XT*)A.out + tok, (uint32_t)(nC * xs));
    // S, Yd, dy in quarters of 16 channels: streams 16I + r, channels ch + 16g + 4q .. +4
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      Vec<GT, 4> gg[4];
      Vec<XT, 4> xx[4];
      Vec<YT, 4> yy[4];
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const uint32_t row = (uint32_t)((16 * I + (FULL ? 0 : r)) * C);
        const uint32_t lo = (uint32_t)((FULL ? r * C : 0) + 4 * q), co = ch + 16 * g;
        mx_bload4(gg[I], rg, (lo + (FULL ? 0u : row)) * gs, (co + (FULL ? row : 0u)) * gs);
        mx_bload4(xx[I], rx, (lo + (FULL ? 0u : row)) * xs, (co + (FULL ? row : 0u)) * xs);
        if (hasy) mx_bload4(yy[I], ry, (lo + (FULL ? 0u : row)) * ys, (co + (FULL ? row : 0u)) * ys);
        else yy[I].zero();
      }
      float gv[4][4];
#pragma unroll
      for (int I = 0; I < 4; ++I)
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[I][e] = gg[I].get(e);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
#pragma unroll
        for (int e = 0; e < 4; ++e) yd[I] = fmaf(gv[I][e], yy[I].get(e), yd[I]);
        if (hasdy) {
          const uint32_t row = (uint32_t)((16 * I + (FULL ? 0 : r)) * C);
          const uint32_t lo = (uint32_t)((FULL ? r * C : 0) + 4 * q), co = ch + 16 * g;
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = pr[I] * gv[I][e];
          mx_bstore4<YT>(o, rdy, (lo + (FULL ? 0u : row)) * ys, (co + (FULL ? row : 0u)) * ys);
        }
      }
      // S += G X^T: row block I (g rows), column block J (x rows), K = the four lane groups' channels
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int I = 0; I < 4; ++I)
#pragma unroll
          for (int J = 0; J < 4; ++J) sacc[I][J] = mfma4(gv[I][e], xx[J].get(e), sacc[I][J]);
    }
    // dx = Mf^T G: G again as streams 4m + q, channels ch + 4r .. +4 (from the caches)
    Vec<GT, 4> gb[16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const uint32_t row = (uint32_t)((4 * m + (FULL ? 0 : q)) * C);
      mx_bload4(gb[m], rg, (uint32_t)(((FULL ? q * C : 0) + 4 * r) * gs) + (FULL ? 0u : row * gs),
                (ch + (FULL ? row : 0u)) * gs);
    }
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      float amt[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 u = s_bw[(J * 4 + j) * 64 + lane];
        amt[4 * j] = u.x; amt[4 * j + 1] = u.y; amt[4 * j + 2] = u.z; amt[4 * j + 3] = u.w;
      }
      float o[4][4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 16; ++m) acc = mfma4(amt[m], gb[m].get(v), acc);
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k][v] = acc[k];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t row = (uint32_t)((16 * J + (FULL ? 0 : 4 * q) + k) * C);
        mx_bstore4<XT>(o[k], rdx, (uint32_t)(((FULL ? 4 * q * C : 0) + 4 * r) * xs) + (FULL ? 0u : row * xs),
                       (ch + (FULL ? row : 0u)) * xs);
      }
    }
  }

  // ---- the workgroup's partial row [S n*n | Yd n | zero pad]: the waves' sums added in wave order
#pragma unroll
  for (int I = 0; I < 4; ++I) yd[I] = strided_sum<16, 64>(yd[I]);
  const int nwaves = blockDim.x >> 6;
  for (int wv = 0; wv < nwaves; ++wv) {
    if (wave == wv) {
#pragma unroll
      for (int I = 0; I < 4; ++I)
#pragma unroll
        for (int J = 0; J < 4; ++J)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const int idx = (16 * I + 4 * q + k) * 64 + 16 * J + r;
            s_red[idx] = wv == 0 ? sacc[I][J][k] : s_red[idx] + sacc[I][J][k];
          }
      if (q == 0) {
#pragma unroll
        for (int I = 0; I < 4; ++I) {
          const int idx = 64 * 64 + 16 * I + r;
          s_red[idx] = wv == 0 ? yd[I] : s_red[idx] + yd[I];
        }
      }
    }
    __syncthreads();
  }
  float* prow = A.part + (int64_t)blockIdx.x * A.P;
  for (int k = threadIdx.x; k < A.P; k += blockDim.x) {
    float v = 0.0f;
    if (k < n * n) v = s_red[(k / n) * 64 + (k % n)];
    else if (k < n * n + n) v = s_red[64 * 64 + (k - n * n)];
    prow[k] = v;
  }
}

template <typename F>
int mx_by_dtype(int code, F&& f) {
  switch (code) {
    case MHC_DTYPE_F32: return f((float*)nullptr);
    case MHC_DTYPE_BF16: return f((__bf16*)nullptr);
    case MHC_DTYPE_F16: return f((_Float16*)nullptr);
    default: return 1;
  }
}

// second operand type: fp32 or the first one's
template <typename T1, typename F>
int mx_by_pair(int code, F&& f) {
  if (code == MHC_DTYPE_F32) return f((float*)nullptr);
  if ((code == MHC_DTYPE_BF16 && std::is_same<T1, __bf16>::value) ||
      (code == MHC_DTYPE_F16 && std::is_same<T1, _Float16>::value))
    return f((T1*)nullptr);
  return 1;
}

bool mx_covered(const Mix32Args& A, std::initializer_list<const void*> ptrs) {
  if (A.n <= 16 || A.n > 64 || A.C % kMxSlab != 0 || A.T < 1) return false;
  if (knob(kKnobMix32, 1) == 0) return false;
  for (const void* p : ptrs)
    if (p != nullptr && !aligned(p, 16)) return false;
  return true;
}

}  // namespace

int mix32_fwd(const Mix32Args& A, int x_dtype, int y_dtype, int out_dtype, hipStream_t s) {
  if (!mx_covered(A, {A.x, A.y, A.out})) return 1;
  const int64_t items = A.T * (A.C / kMxSlab);
  const int per_cu = knob(kKnobMixFwdGrid, 2);
  int64_t blocks = ceil_div(items, kMxWaves);
  if (per_cu > 0) blocks = std::min<int64_t>(blocks, (int64_t)device_cu_count() * per_cu);
  blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, kMaxGrid));
  return mx_by_dtype(x_dtype, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return mx_by_pair<XT>(y_dtype, [&](auto* yp) {
      using YT = std::remove_pointer_t<decltype(yp)>;
      return mx_by_pair<XT>(out_dtype, [&](auto* op) {
        using OT = std::remove_pointer_t<decltype(op)>;
        if (A.n > 32) {
          if (A.n == 64 && A.y)
            hipLaunchKernelGGL((mix64_fwd_kernel<XT, YT, OT, true>), dim3((unsigned)blocks), dim3(kMxThreads), 0, s, A);
          else
            hipLaunchKernelGGL((mix64_fwd_kernel<XT, YT, OT, false>), dim3((unsigned)blocks), dim3(kMxThreads), 0, s, A);
          MHC_CHECK_LAUNCH("mix64_fwd_kernel");
          return (int)MHC_OK;
        }
        if (A.n == 32 && A.y)
          hipLaunchKernelGGL((mix32_fwd_kernel<XT, YT, OT, true>), dim3((unsigned)blocks), dim3(kMxThreads), 0, s, A);
        else
          hipLaunchKernelGGL((mix32_fwd_kernel<XT, YT, OT, false>), dim3((unsigned)blocks), dim3(kMxThreads), 0, s, A);
        MHC_CHECK_LAUNCH("mix32_fwd_kernel");
        return (int)MHC_OK;
      });
    });
  });
}

int mix32_bwd(const Mix32Args& A, int x_dtype, int y_dtype, int g_dtype, int64_t gmax, hipStream_t s,
              int64_t* num_partials) {
  if (!mx_covered(A, {A.x, A.y, A.g, A.out, A.dy})) return 1;
  // 32 < n < 64 (rows in the lane offsets, more registers than the kernel has) and calls without y or dy
  // take the generic kernels
  if (A.n > 32 && !(A.n == 64 && A.y && A.dy)) return 1;
  const int64_t items = A.T * (A.C / kMxSlab);
  return mx_by_dtype(x_dtype, [&](auto* xp) {
    using XT = std::remove_pointer_t<decltype(xp)>;
    return mx_by_pair<XT>(y_dtype, [&](auto* yp) {
      using YT = std::remove_pointer_t<decltype(yp)>;
      return mx_by_pair<XT>(g_dtype, [&](auto* gp) {
        using GT = std::remove_pointer_t<decltype(gp)>;
        // one resident wave of workgroups (each ends in one partial row)
        const bool wide = A.n > 32;
        const bool full = A.n == (wide ? 64 : 32) && A.y && A.dy;
        const void* kfn = wide ? (const void*)mix64_bwd_kernel<XT, YT, GT, true>
                               : (full ? (const void*)mix32_bwd_kernel<XT, YT, GT, true>
                                       : (const void*)mix32_bwd_kernel<XT, YT, GT, false>);
        const int occ = occupancy_blocks(kfn, kMxThreads, 0);
        if (occ <= 0) return 1;
        const int per_cu = knob(kKnobMixBwdGrid, occ);
        int64_t blocks = ceil_div(items, kMxWaves);
        if (per_cu > 0) blocks = std::min<int64_t>(blocks, (int64_t)device_cu_count() * per_cu);
        blocks = std::max<int64_t>(1, std::min<int64_t>(blocks, gmax));
        if (wide) {
          hipLaunchKernelGGL((mix64_bwd_kernel<XT, YT, GT, true>), dim3((unsigned)blocks), dim3(kMxThreads), 0, s, A);
          MHC_CHECK_LAUNCH("mix64_bwd_kernel");
        } else if (full) {
          hipLaunchKernelGGL((mix32_bwd_kernel<XT, YT, GT, true>), dim3((unsigned)blocks), dim3(kMxThreads), 0, s, A);
          MHC_CHECK_LAUNCH("mix32_bwd_kernel");
        } else {
          hipLaunchKernelGGL((mix32_bwd_kernel<XT, YT, GT, false>), dim3((unsigned)blocks), dim3(kMxThreads), 0, s, A);
          MHC_CHECK_LAUNCH("mix32_bwd_kernel");
        }
        *num_partials = blocks;
        return (int)MHC_OK;
      });
    });
  });
}

}  // namespace mhc
