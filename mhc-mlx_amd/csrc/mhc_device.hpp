// Device-side building blocks shared by the mHC kernels (gfx950 / CDNA4).
//
// Everything here is wave64-specific: reductions are butterflies over 64
// lanes, element tiles are loaded with the widest naturally aligned global
// load (16 B where the channel vector allows it), and 16-bit element tiles are
// kept packed two-per-VGPR until they are needed in fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MHC_DEV __device__ __forceinline__

namespace mhc {

constexpr int kWave = 64;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

// Element type codes shared with the C ABI (include/mhc_hip.h).
enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

// --------------------------------------------------------------------------
// scalar conversions
// --------------------------------------------------------------------------

template <typename T> struct ElemTraits;
template <> struct ElemTraits<float> { static constexpr int kBytes = 4; };
template <> struct ElemTraits<__bf16> { static constexpr int kBytes = 2; };
template <> struct ElemTraits<_Float16> { static constexpr int kBytes = 2; };

// low / high 16-bit element of a packed word, as fp32
template <typename T> MHC_DEV float lo16(uint32_t w);
template <typename T> MHC_DEV float hi16(uint32_t w);
template <> MHC_DEV float lo16<__bf16>(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
template <> MHC_DEV float hi16<__bf16>(uint32_t w) { return __builtin_bit_cast(float, w & 0xFFFF0000u); }
template <> MHC_DEV float lo16<_Float16>(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
template <> MHC_DEV float hi16<_Float16>(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// pack two fp32 values into one word of two 16-bit elements (RNE)
template <typename T> MHC_DEV uint32_t pack2(float a, float b);
template <> MHC_DEV uint32_t pack2<__bf16>(float a, float b) {
  f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
template <> MHC_DEV uint32_t pack2<_Float16>(float a, float b) {
  f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

template <typename T> MHC_DEV float load1(const T* p);
template <> MHC_DEV float load1<float>(const float* p) { return *p; }
template <> MHC_DEV float load1<__bf16>(const __bf16* p) {
  return __builtin_bit_cast(float, (uint32_t)(*reinterpret_cast<const uint16_t*>(p)) << 16);
}
template <> MHC_DEV float load1<_Float16>(const _Float16* p) { return (float)*p; }

template <typename T> MHC_DEV void store1(T* p, float v);
template <> MHC_DEV void store1<float>(float* p, float v) { *p = v; }
template <> MHC_DEV void store1<__bf16>(__bf16* p, float v) { *p = (__bf16)v; }
template <> MHC_DEV void store1<_Float16>(_Float16* p, float v) { *p = (_Float16)v; }

// --------------------------------------------------------------------------
// Vec<T, V>: V consecutive channels of one stream, raw (packed) storage
// --------------------------------------------------------------------------

template <typename T, int V>
struct Vec {
  static constexpr int kBytes = V * ElemTraits<T>::kBytes;
  static constexpr int kWords = (kBytes + 3) / 4;
  uint32_t w[kWords];

  MHC_DEV void zero() {
#pragma unroll
    for (int k = 0; k < kWords; ++k) w[k] = 0u;
  }

  // element k as fp32
  MHC_DEV float get(int k) const {
    if constexpr (ElemTraits<T>::kBytes == 4) {
      return __builtin_bit_cast(float, w[k]);
    } else {
      return (k & 1) ? hi16<T>(w[k >> 1]) : lo16<T>(w[k >> 1]);
    }
  }

  // Vector load of V elements; p must be aligned to min(16, kBytes).  The
  // activations are streamed once, so loads of up to 16 bytes per lane carry
  // the non-temporal hint.  Wider ones (a lane's 32 bytes as two 16-byte
  // loads, so each instruction reads every other 16 bytes of the wave's
  // span) stay cached: with the hint that pattern streams at 48% of HBM peak
  // on gfx950, without it at 72% (1 GiB copy, read and write).  NT = false
  // drops the hint for data that is read again soon.
  template <bool NT = true>
  MHC_DEV void load(const T* p) {
    const char* b = reinterpret_cast<const char*>(p);
    if constexpr (kBytes % 16 == 0) {
#pragma unroll
      for (int k = 0; k < kBytes / 16; ++k) {
        const u32x4* a = reinterpret_cast<const u32x4*>(b) + k;
        u32x4 u;
        if constexpr (kBytes == 16 && NT) u = __builtin_nontemporal_load(a);
        else u = *a;
        w[4 * k + 0] = u.x; w[4 * k + 1] = u.y; w[4 * k + 2] = u.z; w[4 * k + 3] = u.w;
      }
    } else if constexpr (kBytes == 8) {
      const u32x2* a = reinterpret_cast<const u32x2*>(b);
      const u32x2 u = NT ? __builtin_nontemporal_load(a) : *a;
      w[0] = u.x; w[1] = u.y;
    } else if constexpr (kBytes == 4) {
      const uint32_t* a = reinterpret_cast<const uint32_t*>(b);
      w[0] = NT ? __builtin_nontemporal_load(a) : *a;
    } else {
      static_assert(kBytes == 2, "unsupported vector width");
      w[0] = (uint32_t)(*reinterpret_cast<const uint16_t*>(b));
    }
  }

  // Element-wise load of the first `valid` elements (any alignment); rest zero.
  MHC_DEV void load_partial(const T* p, int valid) {
    zero();
    if constexpr (ElemTraits<T>::kBytes == 4) {
#pragma unroll
      for (int k = 0; k < V; ++k)
        if (k < valid) w[k] = __builtin_bit_cast(uint32_t, p[k]);
    } else {
      const uint16_t* q = reinterpret_cast<const uint16_t*>(p);
#pragma unroll
      for (int k = 0; k < V; ++k)
        if (k < valid) w[k >> 1] |= (uint32_t)q[k] << (16 * (k & 1));
    }
  }
};

// Non-temporal stores of whole 4 / 8 / 16-byte words.
MHC_DEV void st_nt(uint32_t* p, uint32_t a) { __builtin_nontemporal_store(a, p); }
MHC_DEV void st_nt(uint32_t* p, uint32_t a, uint32_t b) {
  const u32x2 v = {a, b};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p));
}
MHC_DEV void st_nt(uint32_t* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u32x4 v = {a, b, c, d};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// A 16-byte buffer store whose data registers are not written again until two
// wait states after it.  The compiler pads a VALU write of the registers of a
// store of more than 8 bytes (the store reads its data after it issues) only
// when the store's soffset is not an SGPR; on gfx950 an SGPR soffset is no
// exemption: with a second wave on the SIMD, lanes 12..15 of each 16-lane row
// stored the value that the next instruction wrote into the data registers.
// The s_nop reads the data registers, so they stay unwritten until it has
// issued; the scheduling barriers keep it right behind the store.
template <int AUX>
MHC_DEV void buf_store_b128(u32x4 v, __amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, voff, soff, AUX);
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 1" ::"v"(v));
  __builtin_amdgcn_sched_barrier(0);
}

// A 16-byte word: non-temporal when the lane's whole span is this word,
// cached when it is part of a wider span (see Vec::load).
template <bool NT>
MHC_DEV void st16(uint32_t* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  if constexpr (NT) {
    st_nt(p, a, b, c, d);
  } else {
    const u32x4 v = {a, b, c, d};
    *reinterpret_cast<u32x4*>(p) = v;
  }
}

// Store V fp32 values as T; p aligned to min(16, V*sizeof(T)).  Streamed
// outputs, so stores of up to 16 bytes per lane carry the non-temporal hint;
// wider ones too when NT_WIDE (a kernel where that output is a small share
// of the traffic: residual_add_agg's fp32 y_agg runs 645 us with the hint,
// 663 us without, at 32768 x 4 x 4096).
template <typename T, int V, bool NT_WIDE = false>
MHC_DEV void store_vec(T* p, const float (&v)[V]) {
  constexpr int kBytes = V * ElemTraits<T>::kBytes;
  constexpr bool kNT = kBytes == 16 || NT_WIDE;
  uint32_t* b = reinterpret_cast<uint32_t*>(p);
  if constexpr (ElemTraits<T>::kBytes == 4) {
    if constexpr (kBytes % 16 == 0) {
#pragma unroll
      for (int k = 0; k < V / 4; ++k)
        st16<kNT>(b + 4 * k, __builtin_bit_cast(uint32_t, v[4 * k]),
                           __builtin_bit_cast(uint32_t, v[4 * k + 1]), __builtin_bit_cast(uint32_t, v[4 * k + 2]),
                           __builtin_bit_cast(uint32_t, v[4 * k + 3]));
    } else if constexpr (kBytes == 8) {
      st_nt(b, __builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]));
    } else {
      st_nt(b, __builtin_bit_cast(uint32_t, v[0]));
    }
  } else {
    if constexpr (V == 1) {
      store1<T>(p, v[0]);
    } else {
      uint32_t wd[V / 2];
#pragma unroll
      for (int k = 0; k < V / 2; ++k) wd[k] = pack2<T>(v[2 * k], v[2 * k + 1]);
      if constexpr (kBytes % 16 == 0) {
#pragma unroll
        for (int k = 0; k < kBytes / 16; ++k)
          st16<kNT>(b + 4 * k, wd[4 * k], wd[4 * k + 1], wd[4 * k + 2], wd[4 * k + 3]);
      } else if constexpr (kBytes == 8) {
        st_nt(b, wd[0], wd[1]);
      } else {
        st_nt(b, wd[0]);
      }
    }
  }
}

template <typename T, int V>
MHC_DEV void store_partial(T* p, const float (&v)[V], int valid) {
#pragma unroll
  for (int k = 0; k < V; ++k)
    if (k < valid) store1<T>(p + k, v[k]);
}

// Compiler-only fence: no instruction written before it is scheduled after
// it or the other way round (keeps a work item's loads issued together,
// ahead of the first wait, instead of interleaved with their uses).
MHC_DEV void issue_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// A value every lane of the wave holds equally, moved to a scalar register
// (parameters read by all lanes: one SGPR instead of one VGPR per value).
MHC_DEV float uniform_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// --------------------------------------------------------------------------
// wave64 reductions
//
// Steps inside a 16-lane DPP row use DPP lane permutes (no LDS traffic):
// quad_perm for lane^1 and lane^2, row_half_mirror (lane^7 within 8) and
// row_mirror (lane^15 within 16) once the lower bits are already reduced,
// row_ror:8 (== lane^8) and row_ror:4 (== lane^4 once bit 3 is reduced).
// Steps across rows (lane^16, lane^32) use ds_bpermute.  Every step adds
// the same pair of values on both partner lanes, so all lanes of a group end
// with bitwise-identical results.
// --------------------------------------------------------------------------

MHC_DEV float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }

// One all-reduce step across lane ^ 16 or lane ^ 32 on gfx950's permlane
// swaps (v_permlane16_swap / v_permlane32_swap: VALU, no LDS round trip as
// with ds_bpermute).  Swapping a value with itself leaves the lower and the
// upper member of each lane pair in the two results, in the same order on
// both lanes, so op(lo, hi) is bitwise the same on both partners (and equal
// to op(v, partner) for a commutative op).
template <int M, typename Op>
MHC_DEV float xor_allreduce(float v, Op op) {
  static_assert(M == 16 || M == 32, "permlane swaps exchange 16- or 32-lane halves");
  const unsigned u = __builtin_bit_cast(unsigned, v);
  unsigned lo, hi;
  if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    lo = r[0];  // vector elements copied to scalars before any bit cast
    hi = r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    lo = r[0];
    hi = r[1];
  }
  return op(__builtin_bit_cast(float, lo), __builtin_bit_cast(float, hi));
}

template <int CTRL>
MHC_DEV float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF,
                                                               false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane ^ 7 within 8
constexpr int kDppMirror = 0x140;     // lane ^ 15 within 16
constexpr int kDppRor4 = 0x124;       // row_ror:4
constexpr int kDppRor8 = 0x128;       // row_ror:8

struct SumOp {
  MHC_DEV float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  MHC_DEV float operator()(float a, float b) const { return fmaxf(a, b); }
};

// all-reduce across aligned groups of `Lanes` lanes, Lanes a power of 2
template <int Lanes, typename Op>
MHC_DEV float group_reduce(float v, Op op) {
  if constexpr (Lanes >= 2) v = op(v, dpp_mov<kDppXor1>(v));
  if constexpr (Lanes >= 4) v = op(v, dpp_mov<kDppXor2>(v));
  if constexpr (Lanes >= 8) v = op(v, dpp_mov<kDppHalfMirror>(v));
  if constexpr (Lanes >= 16) v = op(v, dpp_mov<kDppMirror>(v));
  // (ds_bpermute here: the permlane form below made the n = 4 forward, whose
  // per-token wave_sum sits on every workgroup's path, 5% slower)
  if constexpr (Lanes >= 32) v = op(v, shfl_xor(v, 16));
  if constexpr (Lanes >= 64) v = op(v, shfl_xor(v, 32));
  return v;
}

template <int Lanes>
MHC_DEV float group_sum(float v) { return group_reduce<Lanes>(v, SumOp{}); }

template <int Lanes>
MHC_DEV float group_max(float v) { return group_reduce<Lanes>(v, MaxOp{}); }

// all-reduce (sum) across lanes {l, l^Stride, l^2Stride, ...} up to Span lanes
template <int Stride, int Span>
MHC_DEV float strided_sum(float v) {
  if constexpr (Stride <= 1 && Span >= 2) v += dpp_mov<kDppXor1>(v);
  if constexpr (Stride <= 2 && Span >= 4) v += dpp_mov<kDppXor2>(v);
  if constexpr (Stride <= 4 && Span >= 16) {
    v += dpp_mov<kDppRor8>(v);  // lane ^ 8
    v += dpp_mov<kDppRor4>(v);  // lane ^ 4 (bit 3 already reduced)
  } else if constexpr (Stride == 8 && Span >= 16) {
    v += dpp_mov<kDppRor8>(v);
  } else if constexpr (Stride <= 4 && Span == 8) {
    v += shfl_xor(v, 4);
  }
  if constexpr (Stride <= 16 && Span >= 32) v = xor_allreduce<16>(v, SumOp{});
  if constexpr (Stride <= 32 && Span >= 64) v = xor_allreduce<32>(v, SumOp{});
  return v;
}

MHC_DEV float wave_sum(float v) { return group_sum<kWave>(v); }

// Butterfly reduce-scatter of 64*R values per lane: afterwards v[0..R) of
// lane L holds the wave-wide sum of original entries [L*R, L*R + R).
template <int R>
MHC_DEV void wave_reduce_scatter(float (&v)[64 * R], int lane) {
#pragma unroll
  for (int s = 0; s < 6; ++s) {
    const int m = 32 >> s;
    const int half = (64 * R) >> (s + 1);
    const bool upper = (lane & m) != 0;
#pragma unroll
    for (int k = 0; k < half; ++k) {
      // select values, not array elements: `upper ? v[a] : v[b]` is an
      // lvalue, which the compiler may turn into a select of addresses and
      // move v to scratch memory
      const float lo = v[k], hi = v[k + half];
      const float keep = upper ? hi : lo;
      const float send = upper ? lo : hi;
      v[k] = keep + shfl_xor(send, m);
    }
  }
}

// --------------------------------------------------------------------------
// synchronisation
// --------------------------------------------------------------------------

// s_waitcnt immediate for lgkmcnt(0) alone (gfx9 encoding: vmcnt[3:0] |
// expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]; vmcnt and expcnt left
// at their maximum).
constexpr int kWaitLgkm0 = 0xC07F;
// s_waitcnt immediate for vmcnt(0) alone.
constexpr int kWaitVm0 = 0x0F70;

// Workgroup barrier for data exchanged through LDS only.  __syncthreads()
// is a workgroup-scope release/acquire fence and waits for every
// outstanding global access as well (for instance the previous token's
// output stores); here only LDS traffic has to be complete.
MHC_DEV void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// --------------------------------------------------------------------------
// MFMA (v_mfma_f32_16x16x16 bf16 / fp16: exact 16-bit products, fp32
// accumulation).  Operand layout for lane l (r = l & 15, q = l >> 4):
//   A: row r, k = 4q .. 4q+3        B: column r, k = 4q .. 4q+3
//   D: rows 4q .. 4q+3 of column r (acc[0..3])
// Each uint2 operand holds four 16-bit elements, k ascending from the low
// half of .x.
// --------------------------------------------------------------------------

template <typename T>
MHC_DEV f32x4 mfma16(uint2 a, uint2 b, f32x4 c);
template <>
MHC_DEV f32x4 mfma16<__bf16>(uint2 a, uint2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                   0, 0, 0);
}
template <>
MHC_DEV f32x4 mfma16<_Float16>(uint2 a, uint2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0,
                                               0, 0);
}

// 16-bit bit pattern of v rounded to T (RNE) and back.
template <typename T> MHC_DEV uint32_t bits16(float v);
template <> MHC_DEV uint32_t bits16<__bf16>(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }
template <> MHC_DEV uint32_t bits16<_Float16>(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }
template <typename T> MHC_DEV float from16(uint32_t b) { return lo16<T>(b); }

// fp32 v as three 16-bit terms h[0] + h[1] + h[2] (each the RNE rounding of
// the remainder left by the previous ones).  For bf16 the sum is exactly v
// (3 x 8 significant bits cover fp32's 24; bf16 shares fp32's exponent
// range); for fp16 the remainder after three terms is below 2^-33 |v| (plus
// fp16's 2^-24 underflow step), far inside fp32 rounding of a 16-term dot
// product.  An MFMA over the three terms against 16-bit data therefore forms
// the fp32 product of v with that data.
template <typename T>
MHC_DEV void split3(float v, uint32_t (&h)[3]) {
  h[0] = bits16<T>(v);
  const float r1 = v - from16<T>(h[0]);
  h[1] = bits16<T>(r1);
  const float r2 = r1 - from16<T>(h[1]);
  h[2] = bits16<T>(r2);
}

// split3 of four values as the three packed MFMA operands (terms e of
// v[0..3], v[0] in the low half of .x): the same terms as split3, two values
// per conversion instruction.
template <typename T>
MHC_DEV void split3x4(const float (&v)[4], uint2 (&out)[3]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float a = v[2 * h], b = v[2 * h + 1];
    uint32_t w[3];
#pragma unroll
    for (int e = 0; e < 3; ++e) {
      w[e] = pack2<T>(a, b);
      a -= lo16<T>(w[e]);
      b -= hi16<T>(w[e]);
    }
#pragma unroll
    for (int e = 0; e < 3; ++e) (h == 0 ? out[e].x : out[e].y) = w[e];
  }
}

// Two packed words of 16-bit elements -> one word of their low (high)
// halves, a's in the low half: element v of four streams becomes an MFMA
// operand without leaving registers.
template <typename XT>
MHC_DEV uint32_t pack_lo16(uint32_t a, uint32_t b) { return (a & 0xFFFFu) | (b << 16); }
template <typename XT>
MHC_DEV uint32_t pack_hi16(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xFFFF0000u); }

// --------------------------------------------------------------------------
// math
// --------------------------------------------------------------------------

// reference.py:53-54 activations
MHC_DEV float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

// The same from the hardware exp2 and reciprocal (v_exp_f32, v_rcp_f32, each
// within 1 ulp; the exponent is rounded once after scaling by log2 e):
// relative error within a few 1e-7 over |z| <= 30 and exact limits 0 / 1
// beyond.  For kernels that evaluate activations per token and lane.
MHC_DEV float sigmoid_fast(float z) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z * 1.4426950408889634f));
}

}  // namespace mhc
