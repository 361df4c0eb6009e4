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

  // Vector load of V elements; p must be aligned to min(16, kBytes).
  MHC_DEV void load(const T* p) {
    const char* b = reinterpret_cast<const char*>(p);
    if constexpr (kBytes % 16 == 0) {
#pragma unroll
      for (int k = 0; k < kBytes / 16; ++k) {
        uint4 u = reinterpret_cast<const uint4*>(b)[k];
        w[4 * k + 0] = u.x; w[4 * k + 1] = u.y; w[4 * k + 2] = u.z; w[4 * k + 3] = u.w;
      }
    } else if constexpr (kBytes == 8) {
      uint2 u = *reinterpret_cast<const uint2*>(b);
      w[0] = u.x; w[1] = u.y;
    } else if constexpr (kBytes == 4) {
      w[0] = *reinterpret_cast<const uint32_t*>(b);
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

// Store V fp32 values as T; p aligned to min(16, V*sizeof(T)).
template <typename T, int V>
MHC_DEV void store_vec(T* p, const float (&v)[V]) {
  constexpr int kBytes = V * ElemTraits<T>::kBytes;
  char* b = reinterpret_cast<char*>(p);
  if constexpr (ElemTraits<T>::kBytes == 4) {
    if constexpr (kBytes % 16 == 0) {
#pragma unroll
      for (int k = 0; k < V / 4; ++k)
        reinterpret_cast<float4*>(b)[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    } else if constexpr (kBytes == 8) {
      *reinterpret_cast<float2*>(b) = make_float2(v[0], v[1]);
    } else {
      *reinterpret_cast<float*>(b) = v[0];
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
          reinterpret_cast<uint4*>(b)[k] = make_uint4(wd[4 * k], wd[4 * k + 1], wd[4 * k + 2], wd[4 * k + 3]);
      } else if constexpr (kBytes == 8) {
        *reinterpret_cast<uint2*>(b) = make_uint2(wd[0], wd[1]);
      } else {
        *reinterpret_cast<uint32_t*>(b) = wd[0];
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

// --------------------------------------------------------------------------
// wave64 reductions (butterflies: every lane ends with a bitwise-identical
// result because each pairwise add is commutative-symmetric)
// --------------------------------------------------------------------------

MHC_DEV float shfl_xor(float v, int m) { return __shfl_xor(v, m, kWave); }

// all-reduce (sum) across aligned groups of `Lanes` lanes, Lanes a power of 2
template <int Lanes>
MHC_DEV float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < Lanes; m <<= 1) v += shfl_xor(v, m);
  return v;
}

template <int Lanes>
MHC_DEV float group_max(float v) {
#pragma unroll
  for (int m = 1; m < Lanes; m <<= 1) v = fmaxf(v, shfl_xor(v, m));
  return v;
}

// all-reduce across lanes {l, l^Stride, l^2Stride, ...} up to Span lanes
template <int Stride, int Span>
MHC_DEV float strided_sum(float v) {
#pragma unroll
  for (int m = Stride; m < Span; m <<= 1) v += shfl_xor(v, m);
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
      const float keep = upper ? v[k + half] : v[k];
      const float send = upper ? v[k] : v[k + half];
      v[k] = keep + shfl_xor(send, m);
    }
  }
}

// --------------------------------------------------------------------------
// math
// --------------------------------------------------------------------------

// reference.py:53-54 activations
MHC_DEV float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

}  // namespace mhc
