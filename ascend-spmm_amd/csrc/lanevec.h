// Per-lane vector helpers shared by the CSR gather kernel and the vector part
// of the block kernel.  Both paths accumulate a row with exactly this code, so
// a row computes the same fp32 sequence whichever kernel owns it.
#pragma once

#include "common.h"

namespace spmm {
namespace lanes {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

typedef unsigned int raw16_t __attribute__((ext_vector_type(4)));

// Raw 16-byte load (converted later, so the load can be issued early).
template <typename T>
__device__ inline raw16_t load_raw16(const T* p) {
  return *reinterpret_cast<const raw16_t*>(p);
}

// Elements per lane: 16 bytes of the value type.  store() writes output rows
// with non-temporal (streaming) stores: no kernel re-reads them, and on
// MI355X this took 2-6% off the gather-bound configurations (config 4 at
// N=512: 178 -> 167 us) by keeping the output out of the caches the gathers
// use.
template <typename T> struct LaneVec;
template <> struct LaneVec<_Float16> {
  static constexpr int V = 8;
  __device__ static inline void unpack(const raw16_t& r, float* f) {
    half8_t h = __builtin_bit_cast(half8_t, r);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = static_cast<float>(h[i]);
  }
  __device__ static inline void load(const _Float16* p, float* f) {
    half8_t h = *reinterpret_cast<const half8_t*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = static_cast<float>(h[i]);
  }
  __device__ static inline void store(_Float16* p, const float* f) {
    half8_t h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = static_cast<_Float16>(f[i]);
    __builtin_nontemporal_store(__builtin_bit_cast(raw16_t, h), reinterpret_cast<raw16_t*>(p));
  }
};
template <> struct LaneVec<float> {
  static constexpr int V = 4;
  __device__ static inline void unpack(const raw16_t& r, float* f) {
    float4_t v = __builtin_bit_cast(float4_t, r);
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = v[i];
  }
  __device__ static inline void load(const float* p, float* f) {
    float4_t v = *reinterpret_cast<const float4_t*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = v[i];
  }
  __device__ static inline void store(float* p, const float* f) {
    float4_t v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = f[i];
    __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(p));
  }
};

__device__ inline int64_t clampi(int64_t x, int64_t lo, int64_t hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// acc[0..V) += sum_{p in [a, b)} value[p] * dense[col[p], c0 .. c0+V), in order.
template <typename T, typename I>
__device__ inline void accumulate(float* acc, int64_t a, int64_t b, const I* __restrict__ col,
                                  const T* __restrict__ value, const T* __restrict__ dense,
                                  int64_t K, int64_t N, int64_t c0) {
  constexpr int V = LaneVec<T>::V;
  int64_t p = a;
  for (; p + 4 <= b; p += 4) {
    int64_t c[4];
    float v[4];
    float x[4][V];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      c[u] = static_cast<int64_t>(col[p + u]);
      v[u] = static_cast<float>(value[p + u]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (static_cast<uint64_t>(c[u]) < static_cast<uint64_t>(K)) {
        LaneVec<T>::load(dense + c[u] * N + c0, x[u]);
      } else {
#pragma unroll
        for (int i = 0; i < V; ++i) x[u][i] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (static_cast<uint64_t>(c[u]) < static_cast<uint64_t>(K)) {
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = __builtin_fmaf(v[u], x[u][i], acc[i]);
      }
    }
  }
  for (; p < b; ++p) {
    const int64_t cc = static_cast<int64_t>(col[p]);
    if (static_cast<uint64_t>(cc) < static_cast<uint64_t>(K)) {
      const float vv = static_cast<float>(value[p]);
      float x[V];
      LaneVec<T>::load(dense + cc * N + c0, x);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = __builtin_fmaf(vv, x[i], acc[i]);
    }
  }
}

}  // namespace lanes
}  // namespace spmm
