// RoPE arithmetic shared by the RoPE kernels and the decode kernel that rotates
// its query rows and the new key rows in registers:
//
//   out[d]        = r(x[d]        * cos[d]) + r(-x[d + D/2] * sin[d])
//   out[d + D/2]  = r(x[d + D/2]  * cos[d]) + r( x[d]       * sin[d])      (d < D/2)
//
// every product rounded to the element type before the add, as
// tokserve/kernels/_triton_rope.py:63-66 and apply_rope
// (tokserve/engine/rope.py:150-153) do; the sums are rounded where they are stored.
#pragma once

#include "common.hpp"

namespace tks {

// o1 (dims d..d+V) and o2 (dims d+D/2..) from x1 = x[d..], x2 = x[d+D/2..].
template <typename T, int V>
__device__ __forceinline__ void rotate_math(const float *x1, const float *x2, const float *c,
                                            const float *s, float *o1, float *o2) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const float a1 = round_through<T>(x1[j] * c[j]);
    const float b1 = round_through<T>(-x2[j] * s[j]);
    const float a2 = round_through<T>(x2[j] * c[j]);
    const float b2 = round_through<T>(x1[j] * s[j]);
    o1[j] = a1 + b1;
    o2[j] = a2 + b2;
  }
}

// Rotates one chunk pair of x into o1 (dims c..c+V) and o2 (dims c+D/2..).
template <typename T, int V>
__device__ __forceinline__ void rotate_values(const T *x, const float *c, const float *s,
                                              int half, float *o1, float *o2) {
  float x1[V], x2[V];
  if constexpr (V * sizeof(T) == 16) {
    unpack<T>(ld16(x), x1);
    unpack<T>(ld16(x + half), x2);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      x1[j] = to_float(x[j]);
      x2[j] = to_float(x[half + j]);
    }
  }
  rotate_math<T, V>(x1, x2, c, s, o1, o2);
}

template <typename T, int V>
__device__ __forceinline__ void store_pair(T *y, const float *o1, const float *o2, int half) {
  if constexpr (V * sizeof(T) == 16) {
    st16(y, pack<T>(o1));
    st16(y + half, pack<T>(o2));
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      y[j] = from_float<T>(o1[j]);
      y[half + j] = from_float<T>(o2[j]);
    }
  }
}

template <typename T, int V>
__device__ __forceinline__ void load_table(const T *crow, const T *srow, int c, float *cf,
                                           float *sf) {
  if constexpr (V * sizeof(T) == 16) {
    unpack<T>(ld16(crow + c), cf);
    unpack<T>(ld16(srow + c), sf);
  } else {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      cf[j] = to_float(crow[c + j]);
      sf[j] = to_float(srow[c + j]);
    }
  }
}

}  // namespace tks
