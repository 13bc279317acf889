// Shared device helpers for the gfx950 kernels: element conversions with
// torch's rounding (round-to-nearest-even, canonical NaN), 16-byte vector
// access, wave64 DPP reductions and the status plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tokserve_hip.h"

namespace tks {

// ---------------------------------------------------------------- status ---

// Records the HIP error of the last failing launch for tks_last_hip_error().
void set_hip_error(hipError_t err);

inline int32_t check_launch() {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_hip_error(err);
    return TKS_ERR_LAUNCH;
  }
  return TKS_OK;
}

inline bool valid_dtype(int32_t dtype) {
  return dtype == TKS_FLOAT32 || dtype == TKS_FLOAT16 || dtype == TKS_BFLOAT16;
}

inline int elem_bytes(int32_t dtype) { return dtype == TKS_FLOAT32 ? 4 : 2; }

// A pool scale must be a positive finite float.
inline bool valid_scale(float s) { return s > 0.f && s <= 3.4028234663852886e38f; }

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------ elements ---

struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float to_float(float x) { return x; }
__device__ __forceinline__ float to_float(_Float16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_float(bf16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x.bits) << 16);
}

// Round-to-nearest-even float -> bfloat16 (the rounding c10::BFloat16 uses), done
// by the hardware converter (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  const __bf16 h = static_cast<__bf16>(f);
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

template <typename T>
__device__ __forceinline__ T from_float(float f);
template <>
__device__ __forceinline__ float from_float<float>(float f) {
  return f;
}
template <>
__device__ __forceinline__ _Float16 from_float<_Float16>(float f) {
  return static_cast<_Float16>(f);
}
template <>
__device__ __forceinline__ bf16_t from_float<bf16_t>(float f) {
  return bf16_t{f32_to_bf16_bits(f)};
}

// The fp32 value as a register holds it. An empty asm the compiler cannot look
// through: a product computed before it is rounded to fp32 and cannot be fused
// with an fp16 conversion after it. (The compiler turns fp16(a * b) into one
// mixed-precision FMA, v_fma_mixlo_f16, which rounds the exact product to fp16
// once; that differs from rounding the fp32 product whenever the product is
// inexact in fp32, and #pragma clang fp contract(off) does not prevent it.)
__device__ __forceinline__ float fp32_value(float f) {
  __asm__("" : "+v"(f));
  return f;
}

// Round a float through T and back (the `.to(dtype)` of the torch path).
template <typename T>
__device__ __forceinline__ float round_through(float f) {
  return to_float(from_float<T>(f));
}

// Elements per 16-byte vector.
template <typename T>
struct Vec {
  static constexpr int N = 16 / sizeof(T);
};

// 16-byte vector load/store as four dwords.
__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }
// Non-temporal 16-byte load (cache lines marked stream-once) for data read
// exactly once per launch, such as K/V pages in decode.
__device__ __forceinline__ uint4 ld16_stream(const void *p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st16(void *p, uint4 v) { *reinterpret_cast<uint4 *>(p) = v; }

// Unpack the 16-byte vector `v` of T into floats.
template <typename T>
__device__ __forceinline__ void unpack(uint4 v, float *out);
template <>
__device__ __forceinline__ void unpack<float>(uint4 v, float *out) {
  out[0] = __uint_as_float(v.x);
  out[1] = __uint_as_float(v.y);
  out[2] = __uint_as_float(v.z);
  out[3] = __uint_as_float(v.w);
}
template <>
__device__ __forceinline__ void unpack<bf16_t>(uint4 v, float *out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void unpack<_Float16>(uint4 v, float *out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    _Float16 lo, hi;
    uint16_t l16 = static_cast<uint16_t>(w[i] & 0xffffu), h16 = static_cast<uint16_t>(w[i] >> 16);
    __builtin_memcpy(&lo, &l16, 2);
    __builtin_memcpy(&hi, &h16, 2);
    out[2 * i] = static_cast<float>(lo);
    out[2 * i + 1] = static_cast<float>(hi);
  }
}

// --------------------------------------------------------- fp8 (e4m3) ---
//
// OCP FP8 E4M3 (torch.float8_e4m3fn): sign, 4 exponent bits (bias 7), 3
// mantissa bits, subnormals, no infinities, NaN = S.1111.111, largest finite
// 448. Used only for K/V pools. Decoding is exact into f32, f16 and bf16;
// encoding (v_cvt_pk_fp8_f32) rounds to nearest even after the value is
// clamped to [-448, 448], and a NaN keeps its sign (fp8x4_nan_sign): the
// result of torch's x.clamp(-448, 448).to(torch.float8_e4m3fn).

struct fp8e4m3_t {
  uint8_t bits;
};
constexpr float kFp8Max = 448.f;

// Bytes 0, 1 (hi = false) or 2, 3 (hi = true) of w as floats.
__device__ __forceinline__ void fp8x2_to_float(uint32_t w, bool hi, float *out) {
#if __HIP_DEVICE_COMPILE__
  const auto f = hi ? __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true)
                    : __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  out[0] = f[0];
  out[1] = f[1];
#else
  (void)w; (void)hi; (void)out;
#endif
}

__device__ __forceinline__ void fp8x4_to_float(uint32_t w, float *out) {
  fp8x2_to_float(w, false, out);
  fp8x2_to_float(w, true, out + 2);
}

__device__ __forceinline__ float to_float(fp8e4m3_t x) {
  float f[2];
  fp8x2_to_float(x.bits, false, f);
  return f[0];
}

__device__ __forceinline__ float fp8_clamp(float x) {
  return x > kFp8Max ? kFp8Max : (x < -kFp8Max ? -kFp8Max : x);  // NaN compares false: kept
}

// Four floats -> four e4m3 bytes (element 0 in the low byte).
__device__ __forceinline__ uint32_t float4_to_fp8x4(float a, float b, float c, float d) {
#if __HIP_DEVICE_COMPILE__
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(a), fp8_clamp(b), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(fp8_clamp(c), fp8_clamp(d), w, true);
  return static_cast<uint32_t>(w);
#else
  (void)a; (void)b; (void)c; (void)d;
  return 0;
#endif
}

// The converter writes one NaN code whatever the input's sign; torch keeps the
// sign (S.1111.111). Rewrites the NaN bytes of w from the signs of the four
// source values x[0..3] (NaN before any scaling, so the sign is the input's).
__device__ __forceinline__ uint32_t fp8x4_nan_sign(uint32_t w, const float *x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t bits = __float_as_uint(x[i]);
    const bool nan = (bits & 0x7fffffffu) > 0x7f800000u;
    const uint32_t code = (bits >> 31) ? 0xffu : 0x7fu;
    w = nan ? ((w & ~(0xffu << (8 * i))) | (code << (8 * i))) : w;
  }
  return w;
}

template <>
__device__ __forceinline__ void unpack<fp8e4m3_t>(uint4 v, float *out) {
  fp8x4_to_float(v.x, out);
  fp8x4_to_float(v.y, out + 4);
  fp8x4_to_float(v.z, out + 8);
  fp8x4_to_float(v.w, out + 12);
}

// e4m3 codes of x[i] / scale for N values (a multiple of 4) already held at the row
// dtype's precision, four codes per word (element 0 in the low byte): the division in
// fp32, the clamp to +-448 and one rounding to e4m3, NaN keeping the sign of x.
template <int N>
__device__ __forceinline__ void e4m3_words(const float *x, float scale, uint32_t *w) {
  static_assert(N % 4 == 0, "whole e4m3 words");
#pragma unroll
  for (int i = 0; i < N / 4; ++i)
    w[i] = fp8x4_nan_sign(float4_to_fp8x4(x[4 * i] / scale, x[4 * i + 1] / scale,
                                          x[4 * i + 2] / scale, x[4 * i + 3] / scale),
                          x + 4 * i);
}

// The code of one such value.
__device__ __forceinline__ uint8_t e4m3_code(float x, float scale) {
  const float x4[4] = {x, 0.f, 0.f, 0.f};
  return static_cast<uint8_t>(fp8x4_nan_sign(float4_to_fp8x4(x / scale, 0.f, 0.f, 0.f), x4) &
                              0xffu);
}

// The same codes for N = 1, 4, 8 or 16 values stored to dst (N bytes; the 4-, 8- and
// 16-byte stores need that alignment).
template <int N>
__device__ __forceinline__ void encode_e4m3(const float *x, float scale, uint8_t *dst) {
  if constexpr (N == 1) {
    dst[0] = e4m3_code(x[0], scale);
  } else {
    static_assert(N == 4 || N == 8 || N == 16, "one 4-, 8- or 16-byte store");
    uint32_t w[N / 4];
    e4m3_words<N>(x, scale, w);
    if constexpr (N == 16) {
      st16(dst, make_uint4(w[0], w[1], w[2], w[3]));
    } else if constexpr (N == 8) {
      *reinterpret_cast<uint2 *>(dst) = make_uint2(w[0], w[1]);
    } else {
      *reinterpret_cast<uint32_t *>(dst) = w[0];
    }
  }
}

template <typename T>
__device__ __forceinline__ uint16_t bits16(T x) {
  uint16_t b;
  __builtin_memcpy(&b, &x, 2);
  return b;
}

// Pack floats (rounded to T) into a 16-byte vector.
template <typename T>
__device__ __forceinline__ uint4 pack(const float *in);
template <>
__device__ __forceinline__ uint4 pack<float>(const float *in) {
  return make_uint4(__float_as_uint(in[0]), __float_as_uint(in[1]), __float_as_uint(in[2]),
                    __float_as_uint(in[3]));
}
template <>
__device__ __forceinline__ uint4 pack<bf16_t>(const float *in) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = static_cast<uint32_t>(f32_to_bf16_bits(in[2 * i])) |
           (static_cast<uint32_t>(f32_to_bf16_bits(in[2 * i + 1])) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}
template <>
__device__ __forceinline__ uint4 pack<_Float16>(const float *in) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = static_cast<uint32_t>(bits16(static_cast<_Float16>(in[2 * i]))) |
           (static_cast<uint32_t>(bits16(static_cast<_Float16>(in[2 * i + 1]))) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// ------------------------------------------------------- wave reductions ---

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadSwap1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// All-reduce over the 16 lanes of a DPP row (lanes 16r .. 16r+15).
__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp<kDppQuadSwap1>(x));
  x = fmaxf(x, dpp<kDppQuadSwap2>(x));
  x = fmaxf(x, dpp<kDppHalfMirror>(x));
  x = fmaxf(x, dpp<kDppMirror>(x));
  return x;
}
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<kDppQuadSwap1>(x);
  x += dpp<kDppQuadSwap2>(x);
  x += dpp<kDppHalfMirror>(x);
  x += dpp<kDppMirror>(x);
  return x;
}

// All-reduce over the 64 lanes of a wave.
__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}
__device__ __forceinline__ float wave_max(float x) {
  x = row16_max(x);
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace tks
