/*
 * e4m3.c -- TEST INFRASTRUCTURE ONLY (the oracle's fp8 pool encoding).
 *
 * OCP 8-bit floating point, E4M3 variant (the OCP FP8 specification, v1.0,
 * 2023; torch.float8_e4m3fn): sign bit, 4 exponent bits with bias 7, 3
 * mantissa bits; exponent field 0 holds subnormals m * 2^-9; no infinities;
 * S.1111.111 is NaN; the largest finite magnitude is S.1111.110 = 448.
 * Written from the format's definition, independently of torch's converter,
 * to pin the torch-based restatement in oracle/paged.py.
 *
 * Encoding of a pool element (the build's own fp8 pool variant; the reference
 * keeps pools in the model dtype, tokserve/engine/paged/storage.py:40-56):
 *   code = e4m3(clamp(x / scale, -448, 448)), round to nearest, ties to even,
 *   NaN stays NaN (sign kept).
 */
#include <math.h>
#include <stdint.h>

float oracle_e4m3_decode(uint8_t code) {
  const int sign = code >> 7, e = (code >> 3) & 15, m = code & 7;
  float v;
  if (e == 15 && m == 7) return sign ? -NAN : NAN;
  if (e == 0)
    v = ldexpf((float)m, -9);
  else
    v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return sign ? -v : v;
}

/* Code of an exactly representable magnitude v in [0, 448]. */
static uint8_t encode_exact(float v) {
  if (v < 0x1p-6f) return (uint8_t)(v / 0x1p-9f); /* 0 .. 7 subnormal, 8 would be 2^-6 */
  int exp2;
  (void)frexpf(v, &exp2); /* v = f * 2^exp2, f in [0.5, 1) */
  const int e = exp2 - 1 + 7;
  const int m = (int)(ldexpf(v, -(exp2 - 1)) * 8.0f) - 8;
  return (uint8_t)((e << 3) | m);
}

uint8_t oracle_e4m3_encode(float x) {
  const uint8_t sign = signbit(x) ? 0x80 : 0;
  if (isnan(x)) return sign | 0x7f;
  float a = fabsf(x);
  if (a > 448.0f) a = 448.0f;
  if (a == 0.0f) return sign;
  /* Spacing of representable values around a: 2^-9 below 2^-6, else 2^(floor(log2 a) - 3). */
  float quantum;
  if (a < 0x1p-6f) {
    quantum = 0x1p-9f;
  } else {
    int exp2;
    (void)frexpf(a, &exp2);
    quantum = ldexpf(1.0f, exp2 - 1 - 3);
  }
  const float n = rintf(a / quantum); /* exact quotient (power-of-two divisor); ties to even */
  return sign | encode_exact(n * quantum);
}

void oracle_e4m3_encode_array(const float *x, int64_t n, float scale, uint8_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_encode(x[i] / scale);
}

void oracle_e4m3_decode_array(const uint8_t *codes, int64_t n, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3_decode(codes[i]);
}

/*
 * Per-row scales (the build's second fp8 pool variant; one scale per pool row,
 * i.e. per (token, KV head)): for a row x of n values
 *   amax = max |x_i| (NaN when any x_i is NaN),
 *   s    = amax / 448, replaced by 1 when it is 0, NaN or infinite,
 *   code = e4m3(clamp(x_i / s, -448, 448)),
 * so the row's largest finite magnitude maps to code magnitude 448.
 */
float oracle_e4m3_row_scale(const float *x, int64_t n) {
  float amax = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    if (isnan(x[i])) return 1.0f;
    const float a = fabsf(x[i]);
    if (a > amax) amax = a;
  }
  const float s = amax / 448.0f;
  return (s > 0.0f && isfinite(s)) ? s : 1.0f;
}

void oracle_e4m3_encode_rows(const float *x, int64_t rows, int64_t n, uint8_t *out,
                             float *scales) {
  for (int64_t r = 0; r < rows; ++r) {
    const float s = oracle_e4m3_row_scale(x + r * n, n);
    scales[r] = s;
    oracle_e4m3_encode_array(x + r * n, n, s, out + r * n);
  }
}
