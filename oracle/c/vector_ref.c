/*
 * CPU oracle for the vector chain rows (TEST INFRASTRUCTURE ONLY).
 *
 * Step-by-step emulation of the reference's per-lane recurrences
 * (bench_vector.py:87-179):
 *   fp32/fp64   x <- fma(x, a, b)              one rounding (C99 fmaf/fma)
 *   fp16/bf16   x <- RN_fmt(x*a + b)           "single": one rounding of the exact value
 *               x <- RN_fmt(RN_f32(x*a + b))   "widened": fp32 result rounded again
 *                                              (the reference's _widened_fma_update)
 *   int8 dot4   x <- sum_j sbyte_j(x)*sbyte_j(W) + b   int32, wrapping
 *                                              (the reference's DP4A feedback form)
 * Narrow-format rounding is exact: the product x*a of two narrow values is
 * exact in double, TwoSum gives the sum's exact residual, and ties are broken
 * with that residual, so a double that lands on a narrow midpoint cannot
 * mislead round-to-nearest-even.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Round-to-nearest-even of (v + residual) to a binary format with `precision`
 * significand bits, minimum normal exponent emin (value 2^emin) and largest
 * finite value max_finite; residual is the exact remainder beyond v. */
static double round_format(double v, double residual, int precision, int emin, double max_finite) {
  if (v == 0.0 && residual == 0.0) return v;
  if (isnan(v) || isinf(v)) return v;
  double magnitude = fabs(v);
  double sign = v < 0 ? -1.0 : 1.0;
  double rest = residual * sign; /* residual in the direction of |v| */
  int exponent;
  frexp(magnitude, &exponent); /* magnitude = m * 2^exponent, m in [0.5, 1) */
  int e = exponent - 1;        /* magnitude in [2^e, 2^(e+1)) */
  if (e < emin) e = emin;      /* subnormal range shares the minimum quantum */
  double quantum = ldexp(1.0, e - (precision - 1));
  double scaled = magnitude / quantum; /* exact: power-of-two scaling */
  double floor_part = floor(scaled);
  double fraction = scaled - floor_part;
  double result;
  if (fraction > 0.5 || (fraction == 0.5 && rest > 0)) {
    result = floor_part + 1.0;
  } else if (fraction < 0.5 || (fraction == 0.5 && rest < 0)) {
    result = floor_part;
  } else {
    result = fmod(floor_part, 2.0) == 0.0 ? floor_part : floor_part + 1.0;
  }
  result *= quantum;
  if (result > max_finite) return sign * INFINITY;
  return sign * result;
}

/* Exact x*a + b as (sum, residual) when x*a is exact in double. */
static void two_sum_product(double x, double a, double b, double* sum, double* residual) {
  double product = x * a;
  double s = product + b;
  double bb = s - product;
  *residual = (product - (s - bb)) + (b - bb);
  *sum = s;
}

static double round_f16(double v, double r) { return round_format(v, r, 11, -14, 65504.0); }
static double round_bf16(double v, double r) { return round_format(v, r, 8, -126, 3.3895313892515355e38); }
static double round_f32(double v, double r) { return round_format(v, r, 24, -126, 3.4028234663852886e38); }

/* One narrow-format update; mode 0 = single rounding, 1 = via fp32. */
static double narrow_step(double x, double a, double b, int bf16, int widened) {
  double sum, residual;
  two_sum_product(x, a, b, &sum, &residual);
  if (widened) {
    double f32 = round_f32(sum, residual);
    return bf16 ? round_bf16(f32, 0.0) : round_f16(f32, 0.0);
  }
  return bf16 ? round_bf16(sum, residual) : round_f16(sum, residual);
}

/* ---- exported chains: x[n] in/out, iterations updates each ---------------- */

void oracle_chain_f32(float* x, long n, float a, float b, long iterations) {
  for (long i = 0; i < n; ++i) {
    float v = x[i];
    for (long t = 0; t < iterations; ++t) v = fmaf(v, a, b);
    x[i] = v;
  }
}

void oracle_chain_f64(double* x, long n, double a, double b, long iterations) {
  for (long i = 0; i < n; ++i) {
    double v = x[i];
    for (long t = 0; t < iterations; ++t) v = fma(v, a, b);
    x[i] = v;
  }
}

/* Narrow chains operate on exact double values of the narrow states. */
void oracle_chain_narrow(double* x, long n, double a, double b, long iterations, int bf16, int widened) {
  for (long i = 0; i < n; ++i) {
    double v = x[i];
    for (long t = 0; t < iterations; ++t) v = narrow_step(v, a, b, bf16, widened);
    x[i] = v;
  }
}

/* Correctly rounded conversion of doubles to a narrow format (for inputs). */
void oracle_round_narrow(double* x, long n, int bf16) {
  for (long i = 0; i < n; ++i) x[i] = bf16 ? round_bf16(x[i], 0.0) : round_f16(x[i], 0.0);
}

static int32_t dot4_step(int32_t x, int32_t w, int32_t b) {
  int64_t total = 0;
  for (int j = 0; j < 4; ++j) {
    int8_t xs = (int8_t)(((uint32_t)x >> (8 * j)) & 255u);
    int8_t ws = (int8_t)(((uint32_t)w >> (8 * j)) & 255u);
    total += (int64_t)xs * (int64_t)ws;
  }
  return (int32_t)(uint32_t)((uint64_t)total + (uint64_t)(int64_t)b); /* int32 wrap-around */
}

void oracle_chain_dot4(int32_t* x, long n, int32_t w, int32_t b, long iterations) {
  for (long i = 0; i < n; ++i) {
    int32_t v = x[i];
    for (long t = 0; t < iterations; ++t) v = dot4_step(v, w, b);
    x[i] = v;
  }
}
