/*
 * wtc_oracle.c -- CPU restatement of the Welder typical chain
 *   out[M,N] = softmax_row(scale * (A[M,K] . B[K,N]))
 * and of the reference harness's input generators and number formats.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path (the HIP library,
 * the C-ABI, the wtc-compiler CLI, bench.py's timed region) may link, load
 * or call this file.  It is used by tests/, by __graft_entry__.smoke() as the
 * checker, and by bench.py's cpu_baseline leg.
 *
 * Every function names the reference file:line it restates (paths relative
 * to the reference repository root).  How each function is pinned:
 *   - generators: closed forms of the reference (linear, xorshift32),
 *     checked against hand-computed values in tests/test_oracle.py;
 *   - f16 / bf16 / e4m3 converters: checked bit-for-bit against numpy
 *     float16 and torch bfloat16 / float8_e4m3fn over all f16 bit patterns
 *     and dense random samples;
 *   - chain rows: checked against closed forms (K=1 one-hot, all-equal rows
 *     -> 1/N, shift invariance), brute-force numpy float64 on small shapes,
 *     and the committed golden fixtures in tests/golden/;
 *   - f16-accumulate rows (the reference lowering's precision, information
 *     only): checked against a numpy float16 loop on tiny shapes.
 * The normal generator wtc_ref_fill_normal_f32 is this build's own (the
 * reference has none); it is pinned by its golden prefix and its moments.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define WTC_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* Generators                                                          */
/* ------------------------------------------------------------------ */

/* xorshift32 (13, 17, 5).
 * backend/welder/compiler/solver/WelderProfilerRuntime.h:141-149,
 * backend/welder/bench/verify_matmul_softmax.py:48-53 */
WTC_EXPORT uint32_t wtc_ref_xorshift32(uint32_t s) {
  s ^= s << 13;
  s ^= s >> 17;
  s ^= s << 5;
  return s;
}

/* --init=random: seed 0 -> 1, u = float(rng) * 2^-32, value = u*2-1, all in
 * f32 arithmetic as the profiler does (WelderProfilerRuntime.h:141-149).
 * Each buffer restarts from the seed (initMemrefF32 builds a fresh rng per
 * call, WelderProfilerRuntime.h:141). */
WTC_EXPORT void wtc_ref_fill_random_f32(float *out, int64_t n, uint64_t seed) {
  uint32_t rng = (uint32_t)(seed == 0 ? 1 : seed);
  for (int64_t i = 0; i < n; ++i) {
    rng = wtc_ref_xorshift32(rng);
    float u = (float)rng * (1.0f / 4294967296.0f);
    out[i] = u * 2.0f - 1.0f;
  }
}

/* --init=linear: (flat % 1024) * 0.001f - 0.5f.
 * WelderProfilerRuntime.h:136-139, verify_matmul_softmax.py:43-45 */
WTC_EXPORT void wtc_ref_fill_linear_f32(float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    int64_t t = i % 1024;
    out[i] = (float)t * 0.001f - 0.5f;
  }
}

/* uniform[lo, hi) on the same xorshift32 stream: u*(hi-lo)+lo in f32.
 * With lo=-1, hi=1 this is bit-identical to wtc_ref_fill_random_f32. */
WTC_EXPORT void wtc_ref_fill_uniform_f32(float *out, int64_t n, uint64_t seed,
                                         float lo, float hi) {
  uint32_t rng = (uint32_t)(seed == 0 ? 1 : seed);
  for (int64_t i = 0; i < n; ++i) {
    rng = wtc_ref_xorshift32(rng);
    float u = (float)rng * (1.0f / 4294967296.0f);
    out[i] = u * (hi - lo) + lo;
  }
}

/* N(0, stddev^2), this build's own generator (no reference counterpart):
 * Box-Muller on the xorshift32 stream.  u1 = ((r >> 8) + 0.5) * 2^-24 lies in
 * (0, 1), u2 = (r >> 8) * 2^-24; z0 = sqrt(-2 ln u1) cos(2 pi u2),
 * z1 = sqrt(-2 ln u1) sin(2 pi u2); computed in double, stored as f32. */
WTC_EXPORT void wtc_ref_fill_normal_f32(float *out, int64_t n, uint64_t seed,
                                        float stddev) {
  uint32_t rng = (uint32_t)(seed == 0 ? 1 : seed);
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t i = 0; i < n; i += 2) {
    rng = wtc_ref_xorshift32(rng);
    double u1 = ((double)(rng >> 8) + 0.5) * (1.0 / 16777216.0);
    rng = wtc_ref_xorshift32(rng);
    double u2 = (double)(rng >> 8) * (1.0 / 16777216.0);
    double r = sqrt(-2.0 * log(u1));
    out[i] = (float)(r * cos(two_pi * u2) * stddev);
    if (i + 1 < n)
      out[i + 1] = (float)(r * sin(two_pi * u2) * stddev);
  }
}

/* ------------------------------------------------------------------ */
/* Number formats                                                      */
/* ------------------------------------------------------------------ */

static uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
static float bits_f32(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* IEEE binary16, round to nearest even, overflow -> inf, NaN kept quiet.
 * Same rounding as verify_matmul_softmax.py:66-107 (the verifier's RNE). */
WTC_EXPORT uint16_t wtc_ref_f32_to_f16(float x) {
  uint32_t u = f32_bits(x);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t exp = (u >> 23) & 0xFFu;
  uint32_t mant = u & 0x7FFFFFu;
  if (exp == 0xFFu)
    return (uint16_t)(sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0u));
  int32_t e16 = (int32_t)exp - 127 + 15;
  if (e16 >= 31)
    return (uint16_t)(sign | 0x7C00u);
  if (e16 <= 0) {
    if (e16 < -10)
      return (uint16_t)sign;
    mant |= 0x800000u;
    uint32_t shift = (uint32_t)(14 - e16);
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u)))
      ++q; /* may carry into the smallest normal: still a valid encoding */
    return (uint16_t)(sign | q);
  }
  uint32_t q = mant >> 13;
  uint32_t rem = mant & 0x1FFFu;
  uint32_t out = ((uint32_t)e16 << 10) | q;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))
    ++out; /* carry propagates into the exponent, reaching 0x7C00 = inf */
  return (uint16_t)(sign | out);
}

/* verify_matmul_softmax.py:110-127 */
WTC_EXPORT float wtc_ref_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t mant = (uint32_t)h & 0x3FFu;
  if (exp == 0) {
    float v = (float)mant * (1.0f / 16777216.0f); /* mant * 2^-24 */
    return sign ? -v : v;
  }
  if (exp == 31)
    return bits_f32(sign | 0x7F800000u | (mant << 13));
  return bits_f32(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

/* The profiler's own f32 -> f16 (WelderProfilerEval.h:50-100): adds half an
 * ulp and truncates (round half away from zero in magnitude), NaN -> 0x7e00.
 * Kept to document how far the reference harness's inputs differ from RNE. */
WTC_EXPORT uint16_t wtc_ref_f32_to_f16_profiler(float x) {
  uint32_t bits = f32_bits(x);
  uint32_t sign = (bits >> 31) & 1u;
  int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
  uint32_t mant = bits & 0x7FFFFFu;
  uint16_t out_sign = (uint16_t)(sign << 15);
  if (exp == 0xFF)
    return (uint16_t)(out_sign | (mant == 0 ? 0x7C00u : 0x7E00u));
  int32_t half_exp = exp - 127 + 15;
  if (half_exp >= 31)
    return (uint16_t)(out_sign | 0x7C00u);
  if (half_exp <= 0) {
    if (half_exp < -10)
      return out_sign;
    mant |= 0x800000u;
    int32_t shift = 14 - half_exp;
    uint32_t r = mant + (1u << (shift - 1));
    return (uint16_t)(out_sign | (uint16_t)(r >> shift));
  }
  uint32_t r = mant + 0x1000u;
  if (r & 0x800000u) {
    r = 0;
    ++half_exp;
    if (half_exp >= 31)
      return (uint16_t)(out_sign | 0x7C00u);
  }
  return (uint16_t)(out_sign | (uint16_t)(half_exp << 10) |
                    (uint16_t)((r >> 13) & 0x3FFu));
}

/* bfloat16, round to nearest even (the upper half of the f32 pattern). */
WTC_EXPORT uint16_t wtc_ref_f32_to_bf16(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu))
    return (uint16_t)((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

WTC_EXPORT float wtc_ref_bf16_to_f32(uint16_t h) {
  return bits_f32((uint32_t)h << 16);
}

/* OCP FP8 E4M3 (the "fn" variant used by gfx950): bias 7, no infinities,
 * 0x7F / 0xFF are NaN, largest finite 448.  Round to nearest even with
 * saturation to +-448 (values that would round past 448 clamp to it). */
WTC_EXPORT uint8_t wtc_ref_f32_to_e4m3(float x) {
  uint32_t u = f32_bits(x);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu))
    return (uint8_t)(sign | 0x7Fu);
  double a = fabs((double)x);
  if (a >= 448.0)
    return (uint8_t)(sign | 0x7Eu);
  if (a < 0.015625) { /* below 2^-6: subnormal grid of step 2^-9 */
    double q = nearbyint(a * 512.0); /* FE_TONEAREST: ties to even */
    return (uint8_t)(sign | (uint8_t)q); /* q == 8 is the smallest normal */
  }
  int e;
  double fr = frexp(a, &e); /* a = fr * 2^e, fr in [0.5, 1) */
  int ue = e - 1;           /* a = (2 fr) * 2^ue, 2 fr in [1, 2) */
  double m = nearbyint((2.0 * fr - 1.0) * 8.0);
  if (m >= 8.0) {
    m = 0.0;
    ++ue;
  }
  int code = ((ue + 7) << 3) | (int)m;
  if (code > 0x7E)
    code = 0x7E;
  return (uint8_t)(sign | (uint8_t)code);
}

WTC_EXPORT float wtc_ref_e4m3_to_f32(uint8_t q) {
  int sign = q & 0x80;
  int e = (q >> 3) & 0xF;
  int m = q & 0x7;
  float v;
  if (e == 0xF && m == 0x7)
    return NAN;
  if (e == 0)
    v = (float)m * (1.0f / 512.0f);
  else
    v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  return sign ? -v : v;
}

/* Bulk converters (the per-element functions above, applied to arrays). */
WTC_EXPORT void wtc_ref_quantize_f16(const float *x, uint16_t *q, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    q[i] = wtc_ref_f32_to_f16(x[i]);
}
WTC_EXPORT void wtc_ref_quantize_bf16(const float *x, uint16_t *q, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    q[i] = wtc_ref_f32_to_bf16(x[i]);
}
/* Per-tensor amax scaling to e4m3: scale = amax / 448 (1 when amax == 0),
 * q = e4m3(x / scale).  Returns the scale; x ~= e4m3_to_f32(q) * scale. */
WTC_EXPORT float wtc_ref_quantize_e4m3_amax(const float *x, uint8_t *q,
                                            int64_t n) {
  float amax = 0.0f;
  for (int64_t i = 0; i < n; ++i) {
    float a = fabsf(x[i]);
    if (a > amax)
      amax = a;
  }
  float scale = amax > 0.0f ? amax / 448.0f : 1.0f;
  for (int64_t i = 0; i < n; ++i)
    q[i] = wtc_ref_f32_to_e4m3(x[i] / scale);
  return scale;
}
WTC_EXPORT void wtc_ref_dequant_f16(const uint16_t *q, float *x, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    x[i] = wtc_ref_f16_to_f32(q[i]);
}
WTC_EXPORT void wtc_ref_dequant_bf16(const uint16_t *q, float *x, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    x[i] = wtc_ref_bf16_to_f32(q[i]);
}
WTC_EXPORT void wtc_ref_dequant_e4m3(const uint8_t *q, float *x, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    x[i] = wtc_ref_e4m3_to_f32(q[i]);
}

/* ------------------------------------------------------------------ */
/* The chain                                                           */
/* ------------------------------------------------------------------ */

/* Sampled rows of out = softmax_row(scale * A.B), float64 throughout.
 * Chain semantics: mlir/matmul_softmax_chain.mlir:10-83 (matmul from a zero
 * fill, max from -FLT_MAX, exp(C - max), sum from 0, divide), the f16 chain
 * mlir/matmul_softmax_chain_f16_native.mlir:7-95, the named form
 * mlir/matmul_softmax_chain_named_softmax.mlir:6-20; the verifier's closed
 * form backend/welder/bench/verify_matmul_softmax.py:242-261.
 * A is [M,K] row-major, B is [K,N] row-major, both already decoded to f32
 * (fp8 dequant scales go into `scale`).  For each of the nrows rows in
 * `rows`, writes logits (scale applied, may be NULL) and probabilities to
 * row r of the [nrows, N] outputs.  Returns 0, or 1 on a bad row index. */
WTC_EXPORT int wtc_ref_chain_rows(const float *A, const float *B, int64_t M,
                                  int64_t N, int64_t K, const int64_t *rows,
                                  int64_t nrows, double scale,
                                  double *out_logits, double *out_probs) {
  double *acc = (double *)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
  if (!acc)
    return 2;
  for (int64_t r = 0; r < nrows; ++r) {
    int64_t i = rows[r];
    if (i < 0 || i >= M) {
      free(acc);
      return 1;
    }
    for (int64_t j = 0; j < N; ++j)
      acc[j] = 0.0;
    for (int64_t k = 0; k < K; ++k) {
      double a = (double)A[i * K + k];
      const float *brow = B + k * N;
      for (int64_t j = 0; j < N; ++j)
        acc[j] += a * (double)brow[j];
    }
    double mx = -3.4028234663852886e+38; /* the chain's max init */
    for (int64_t j = 0; j < N; ++j) {
      acc[j] *= scale;
      if (acc[j] > mx)
        mx = acc[j];
    }
    double sum = 0.0;
    for (int64_t j = 0; j < N; ++j)
      sum += exp(acc[j] - mx);
    for (int64_t j = 0; j < N; ++j) {
      if (out_logits)
        out_logits[r * N + j] = acc[j];
      out_probs[r * N + j] = exp(acc[j] - mx) / sum;
    }
  }
  free(acc);
  return 0;
}

/* The reference lowering's precision (information only): C accumulated in
 * f16 in k order, c = f16(c + f16(a*b)), from a zero fill
 * (bench/baselines/default/baseline/04c.after_linalg_to_loops.mlir:44-108,
 * mlir/matmul_softmax_chain_f16_native.mlir:13-17), widened to f32
 * (:21-31), times `scale` in f32 (a scaled chain such as attention's
 * 1/sqrt(d) multiplies the widened logits; 1 for the reference's chain),
 * then the f32 softmax.  Output in double. */
WTC_EXPORT int wtc_ref_chain_rows_f16acc(const float *A, const float *B,
                                         int64_t M, int64_t N, int64_t K,
                                         const int64_t *rows, int64_t nrows,
                                         float scale, double *out_probs) {
  for (int64_t r = 0; r < nrows; ++r) {
    int64_t i = rows[r];
    if (i < 0 || i >= M)
      return 1;
    float mx = -3.4028235e+38f;
    for (int64_t j = 0; j < N; ++j) {
      float c = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        float p = wtc_ref_f16_to_f32(wtc_ref_f32_to_f16(A[i * K + k] * B[k * N + j]));
        c = wtc_ref_f16_to_f32(wtc_ref_f32_to_f16(c + p));
      }
      c *= scale;
      out_probs[r * N + j] = c;
      if (c > mx)
        mx = c;
    }
    float sum = 0.0f;
    for (int64_t j = 0; j < N; ++j)
      sum += expf((float)out_probs[r * N + j] - mx);
    for (int64_t j = 0; j < N; ++j)
      out_probs[r * N + j] = (double)(expf((float)out_probs[r * N + j] - mx) / sum);
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* CPU baseline: the chain lowered to loops, f32                        */
/* ------------------------------------------------------------------ */

/* A restatement of what `mlir-opt --convert-linalg-to-loops` followed by the
 * LLVM CPU backend makes of the chain (the image has no mlir-opt): fill C=0,
 * i-j-k matmul with k innermost, max-reduce from -FLT_MAX with maximumf,
 * exp(C - max), sum-reduce from 0, divide.  Loop structure follows the
 * linalg.generic iterator order of mlir/matmul_softmax_chain.mlir:16-83.
 * Rows [row0, row0+nrows) only (a bounded sample); `C` is [nrows,N] scratch.
 * threads > 1 splits rows with OpenMP.  Returns elapsed seconds. */
WTC_EXPORT double wtc_cpu_chain_loops_f32(const float *A, const float *B,
                                          float *C, float *out, int64_t N,
                                          int64_t K, int64_t row0,
                                          int64_t nrows, int threads) {
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
#ifdef _OPENMP
  if (threads < 1)
    threads = 1;
#pragma omp parallel for num_threads(threads) schedule(static)
#endif
  for (int64_t r = 0; r < nrows; ++r) {
    const float *arow = A + (row0 + r) * K;
    float *crow = C + r * N;
    for (int64_t j = 0; j < N; ++j)
      crow[j] = 0.0f;
    for (int64_t j = 0; j < N; ++j) {
      float c = crow[j];
      for (int64_t k = 0; k < K; ++k)
        c += arow[k] * B[k * N + j];
      crow[j] = c;
    }
    float mx = -3.4028235e+38f;
    for (int64_t j = 0; j < N; ++j) {
      float x = crow[j];
      mx = (x != x || x > mx) ? x : mx; /* arith.maximumf propagates NaN */
    }
    float *orow = out + r * N;
    for (int64_t j = 0; j < N; ++j)
      orow[j] = expf(crow[j] - mx);
    float sum = 0.0f;
    for (int64_t j = 0; j < N; ++j)
      sum += orow[j];
    for (int64_t j = 0; j < N; ++j)
      orow[j] = orow[j] / sum;
  }
  clock_gettime(CLOCK_MONOTONIC, &t1);
  return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

WTC_EXPORT int wtc_cpu_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
