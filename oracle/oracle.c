/*
 * oracle.c -- CPU restatement of the reference CPU-JIT dense path.
 * TEST INFRASTRUCTURE ONLY (see oracle.h for what is restated and where).
 *
 * Build: see oracle/Makefile. Compiled with -ffp-contract=off so that the
 * scalar mulf+addf path is not fused behind our back; the fma path calls fmaf.
 */
#include "oracle.h"

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#endif

/* Planted mistakes, for the tests that show the pinning checks catch them:
 *  1  W read transposed (W[n][k] instead of W[k][n]; square shapes only)
 *  2  bias dropped
 *  3  ReLU as fmaxf (NaN -> 0 instead of NaN)
 *  4  bias subtracted
 *  5  last k term dropped
 *  6  fma chain replaced by mulf+addf rounding
 *  7  leaky slope applied to the positive side
 *  8  i32 accumulated in f32
 *  9  mulf+addf chain contracted to fma
 * 10  If-ReLU as maximumf (NaN -> NaN instead of +0)
 * 11  If-ReLU keeps -0 (v >= 0 instead of v > 0)
 */
static int g_mutation = 0;

void oracle_set_mutation(int mutation) { g_mutation = mutation; }

enum { ACT_NONE = 0, ACT_RELU = 1, ACT_LEAKY = 2, ACT_IF_RELU = 3 };

static inline float w_at(const float *W, int64_t k, int64_t n, int64_t N, int64_t K) {
  if (g_mutation == 1) return W[n * K + k];
  return W[k * N + n];
}

/* One 8x8x8 tile of the m, n, k tile loops (reference
 * MLIRLoweringPasses.cpp:270-319), clipped at the matrix edges to mc x nc x kc.
 * Each element of the C tile continues its ascending-k chain: on the fma
 * chain one fused multiply-add per k (vector.contract -> outer products ->
 * vector.fma, MLIRLoweringPasses.cpp:103-185, 242-260), on the mulf+addf chain
 * a rounded product then a rounded sum (convert-linalg-to-loops,
 * MLIRLowering.cpp:410). The k loop is outermost, as in the outer-product
 * form; every element still sees its own k terms in ascending order. */
static void micro_8x8x8(const float *A, const float *W, float *C, int64_t m0, int64_t n0,
                        int64_t k0, int64_t mc, int64_t nc, int64_t kc, int64_t N, int64_t K,
                        int use_fma) {
  float c[8][8];
  for (int m = 0; m < 8; ++m)
    for (int n = 0; n < 8; ++n) c[m][n] = (m < mc && n < nc) ? C[(m0 + m) * N + n0 + n] : 0.0f;
  for (int64_t k = 0; k < kc; ++k) {
    if (g_mutation == 5 && k0 + k == K - 1) continue;
    float w[8];
    for (int n = 0; n < 8; ++n) w[n] = n < nc ? w_at(W, k0 + k, n0 + n, N, K) : 0.0f;
    for (int m = 0; m < mc; ++m) {
      const float a = A[(m0 + m) * K + k0 + k];
      if (use_fma) {
        for (int n = 0; n < 8; ++n) c[m][n] = fmaf(a, w[n], c[m][n]);
      } else {
        for (int n = 0; n < 8; ++n) {
          const float p = a * w[n];
          c[m][n] = c[m][n] + p;
        }
      }
    }
  }
  for (int m = 0; m < mc; ++m)
    for (int n = 0; n < nc; ++n) C[(m0 + m) * N + n0 + n] = c[m][n];
}

static void matmul_f32(const float *A, const float *W, float *C, int64_t M, int64_t N, int64_t K,
                       int chain, int threads) {
  /* linalg.fill: runs serially before the parallel matmul. */
  for (int64_t i = 0; i < M * N; ++i) C[i] = 0.0f;
  int use_fma = chain == ORACLE_CHAIN_FMA;
  if ((use_fma && g_mutation == 6) || (!use_fma && g_mutation == 9)) use_fma = !use_fma;
  const int64_t tiles_m = (M + 63) / 64, tiles_n = (N + 63) / 64;
  const int64_t tiles = tiles_m * tiles_n;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : omp_get_max_threads())
  for (int64_t t = 0; t < tiles; ++t) {
    const int64_t m0 = (t / tiles_n) * 64, n0 = (t % tiles_n) * 64;
    const int64_t mh = M - m0 < 64 ? M - m0 : 64;
    const int64_t nh = N - n0 < 64 ? N - n0 : 64;
    for (int64_t mi = 0; mi < mh; mi += 8)
      for (int64_t ni = 0; ni < nh; ni += 8)
        for (int64_t ki = 0; ki < K; ki += 8)
          micro_8x8x8(A, W, C, m0 + mi, n0 + ni, ki, mh - mi < 8 ? mh - mi : 8,
                      nh - ni < 8 ? nh - ni : 8, K - ki < 8 ? K - ki : 8, N, K, use_fma);
  }
}

static inline float maximumf0(float x) {
  if (g_mutation == 3) return fmaxf(x, 0.0f);
  return (x > 0.0f || x != x) ? x : 0.0f; /* NaN -> NaN, -0 -> +0 */
}

static inline float minimumf0(float x) {
  return (x < 0.0f || x != x || x == 0.0f) ? x : 0.0f; /* NaN -> NaN, -0 -> -0 */
}

/* If(v > 0.0, v, 0.0) on f32: arith.cmpf ogt (false for NaN) selecting v or
 * the constant +0.0 (reference LinalgBuilder.cpp:141-178, the comparison
 * predicate at ArithBuilder.cpp:122-126). NaN -> +0, -0 -> +0. */
static inline float if_relu0(float x) {
  if (g_mutation == 10) return maximumf0(x);
  if (g_mutation == 11) return x >= 0.0f ? x : 0.0f;
  return x > 0.0f ? x : 0.0f;
}

int oracle_dense_f32(const float *X, const float *W, const float *b, float *Y, int64_t M,
                     int64_t N, int64_t K, int epilogue, float alpha, int chain, int threads) {
  if (epilogue < 0 || epilogue > 7) return -1;
  if (chain != ORACLE_CHAIN_FMA && chain != ORACLE_CHAIN_MULADD) return -4;
  const int has_bias = epilogue & 1;
  const int act = (epilogue >> 1) & 3;
  matmul_f32(X, W, Y, M, N, K, chain, threads);
  if (!has_bias && act == ACT_NONE) return 0;
  /* The merged bias + activation generic: one serial elementwise pass. */
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float y = Y[m * N + n];
      if (has_bias && g_mutation != 2) y = (g_mutation == 4) ? y - b[n] : y + b[n];
      if (act == ACT_RELU) {
        y = maximumf0(y);
      } else if (act == ACT_IF_RELU) {
        y = if_relu0(y);
      } else if (act == ACT_LEAKY) {
        const float pos = maximumf0(y), neg = minimumf0(y);
        if (g_mutation == 7) {
          const float scaled = pos * alpha;
          y = scaled + neg;
        } else {
          const float scaled = neg * alpha;
          y = pos + scaled;
        }
      }
      Y[m * N + n] = y;
    }
  return 0;
}

/* The same lowering on the fma chain, with the 8x8x8 micro-kernel on 8-wide
 * vectors as the reference JIT emits it: each outer product is one vector.fma
 * over a row of the C tile (reference MLIRLoweringPasses.cpp:242-260;
 * x86Vector lowering, MLIRLowering.cpp:422-424), here one 256-bit FMA per row
 * and k. Every C element sees the same fmaf chain in the same k order as
 * micro_8x8x8 on the fma chain, so the results are bit-identical; it exists
 * to time the reference's CPU schedule at its own vector width (the
 * benchmark's CPU baseline). M, N and K multiples of 8 only (whole 8x8x8
 * tiles); no planted-mistake hooks. */
int oracle_dense_f32_vec(const float *X, const float *W, const float *b, float *Y, int64_t M,
                         int64_t N, int64_t K, int epilogue, float alpha, int threads) {
#if defined(__AVX2__) && defined(__FMA__)
  if (epilogue < 0 || epilogue > 7) return -1;
  if (M % 8 != 0 || N % 8 != 0 || K % 8 != 0) return -2;
  const int has_bias = epilogue & 1;
  const int act = (epilogue >> 1) & 3;
  for (int64_t i = 0; i < M * N; ++i) Y[i] = 0.0f; /* linalg.fill */
  const int64_t tiles_m = (M + 63) / 64, tiles_n = (N + 63) / 64;
  const int64_t tiles = tiles_m * tiles_n;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : omp_get_max_threads())
  for (int64_t t = 0; t < tiles; ++t) {
    const int64_t m0 = (t / tiles_n) * 64, n0 = (t % tiles_n) * 64;
    const int64_t mh = M - m0 < 64 ? M - m0 : 64;
    const int64_t nh = N - n0 < 64 ? N - n0 : 64;
    for (int64_t mi = 0; mi < mh; mi += 8)
      for (int64_t ni = 0; ni < nh; ni += 8)
        for (int64_t ki = 0; ki < K; ki += 8) {
          float *c0 = Y + (m0 + mi) * N + n0 + ni;
          __m256 c[8];
          for (int m = 0; m < 8; ++m) c[m] = _mm256_loadu_ps(c0 + m * N);
          for (int k = 0; k < 8; ++k) {
            const __m256 w = _mm256_loadu_ps(W + (ki + k) * N + n0 + ni);
            for (int m = 0; m < 8; ++m)
              c[m] = _mm256_fmadd_ps(_mm256_set1_ps(X[(m0 + mi + m) * K + ki + k]), w, c[m]);
          }
          for (int m = 0; m < 8; ++m) _mm256_storeu_ps(c0 + m * N, c[m]);
        }
  }
  if (!has_bias && act == ACT_NONE) return 0;
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float y = Y[m * N + n];
      if (has_bias) y = y + b[n];
      if (act == ACT_RELU) {
        y = (y > 0.0f || y != y) ? y : 0.0f;
      } else if (act == ACT_IF_RELU) {
        y = y > 0.0f ? y : 0.0f;
      } else if (act == ACT_LEAKY) {
        const float pos = (y > 0.0f || y != y) ? y : 0.0f;
        const float neg = (y < 0.0f || y != y || y == 0.0f) ? y : 0.0f;
        const float scaled = neg * alpha;
        y = pos + scaled;
      }
      Y[m * N + n] = y;
    }
  return 0;
#else
  (void)X; (void)W; (void)b; (void)Y; (void)M; (void)N; (void)K; (void)epilogue; (void)alpha; (void)threads;
  return -3;
#endif
}

int oracle_dense_i32(const int32_t *X, const int32_t *W, const int32_t *b, int32_t *Y, int64_t M,
                     int64_t N, int64_t K, int epilogue, int threads) {
  if (epilogue < 0 || epilogue > 3) return -1; /* leaky is float-only */
  const int has_bias = epilogue & 1;
  const int act = (epilogue >> 1) & 3;
  for (int64_t i = 0; i < M * N; ++i) Y[i] = 0;
  const int64_t tiles_m = (M + 63) / 64, tiles_n = (N + 63) / 64;
  const int64_t tiles = tiles_m * tiles_n;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : omp_get_max_threads())
  for (int64_t t = 0; t < tiles; ++t) {
    const int64_t m0 = (t / tiles_n) * 64, n0 = (t % tiles_n) * 64;
    const int64_t me = M - m0 < 64 ? M : m0 + 64;
    const int64_t ne = N - n0 < 64 ? N : n0 + 64;
    for (int64_t m = m0; m < me; ++m)
      for (int64_t k = 0; k < K; ++k) {
        if (g_mutation == 5 && k == K - 1) continue;
        const uint32_t a = (uint32_t)X[m * K + k];
        for (int64_t n = n0; n < ne; ++n) {
          const uint32_t w = (uint32_t)(g_mutation == 1 ? W[n * K + k] : W[k * N + n]);
          if (g_mutation == 8) {
            Y[m * N + n] = (int32_t)((float)Y[m * N + n] + (float)(int32_t)a * (float)(int32_t)w);
          } else {
            Y[m * N + n] = (int32_t)((uint32_t)Y[m * N + n] + a * w); /* muli, addi: mod 2^32 */
          }
        }
      }
  }
  if (!has_bias && act == ACT_NONE) return 0;
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      int32_t y = Y[m * N + n];
      if (has_bias && g_mutation != 2)
        y = (int32_t)(g_mutation == 4 ? (uint32_t)y - (uint32_t)b[n] : (uint32_t)y + (uint32_t)b[n]);
      if (act == ACT_RELU) y = y > 0 ? y : 0; /* If(v > 0, v, 0) */
      Y[m * N + n] = y;
    }
  return 0;
}
