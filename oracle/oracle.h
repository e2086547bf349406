/*
 * oracle.h -- CPU restatement of the reference's CPU-JIT lowering of the dense
 * path (linalg.matmul, bias generic, ReLU / leaky-ReLU generic).
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path may link, load or call
 * this library: only tests/, __graft_entry__.smoke() (as the checker) and the
 * cpu_baseline leg of bench.py use it.
 *
 * What it restates (reference file:line):
 *   - linalg.fill 0 then linalg.matmul (cpp/src/builders/LinalgBuilder.cpp:106-139);
 *   - CPU pipeline (cpp/src/MLIRLowering.cpp:353-434): 64x64 output tiles run
 *     in parallel (forall -> scf.parallel -> omp.parallel, MLIRLowering.cpp:362-375,
 *     MLIRLoweringPasses.cpp:470-473); inside a tile, 8x8x8 tiles in m, n, k
 *     loop order (MLIRLoweringPasses.cpp:270-319, 467-469); a static 8x8x8 tile
 *     becomes vector.contract (MLIRLoweringPasses.cpp:103-185) -> outer
 *     products -> vector.fma (MLIRLoweringPasses.cpp:242-260), i.e. per output
 *     element an ascending-k fused multiply-add chain from +0.0; tiles whose
 *     shape is dynamic fall to convert-linalg-to-loops (MLIRLowering.cpp:410):
 *     scalar mulf then addf, each rounded;
 *   - the bias generic (LinalgBuilder.cpp:301-339) merged with the activation
 *     generic (LinalgBuilder.cpp:180-239) by linalg-fuse-elementwise-ops
 *     (MLIRLowering.cpp:355) and run as one separate pass after the matmul:
 *     y = addf(c, b[n]); relu = maximumf(y, 0); leaky = maximumf(y,0) +
 *     alpha * minimumf(y,0);
 *   - i32: arith.muli / arith.addi, two's complement wrapping; ReLU written
 *     tensor_map(v -> If(v > 0, v, 0)) (LinalgBuilder.cpp:141-178);
 *   - the f32 ReLU written as a tensor_map with an If body
 *     (LinalgBuilder.cpp:141-178): y = cmpf ogt(y, 0) ? y : 0, so NaN -> +0
 *     and -0 -> +0, unlike maximumf.
 *
 * Rounding chains. Per output element the reference sums in ascending k from
 * +0.0. A static 8x8x8 tile becomes vector.fma (one rounding per step); a
 * dynamic tile falls to scalar mulf then addf (two roundings per step). Which
 * tiles the MLIR vectorizer sees as static is decided inside MLIR, which is
 * absent here, so the oracle takes the chain as an argument and computes
 * either one; the parity tests hold a result to the bar against both chains
 * element by element, which covers the reference whichever chain (or per-tile
 * mix of chains) it takes.
 *
 * Pinning (tests/test_oracle.py): the reference's known answers, exact
 * rational golden vectors of both chains (tests/golden/make_golden.py), the
 * fp64 forward-error bound, exact wrapping i32 arithmetic, IEEE special values
 * through every epilogue, and planted mistakes that those checks must catch.
 * No function of this library is left unpinned.
 *
 * Operands are contiguous row-major: X[M][K], W[K][N], b[N], Y[M][N].
 * epilogue: bit 0 = add bias; bits 1-2 = activation (0 none, 1 relu as
 * maximumf, 2 leaky, 3 relu as If(v > 0, v, 0); f32 only for 2 and 3).
 */
#ifndef EDSL_ORACLE_H
#define EDSL_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Rounding chain of the f32 sums: vector.fma per k step (static tiles), or
 * mulf then addf per k step (dynamic tiles, convert-linalg-to-loops). */
#define ORACLE_CHAIN_FMA 0
#define ORACLE_CHAIN_MULADD 1

/* Returns 0, -1 on a bad epilogue code, -4 on a bad chain. threads <= 0:
 * OpenMP default. */
int oracle_dense_f32(const float *X, const float *W, const float *b, float *Y, int64_t M,
                     int64_t N, int64_t K, int epilogue, float alpha, int chain, int threads);
int oracle_dense_i32(const int32_t *X, const int32_t *W, const int32_t *b, int32_t *Y,
                     int64_t M, int64_t N, int64_t K, int epilogue, int threads);

/* oracle_dense_f32 on the fma chain with the 8x8x8 micro-kernel on 8-wide FMA
 * vectors, as the reference JIT emits it for static tiles (bit-identical
 * results; M, N and K multiples of 8 only: returns -2 otherwise, -3 when built
 * without AVX2/FMA). For timing the reference's CPU schedule at its own vector
 * width. */
int oracle_dense_f32_vec(const float *X, const float *W, const float *b, float *Y, int64_t M,
                         int64_t N, int64_t K, int epilogue, float alpha, int threads);

/* Test hook: plant a known mistake (0 = none) so the tests can show that the
 * checks pinning this oracle catch it. See oracle.c for the list. */
void oracle_set_mutation(int mutation);

#ifdef __cplusplus
}
#endif

#endif
