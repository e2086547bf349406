// Integer dense layer / matmul: i32 tensors, exact i32 (wrapping) arithmetic.
//
// The reference DSL carries integer tensors as i32 (reference
// cpp/schemas/ast.proto:26-36, mlir_edsl/types.py:175); linalg.matmul over i32
// lowers to arith.muli / arith.addi, which wrap modulo 2^32, and the bias
// generic to arith.addi (reference cpp/src/builders/LinalgBuilder.cpp:106-139,
// 301-339). ReLU on i32 is tensor_map(v -> If(v > 0, v, 0))
// (LinalgBuilder.cpp:141-178).
//
// Fast path (int8 matrix cores): when every X and W value lies in [-128, 127]
// the product can run on v_mfma_i32_32x32x32_i8 exactly: each product fits in
// 15 bits and the i32 accumulator cannot overflow for K < 2^17, so the sum
// equals the exact integer sum -- identical to the wrapping i32 sum in any
// order. A pre-pass narrows X to int8 [M][K] and W to int8 [N][K] (transposed,
// so both MFMA operands are K-contiguous) and flags any out-of-range value.
// The GEMM kernel reads the flag: if set, the whole grid takes the exact
// wrapping-i32 vector-ALU path on the original i32 tensors instead. The flag
// is compared against a per-call epoch, so it never needs clearing.
#include "common.hpp"
#include "kernels.hpp"

namespace edsl {
namespace {

// ------------------------------------------------------------------ pre-pass
constexpr int kNarrowTile = 64;

// Grid: tiles of X ([M][K], 64x64) followed by tiles of W ([K][N], 64x64).
__global__ void __launch_bounds__(256) narrow_i8_kernel(NarrowI8Args a) {
  const int tid = threadIdx.x;
  const int x_tiles_k = (a.K + kNarrowTile - 1) / kNarrowTile;
  const int x_tiles = ((a.M + kNarrowTile - 1) / kNarrowTile) * x_tiles_k;
  bool bad = false;
  if ((int)blockIdx.x < x_tiles) {
    // X: row-major copy, 4 values per thread per pass.
    const int tm = blockIdx.x / x_tiles_k, tk = blockIdx.x % x_tiles_k;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int idx = tid + p * 256;
      const int r = idx / 16;
      const int c = 4 * (idx % 16);
      const int m = tm * kNarrowTile + r;
      const int k = tk * kNarrowTile + c;
      if (m >= a.M) continue;
      const int32_t* src = a.X + (int64_t)m * a.ldx + k;
      int8_t* dst = a.X8 + (int64_t)m * a.K + k;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (k + e < a.K) {
          const int32_t v = src[e];
          bad |= (v < -128) | (v > 127);
          dst[e] = (int8_t)v;
        }
      }
    }
  } else {
    // W: transpose through LDS so both the i32 reads (along n) and the int8
    // writes (along k) are contiguous.
    __shared__ int8_t t[kNarrowTile][kNarrowTile + 4];
    const int b = blockIdx.x - x_tiles;
    const int w_tiles_n = (a.N + kNarrowTile - 1) / kNarrowTile;
    const int tk = b / w_tiles_n, tn = b % w_tiles_n;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int idx = tid + p * 256;
      const int r = idx / 16;          // k within tile
      const int c = 4 * (idx % 16);    // n within tile
      const int k = tk * kNarrowTile + r;
      const int n = tn * kNarrowTile + c;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int32_t v = 0;
        if (k < a.K && n + e < a.N) {
          v = a.W[(int64_t)k * a.ldw + n + e];
          bad |= (v < -128) | (v > 127);
        }
        t[c + e][r] = (int8_t)v;
      }
    }
    __syncthreads();
    // Each thread writes 16 consecutive k of one n row.
    const int r = tid / 4;            // n within tile
    const int c = 16 * (tid % 4);     // k within tile
    const int n = tn * kNarrowTile + r;
    const int k = tk * kNarrowTile + c;
    if (n < a.N) {
      int8_t* dst = a.W8t + (int64_t)n * a.K + k;
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (k + e < a.K) dst[e] = t[r][c + e];
    }
  }
  if (__any(bad) && (tid & 63) == 0) *a.flag = a.epoch;
}

// ------------------------------------------------- exact i32 vector-ALU tile
// 128x128 output tile, 256 threads, 8x8 outputs per thread, K staged in LDS
// in steps of 32. Bounds-checked throughout; unsigned arithmetic = wrapping.
constexpr int kValuTile = 128;
constexpr int kValuK = 32;

struct ValuSmem {
  uint32_t x[kValuTile][kValuK + 1];
  uint32_t w[kValuK][kValuTile + 1];
};

template <int EPI>
__device__ void valu_tile_i32(const GemmI32Args& a, int m0, int n0, ValuSmem& sm) {
  const int tid = threadIdx.x;
  const int ty = tid / 16, tx = tid % 16;
  uint32_t acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = 0u;

  for (int k0 = 0; k0 < a.K; k0 += kValuK) {
    for (int idx = tid; idx < kValuTile * kValuK; idx += 256) {
      const int r = idx / kValuK, c = idx % kValuK;
      const int m = m0 + r, k = k0 + c;
      sm.x[r][c] = (m < a.M && k < a.K) ? (uint32_t)a.X[(int64_t)m * a.ldx + k] : 0u;
    }
    for (int idx = tid; idx < kValuK * kValuTile; idx += 256) {
      const int r = idx / kValuTile, c = idx % kValuTile;
      const int k = k0 + r, n = n0 + c;
      sm.w[r][c] = (k < a.K && n < a.N) ? (uint32_t)a.W[(int64_t)k * a.ldw + n] : 0u;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < kValuK; ++kk) {
      uint32_t xv[8], wv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[i] = sm.x[ty + 16 * i][kk];
#pragma unroll
      for (int j = 0; j < 8; ++j) wv[j] = sm.w[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] += xv[i] * wv[j];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = m0 + ty + 16 * i;
    if (m >= a.M) continue;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n = n0 + tx + 16 * j;
      if (n >= a.N) continue;
      const int32_t b = epi_has_bias(EPI) ? a.bias[n] : 0;
      a.C[(int64_t)m * a.ldc + n] = apply_epilogue_i32<EPI>((int32_t)acc[i][j], b);
    }
  }
}

template <int EPI>
__global__ void __launch_bounds__(256) gemm_i32_valu_kernel(GemmI32Args a) {
  __shared__ ValuSmem sm;
  const int tm = blockIdx.x / a.tiles_n, tn = blockIdx.x % a.tiles_n;
  valu_tile_i32<EPI>(a, tm * kValuTile, tn * kValuTile, sm);
}

// -------------------------------------------------------- int8 MFMA kernel
// 128x128 tile, 4 waves (2x2), wave tile 64x64 = 2x2 blocks of 32x32.
// K staged 128 bytes at a time; LDS rows are 128 B = 8 chunks of 16 B, chunk
// index XOR (row % 8) so the 16-byte fragment reads of 16 rows hit all banks.
// v_mfma_i32_32x32x32_i8: lane l supplies 16 int8 of A row l%32 and 16 int8
// of B^T row (= output column) l%32, both from chunk (2t + l/32) of the
// 32-k step t, so A and B always pair the same k.
constexpr int kBK = 128;   // int8 per K step
constexpr int kChunks = kBK / 16;

struct I8Smem {
  i32x4 a[2][kI8Tile * kChunks];
  i32x4 b[2][kI8Tile * kChunks];
};

template <int EPI>
__global__ void __launch_bounds__(256) gemm_i8_kernel(GemmI32Args a) {
  __shared__ union {
    I8Smem mf;
    ValuSmem valu;
  } sm;
  int tm, tn;
  tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int m0 = tm * kI8Tile, n0 = tn * kI8Tile;

  if (*a.flag == a.epoch) {  // some value outside int8: exact i32 path
    valu_tile_i32<EPI>(a, m0, n0, sm.valu);
    return;
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave >> 1) * 64;
  const int wn = (wave & 1) * 64;
  const int half = lane >> 5;
  const int l32 = lane & 31;

  constexpr int LD = kI8Tile * kChunks / 256;  // 16-byte chunks per thread per operand
  i32x4 ra[LD], rb[LD];
  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int idx = tid + i * 256;
      const int r = idx / kChunks, q = idx % kChunks;
      ra[i] = *reinterpret_cast<const i32x4*>(a.A8 + (int64_t)(m0 + r) * a.K + k0 + 16 * q);
      rb[i] = *reinterpret_cast<const i32x4*>(a.B8t + (int64_t)(n0 + r) * a.K + k0 + 16 * q);
    }
  };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int idx = tid + i * 256;
      const int r = idx / kChunks, q = idx % kChunks;
      sm.mf.a[buf][r * kChunks + (q ^ (r % 8))] = ra[i];
      sm.mf.b[buf][r * kChunks + (q ^ (r % 8))] = rb[i];
    }
  };

  i32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  const int nk = a.K / kBK;
  load_global(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) load_global((kt + 1) * kBK);
#pragma unroll
    for (int t = 0; t < kBK / 32; ++t) {
      const int q = 2 * t + half;
      i32x4 av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int ra_row = wm + 32 * i + l32;
        av[i] = sm.mf.a[buf][ra_row * kChunks + (q ^ (ra_row % 8))];
        const int rb_row = wn + 32 * i + l32;
        bv[i] = sm.mf.b[buf][rb_row * kChunks + (q ^ (rb_row % 8))];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_lds(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows 8*(r/4) + 4*half + r%4 and column l32 of each block.
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn + 32 * j + l32;
    const int32_t b = epi_has_bias(EPI) ? a.bias[n] : 0;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * half + (r & 3);
        a.C[(int64_t)m * a.ldc + n] = apply_epilogue_i32<EPI>(acc[i][j][r], b);
      }
  }
}

#define EDSL_I32_EPI_SWITCH(KERNEL, GRID, ARGS)                                        \
  switch (epi) {                                                                       \
    case epi_code(false, ACT_NONE):                                                    \
      hipLaunchKernelGGL(KERNEL<epi_code(false, ACT_NONE)>, GRID, dim3(256), 0, stream, ARGS); \
      break;                                                                           \
    case epi_code(true, ACT_NONE):                                                     \
      hipLaunchKernelGGL(KERNEL<epi_code(true, ACT_NONE)>, GRID, dim3(256), 0, stream, ARGS); \
      break;                                                                           \
    case epi_code(false, ACT_RELU):                                                    \
      hipLaunchKernelGGL(KERNEL<epi_code(false, ACT_RELU)>, GRID, dim3(256), 0, stream, ARGS); \
      break;                                                                           \
    case epi_code(true, ACT_RELU):                                                     \
      hipLaunchKernelGGL(KERNEL<epi_code(true, ACT_RELU)>, GRID, dim3(256), 0, stream, ARGS); \
      break;                                                                           \
    default:                                                                           \
      return hipErrorInvalidValue;                                                     \
  }

}  // namespace

hipError_t launch_narrow_i8(NarrowI8Args a, hipStream_t stream) {
  const int x_tiles = ((a.M + kNarrowTile - 1) / kNarrowTile) * ((a.K + kNarrowTile - 1) / kNarrowTile);
  const int w_tiles = ((a.K + kNarrowTile - 1) / kNarrowTile) * ((a.N + kNarrowTile - 1) / kNarrowTile);
  hipLaunchKernelGGL(narrow_i8_kernel, dim3(x_tiles + w_tiles), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_gemm_i8(int epi, GemmI32Args a, hipStream_t stream) {
  a.tiles_m = a.M / kI8Tile;
  a.tiles_n = a.N / kI8Tile;
  const dim3 grid(a.tiles_m * a.tiles_n);
  EDSL_I32_EPI_SWITCH(gemm_i8_kernel, grid, a)
  return hipGetLastError();
}

hipError_t launch_gemm_i32_valu(int epi, GemmI32Args a, hipStream_t stream) {
  a.tiles_m = (a.M + kValuTile - 1) / kValuTile;
  a.tiles_n = (a.N + kValuTile - 1) / kValuTile;
  const dim3 grid(a.tiles_m * a.tiles_n);
  EDSL_I32_EPI_SWITCH(gemm_i32_valu_kernel, grid, a)
  return hipGetLastError();
}

}  // namespace edsl
