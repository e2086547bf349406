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
// Only used on the int8 path, where M, N and K are multiples of kI8Tile, so
// X8 rows (K bytes) and W8t rows start 16-byte aligned. The i32 sources may
// have any alignment / row stride: `vec_ok` selects 16-byte source loads.
constexpr int kNarrowTile = 64;
constexpr int kNarrowLdp = kNarrowTile + 4;  // LDS row pitch (bytes) of the transposed tile

__device__ __forceinline__ uint32_t pack_i8x4(i32x4 v, bool& bad) {
  uint32_t out = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    bad |= (v[e] < -128) | (v[e] > 127);
    out |= ((uint32_t)v[e] & 0xffu) << (8 * e);
  }
  return out;
}

__device__ __forceinline__ i32x4 load4(const int32_t* p, bool vec_ok) {
  if (vec_ok) return *reinterpret_cast<const i32x4*>(p);
  return i32x4{p[0], p[1], p[2], p[3]};
}

// Grid: 64x64 tiles of X (no transpose) followed by 64x64 tiles of W
// (transposed through LDS).
__global__ void __launch_bounds__(256) narrow_i8_kernel(NarrowI8Args a, int vec_ok_x, int vec_ok_w) {
  const int tid = threadIdx.x;
  const int x_tiles_k = a.K / kNarrowTile;
  const int x_tiles = (a.M / kNarrowTile) * x_tiles_k;
  bool bad = false;
  if ((int)blockIdx.x < x_tiles) {
    const int tm = blockIdx.x / x_tiles_k, tk = blockIdx.x % x_tiles_k;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int idx = tid + p * 256;
      const int m = tm * kNarrowTile + idx / 16;
      const int k = tk * kNarrowTile + 4 * (idx % 16);
      const i32x4 v = load4(a.X + (int64_t)m * a.ldx + k, vec_ok_x);
      *reinterpret_cast<uint32_t*>(a.X8 + (int64_t)m * a.K + k) = pack_i8x4(v, bad);
    }
  } else {
    __shared__ uint8_t t[kNarrowTile * kNarrowLdp];  // [n][k]
    const int b = blockIdx.x - x_tiles;
    const int w_tiles_n = a.N / kNarrowTile;
    const int tk = b / w_tiles_n, tn = b % w_tiles_n;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int idx = tid + p * 256;
      const int r = idx / 16;        // k within tile
      const int c = 4 * (idx % 16);  // n within tile
      const i32x4 v = load4(a.W + (int64_t)(tk * kNarrowTile + r) * a.ldw + tn * kNarrowTile + c, vec_ok_w);
      const uint32_t q = pack_i8x4(v, bad);
#pragma unroll
      for (int e = 0; e < 4; ++e) t[(c + e) * kNarrowLdp + r] = (uint8_t)(q >> (8 * e));
    }
    __syncthreads();
    // Thread writes 16 consecutive k of one n row as one 16-byte store.
    const int n = tid / 4;
    const int c = 16 * (tid % 4);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(t + n * kNarrowLdp + c);
    const i32x4 out = {(int)src[0], (int)src[1], (int)src[2], (int)src[3]};
    *reinterpret_cast<i32x4*>(a.W8t + (int64_t)(tn * kNarrowTile + n) * a.K + tk * kNarrowTile + c) = out;
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

// NT threads stage the operands; the first 256 compute (8x8 outputs each).
template <int EPI, int NT>
__device__ void valu_tile_i32(const GemmI32Args& a, int m0, int n0, ValuSmem& sm) {
  const int tid = threadIdx.x;
  const bool computes = tid < 256;
  const int ty = (tid & 255) / 16, tx = tid % 16;
  uint32_t acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = 0u;

  for (int k0 = 0; k0 < a.K; k0 += kValuK) {
    for (int idx = tid; idx < kValuTile * kValuK; idx += NT) {
      const int r = idx / kValuK, c = idx % kValuK;
      const int m = m0 + r, k = k0 + c;
      sm.x[r][c] = (m < a.M && k < a.K) ? (uint32_t)a.X[(int64_t)m * a.ldx + k] : 0u;
    }
    for (int idx = tid; idx < kValuK * kValuTile; idx += NT) {
      const int r = idx / kValuTile, c = idx % kValuTile;
      const int k = k0 + r, n = n0 + c;
      sm.w[r][c] = (k < a.K && n < a.N) ? (uint32_t)a.W[(int64_t)k * a.ldw + n] : 0u;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < (computes ? kValuK : 0); ++kk) {
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
  if (!computes) return;
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
  valu_tile_i32<EPI, 256>(a, tm * kValuTile, tn * kValuTile, sm);
}

// -------------------------------------------------------- int8 MFMA kernel
// 128x128 output tile per workgroup of WAVES waves (4: 2x2 waves of 64x64;
// 8: 4x2 waves of 32x64), K staged BKB bytes at a time through two LDS
// buffers (the next stage's global loads are issued before the current
// stage's MFMAs and written to the other buffer after them). LDS rows are BKB
// bytes = BKB/16 chunks of 16 B with the chunk index XOR-ed by (row % 8), so
// the 16-byte fragment reads of 16 consecutive rows spread over the banks.
// Inside a stage the fragments of 32-k step t+1 are read from LDS while the
// MFMAs of step t run, so the matrix cores do not wait on LDS latency.
// v_mfma_i32_32x32x32_i8: lane l supplies 16 int8 of A row l%32 and 16 int8
// of B^T row (= output column) l%32, both from chunk (2t + l/32) of the
// 32-k step t, so A and B always pair the same k.
template <int BKB>
struct I8Smem {
  i32x4 a[2][kI8Tile * (BKB / 16)];
  i32x4 b[2][kI8Tile * (BKB / 16)];
};

template <int EPI, int WAVES, int BKB>
__global__ void __launch_bounds__(WAVES * 64) gemm_i8_kernel(GemmI32Args a) {
  constexpr int NT = WAVES * 64;
  constexpr int CH = BKB / 16;                 // 16-byte chunks per row per stage
  constexpr int TS = BKB / 32;                 // 32-k MFMA steps per stage
  constexpr int WAVES_N = 2;
  constexpr int WAVES_M = WAVES / WAVES_N;
  constexpr int RBM = kI8Tile / WAVES_M / 32;  // 32-row blocks per wave
  constexpr int RBN = kI8Tile / WAVES_N / 32;  // 32-col blocks per wave
  constexpr int LD = kI8Tile * CH / NT;        // chunks per thread per operand per stage
  __shared__ union {
    I8Smem<BKB> mf;
    ValuSmem valu;
  } sm;
  int tm, tn;
  tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int m0 = tm * kI8Tile, n0 = tn * kI8Tile;

  if (*a.flag == a.epoch) {  // some value outside int8: exact i32 path
    valu_tile_i32<EPI, NT>(a, m0, n0, sm.valu);
    return;
  }

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave / WAVES_N) * (32 * RBM);
  const int wn = (wave % WAVES_N) * (32 * RBN);
  const int half = lane >> 5;
  const int l32 = lane & 31;

  i32x4 ra[LD], rb[LD];
  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / CH, q = idx % CH;
      ra[i] = *reinterpret_cast<const i32x4*>(a.A8 + (int64_t)(m0 + r) * a.K + k0 + 16 * q);
      rb[i] = *reinterpret_cast<const i32x4*>(a.B8t + (int64_t)(n0 + r) * a.K + k0 + 16 * q);
    }
  };
  // chunk q of row `row` lives at slot q ^ (row % min(CH, 8)): stays below CH
  auto swz = [](int row, int q) { return row * CH + (q ^ (row % (CH < 8 ? CH : 8))); };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / CH, q = idx % CH;
      sm.mf.a[buf][swz(r, q)] = ra[i];
      sm.mf.b[buf][swz(r, q)] = rb[i];
    }
  };

  i32x16 acc[RBM][RBN];
#pragma unroll
  for (int i = 0; i < RBM; ++i)
#pragma unroll
    for (int j = 0; j < RBN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  auto read_frags = [&](int buf, int t, i32x4 (&av)[RBM], i32x4 (&bv)[RBN]) {
    const int q = 2 * t + half;
#pragma unroll
    for (int i = 0; i < RBM; ++i) av[i] = sm.mf.a[buf][swz(wm + 32 * i + l32, q)];
#pragma unroll
    for (int j = 0; j < RBN; ++j) bv[j] = sm.mf.b[buf][swz(wn + 32 * j + l32, q)];
  };
  auto compute = [&](int buf) {
    i32x4 av[2][RBM], bv[2][RBN];
    read_frags(buf, 0, av[0], bv[0]);
#pragma unroll
    for (int t = 0; t < TS; ++t) {
      if (t + 1 < TS) read_frags(buf, t + 1, av[(t + 1) & 1], bv[(t + 1) & 1]);
#pragma unroll
      for (int i = 0; i < RBM; ++i)
#pragma unroll
        for (int j = 0; j < RBN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[t & 1][i], bv[t & 1][j], acc[i][j], 0, 0, 0);
    }
  };

  const int nk = a.K / BKB;
  load_global(0);
  store_lds(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) load_global((kt + 1) * BKB);
    compute(buf);
    if (more) store_lds(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows 8*(r/4) + 4*half + r%4 and column l32 of each block.
#pragma unroll
  for (int j = 0; j < RBN; ++j) {
    const int n = n0 + wn + 32 * j + l32;
    const int32_t b = epi_has_bias(EPI) ? a.bias[n] : 0;
#pragma unroll
    for (int i = 0; i < RBM; ++i)
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
  if (a.M % kNarrowTile || a.N % kNarrowTile || a.K % kNarrowTile) return hipErrorInvalidValue;
  const int x_tiles = (a.M / kNarrowTile) * (a.K / kNarrowTile);
  const int w_tiles = (a.K / kNarrowTile) * (a.N / kNarrowTile);
  const int vec_x = ((reinterpret_cast<uintptr_t>(a.X) & 15) == 0) && (a.ldx % 4 == 0);
  const int vec_w = ((reinterpret_cast<uintptr_t>(a.W) & 15) == 0) && (a.ldw % 4 == 0);
  hipLaunchKernelGGL(narrow_i8_kernel, dim3(x_tiles + w_tiles), dim3(256), 0, stream, a, vec_x, vec_w);
  return hipGetLastError();
}

template <int WAVES, int BKB>
hipError_t launch_i8_variant(int epi, const GemmI32Args& a, hipStream_t stream) {
  const dim3 grid(a.tiles_m * a.tiles_n), block(WAVES * 64);
#define EDSL_I8_CASE(E)                                                                             \
  case E:                                                                                           \
    hipLaunchKernelGGL((gemm_i8_kernel<E, WAVES, BKB>), grid, block, 0, stream, a);                \
    break;
  switch (epi) {
    EDSL_I8_CASE(epi_code(false, ACT_NONE))
    EDSL_I8_CASE(epi_code(true, ACT_NONE))
    EDSL_I8_CASE(epi_code(false, ACT_RELU))
    EDSL_I8_CASE(epi_code(true, ACT_RELU))
    default:
      return hipErrorInvalidValue;
  }
#undef EDSL_I8_CASE
  return hipGetLastError();
}

hipError_t launch_gemm_i8(int epi, GemmI32Args a, hipStream_t stream, int variant) {
  a.tiles_m = a.M / kI8Tile;
  a.tiles_n = a.N / kI8Tile;
  if (variant < 0) variant = kI8DefaultVariant;
  if (a.K % 256 != 0 && (variant == 1 || variant == 3)) variant = (variant == 1) ? 0 : 2;
  switch (variant) {
    case 0: return launch_i8_variant<4, 128>(epi, a, stream);
    case 1: return launch_i8_variant<4, 256>(epi, a, stream);
    case 2: return launch_i8_variant<8, 128>(epi, a, stream);
    case 3: return launch_i8_variant<8, 256>(epi, a, stream);
    case 4: return launch_i8_variant<4, 64>(epi, a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm_i32_valu(int epi, GemmI32Args a, hipStream_t stream) {
  a.tiles_m = (a.M + kValuTile - 1) / kValuTile;
  a.tiles_n = (a.N + kValuTile - 1) / kValuTile;
  const dim3 grid(a.tiles_m * a.tiles_n);
  EDSL_I32_EPI_SWITCH(gemm_i32_valu_kernel, grid, a)
  return hipGetLastError();
}

}  // namespace edsl
