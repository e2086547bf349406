// fp32 dense layer / matmul with one wave per 128x128 output tile and no LDS.
//
// C[M,N] = epilogue(A[M,K] x B[K,N] (+ bias[N])) -- the same op as the tiles
// of gemm_f32.hip and gemm_f32_m16.hip (reference
// cpp/src/builders/LinalgBuilder.cpp:106-139, 180-239, 301-339), for 16-byte
// aligned operands and row strides.
//
// Design:
//  * v_mfma_f32_16x16x4_f32: lane l supplies A[row l%16][k-slot l/16] and
//    B[k-slot l/16][col l%16] and receives rows 4*(l/16)..+3 of column l%16.
//    Lane group g = l/16 owns k = 16j + 4g .. 16j + 4g + 3 of each 16-deep
//    group j, which is exactly one 16-byte load of an A row: the A fragment of
//    row block i is A[m0 + 16i + l%16][16j + 4g .. +3], straight from memory
//    into the operand register, and the B fragment of k-slot s is
//    B[16j + 4g + s][n0 + 4*(l%16) .. +3] and [.. + 64 ..]: each B load reads
//    four k rows of 256 contiguous bytes. Column block c < 4 holds output
//    columns n0 + 4*(l%16) + c, column block c >= 4 columns n0 + 64 +
//    4*(l%16) + c - 4, so each lane ends with two 4-column vectors per row.
//  * One wave computes the whole 128x128 tile (8x8 blocks, 256 accumulator
//    registers) and runs 256 MFMAs per 16 loads of 16 bytes; it shares nothing
//    with other waves, so there is no LDS stage and no barrier. Loads run one
//    group ahead in a ring of two register sets (a group's 256 MFMAs take
//    ~3.4 us at 2.4 GHz), spread over the MFMAs with scheduling group
//    barriers. One wave per SIMD (512 registers), four tiles per CU.
//  * A and B are read through buffer descriptors: the tile's base in
//    scalar registers and 32-bit offsets, so the loop has no 64-bit address
//    arithmetic (134 vector registers besides the accumulators, against 202
//    with flat 64-bit addresses and 952 against 929-934 us at 4096^3).
//  * Workgroups map to tiles XCD-aware (common.hpp: tile_coords); C is written
//    with non-temporal stores.
//
// GUARD kGuardNone: M, N multiples of 128 and K of 16. kGuardEdge: partial
// tiles (N and K multiples of 4). There the range check of the buffer loads
// does the bounds work: every offset that can leave an operand is in the
// per-lane offset (the scalar offset is zero), rows past M read zero, columns
// past N read values whose outputs are never stored, and A chunks past K are
// sent out of range so that they read zero (B rows past K read zero too).
#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>
#include <utility>

namespace edsl {
namespace {

template <int N>
using Ic = std::integral_constant<int, N>;

template <typename F, int... S>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, S...>) {
  (f(Ic<S>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Raw buffer load of 16 bytes (the <4 x i32> descriptor form of the
// intrinsic, so that a descriptor built from uniform values stays in scalar
// registers). Offsets at or past the descriptor's byte count read zero.
__device__ f32x4 raw_buffer_load_f32x4(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4f32");

// Descriptor of `bytes` bytes from `base` (raw addressing: stride 0, 32-bit
// data format word of the gfx9 family).
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, int64_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const int n = bytes > 0x7fffffff ? 0x7fffffff : bytes < 0 ? 0 : (int)bytes;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  r[2] = __builtin_amdgcn_readfirstlane(n);
  r[3] = 0x00020000;
  return r;
}

constexpr int kTile = 128;
constexpr int RB = 8;      // 16-row MFMA blocks of the tile
constexpr int CB = 8;      // 16-column MFMA blocks of the tile
constexpr int kSets = 2;   // register sets of loads: the current group and the next
constexpr int kSlices = 16;
constexpr int kOutOfRange = 0x7fffffff;  // a per-lane offset past every descriptor

template <int GUARD, int EPI>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_f32_direct_kernel(GemmF32Args args) {
  static_assert(GUARD == kGuardNone || GUARD == kGuardEdge, "guard");
  constexpr bool kEdge = GUARD == kGuardEdge;
  const int lane = threadIdx.x;
  const int g = lane >> 4;
  const int r16 = lane & 15;
  int tm, tn;
  tile_coords(blockIdx.x, args.tiles_m, args.tiles_n, tm, tn);
  const int m0 = __builtin_amdgcn_readfirstlane(tm * kTile);
  const int n0 = __builtin_amdgcn_readfirstlane(tn * kTile);
  const int K = args.K;
  const int ng = (K + 15) / 16;  // 16-deep groups (the last one partial on edge tiles)
  const int lda = (int)args.lda, ldb = (int)args.ldb;

  // A from row m0 on (rows past M out of range), B from column n0 on (rows
  // past K out of range).
  const i32x4 rsrc_a = buffer_rsrc(args.A + (int64_t)m0 * lda, (int64_t)(args.M - m0) * lda * 4);
  const i32x4 rsrc_b = buffer_rsrc(args.B + n0, (int64_t)K * ldb * 4 - (int64_t)n0 * 4);
  const int va = (r16 * lda + 4 * g) * 4;      // + row block 16i, + 16j along K
  const int vb = (4 * g * ldb + 4 * r16) * 4;  // + k slot s, + 16j rows, + 64 columns
  // Edge tiles: per-lane offsets of the row blocks (rows past M are out of
  // range) and of the two column halves, clamped to column N-4 (rows stay
  // inside B; the outputs of clamped columns are never stored).
  int va_i[RB];
  int vb_h[2];
  if constexpr (kEdge) {
#pragma unroll
    for (int i = 0; i < RB; ++i) va_i[i] = va + i * 64 * lda;
#pragma unroll
    for (int h = 0; h < 2; ++h) vb_h[h] = (4 * g * ldb + min(n0 + 64 * h + 4 * r16, args.N - 4) - n0) * 4;
  }

  struct Frag {
    f32x4 a[RB];     // row block i: A[m0 + 16i + r16][16j + 4g .. +3]
    f32x4 b[4][2];   // k slot s, column half h: B[16j + 4g + s][n0 + 64h + 4*r16 .. +3]
  };
  auto load = [&](Frag& f, int j) __attribute__((always_inline)) {
    if constexpr (!kEdge) {
#pragma unroll
      for (int i = 0; i < RB; ++i)
        f.a[i] = raw_buffer_load_f32x4(rsrc_a, va, 64 * j + i * 64 * lda, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        f.b[s][0] = raw_buffer_load_f32x4(rsrc_b, vb, (16 * j + s) * ldb * 4, 0);
        f.b[s][1] = raw_buffer_load_f32x4(rsrc_b, vb + 256, (16 * j + s) * ldb * 4, 0);
      }
    } else {
      // The offsets that can leave A or B are per lane: a row block's row,
      // and the k rows of the lane's chunk, which are all below K or all at
      // or past it (K is a multiple of 4). A chunk past K is sent out of range
      // and reads zero, and so do the four B rows that pair with it (their
      // offsets are at or past K rows of B whatever the scalar k-slot offset
      // adds).
      const bool k_in = 16 * j + 4 * g < K;
#pragma unroll
      for (int i = 0; i < RB; ++i)
        f.a[i] = raw_buffer_load_f32x4(rsrc_a, k_in ? va_i[i] : kOutOfRange, 64 * j, 0);
      const int rowj = 16 * j * ldb * 4;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        f.b[s][0] = raw_buffer_load_f32x4(rsrc_b, vb_h[0] + rowj, s * ldb * 4, 0);
        f.b[s][1] = raw_buffer_load_f32x4(rsrc_b, vb_h[1] + rowj, s * ldb * 4, 0);
      }
    }
  };

  f32x4 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int c = 0; c < CB; ++c) acc[i][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto mfmas = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int c = 0; c < CB; ++c)
          acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i][s], f.b[s][c / 4][c % 4], acc[i][c], 0, 0, 0);
  };
  // The next group's 16 loads spread over the group's 256 MFMAs, one per
  // slice of 16 (the compiler otherwise issues them as one burst).
  constexpr int kLoads = RB + 8;
  constexpr int kMfmas = 4 * RB * CB;
  auto pin = [&]() __attribute__((always_inline)) {
    static_for<kSlices>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      constexpr int v = kLoads / kSlices + (t < kLoads % kSlices ? 1 : 0);
      if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x020, v, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, kMfmas / kSlices, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };

  // Group j is computed from set j % 2 while group j + 1 loads into the other
  // set. Loads past the last group repeat the last group (in range, never
  // used), so the loop body has no branch.
  Frag fr[kSets];
  load(fr[0], 0);  // ng >= 1: the launcher requires K >= 4
  int j = 0;
  for (; j + kSets <= ng; j += kSets) {
    static_for<kSets>([&](auto sc) __attribute__((always_inline)) {
      constexpr int S = decltype(sc)::value;
      load(fr[(S + 1) % kSets], min(j + S + 1, ng - 1));
      mfmas(fr[S]);
      pin();
    });
  }
  static_for<kSets>([&](auto sc) __attribute__((always_inline)) {
    constexpr int S = decltype(sc)::value;
    if (j + S < ng) {
      load(fr[(S + 1) % kSets], min(j + S + 1, ng - 1));
      mfmas(fr[S]);
    }
  });

  // Epilogue: lane holds rows m0 + 16i + 4g + e and columns n0 + 64h +
  // 4*r16 .. +3.
  const float alpha = args.alpha;
  f32x4 biasv[2] = {};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int col = n0 + 64 * h + 4 * r16;
    if constexpr (epi_has_bias(EPI)) {
      if (!kEdge || col < args.N) biasv[h] = *reinterpret_cast<const f32x4*>(args.bias + col);
    }
  }
#pragma unroll
  for (int i = 0; i < RB; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = m0 + 16 * i + 4 * g + e;
      if (kEdge && row >= args.M) continue;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int col = n0 + 64 * h + 4 * r16;
        f32x4 v;
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = apply_epilogue_f32<EPI>(acc[i][4 * h + c][e], biasv[h][c], alpha);
        if (!kEdge || col < args.N)
          __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(args.C + (int64_t)row * args.ldc + col));
      }
    }
    // One row block at a time: the scheduler would otherwise gather the
    // values of many blocks and run out of registers.
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int GUARD>
hipError_t launch_guard(int epi, const GemmF32Args& a, hipStream_t stream) {
  const dim3 grid(a.tiles_m * a.tiles_n);
  const dim3 block(64);
#define EDSL_DIRECT_CASE(E)                                                                \
  case E:                                                                                  \
    hipLaunchKernelGGL((gemm_f32_direct_kernel<GUARD, E>), grid, block, 0, stream, a);    \
    break;
  switch (epi) {
    EDSL_DIRECT_CASE(epi_code(false, ACT_NONE))
    EDSL_DIRECT_CASE(epi_code(true, ACT_NONE))
    EDSL_DIRECT_CASE(epi_code(false, ACT_RELU))
    EDSL_DIRECT_CASE(epi_code(true, ACT_RELU))
    EDSL_DIRECT_CASE(epi_code(false, ACT_LEAKY))
    EDSL_DIRECT_CASE(epi_code(true, ACT_LEAKY))
    EDSL_DIRECT_CASE(epi_code(false, ACT_IF_RELU))
    EDSL_DIRECT_CASE(epi_code(true, ACT_IF_RELU))
    default:
      return hipErrorInvalidValue;
  }
#undef EDSL_DIRECT_CASE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_f32_direct(int guard, int epi, GemmF32Args a, hipStream_t stream) {
  // Shapes, strides and alignment the kernel assumes (the planner only picks
  // it for such layers; checked again here because a wrong launch reads out
  // of bounds).
  if (a.M < 1 || a.N < 4 || a.K < 4 || a.N % 4 || a.K % 4) return hipErrorInvalidValue;
  if (a.lda < a.K || a.ldb < a.N || a.ldc < a.N || a.lda % 4 || a.ldb % 4 || a.ldc % 4) return hipErrorInvalidValue;
  const uintptr_t bias_bits = epi_has_bias(epi) ? (uintptr_t)a.bias : 0;
  if (((uintptr_t)a.A | (uintptr_t)a.B | (uintptr_t)a.C | bias_bits) % 16) return hipErrorInvalidValue;
  if (epi_has_bias(epi) && a.bias == nullptr) return hipErrorInvalidValue;
  if (!gemm_f32_direct_offsets_fit(a.K, a.lda, a.ldb)) return hipErrorInvalidValue;
  if (a.tiles_m != (a.M + kTile - 1) / kTile || a.tiles_n != (a.N + kTile - 1) / kTile) return hipErrorInvalidValue;
  if (guard == kGuardNone) {
    if (a.M % kTile || a.N % kTile || a.K % 16) return hipErrorInvalidValue;
    return launch_guard<kGuardNone>(epi, a, stream);
  }
  if (guard == kGuardEdge) return launch_guard<kGuardEdge>(epi, a, stream);
  return hipErrorInvalidValue;
}

}  // namespace edsl
