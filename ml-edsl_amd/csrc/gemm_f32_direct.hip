// fp32 dense layer / matmul with one wave per output tile and no LDS stage:
// a 128x128 tile (large layers), its 64x64 twin with K optionally split over
// four waves of a workgroup (mid-size layers), R x C tiles of 32x32 to 96x96
// with K split over four waves (mid-size layers whose 64x64 tiles do not fill
// whole rounds of the CUs) and a 16x16 tile with K split over four waves
// (small layers). The K-split tiles sum their partial tiles once through LDS;
// nothing else goes through LDS.
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
// does the bounds work: every offset that can leave an operand -- a row of A
// past M, a row of B past K -- is in the per-lane offset, the scalar offset
// adding only the k position inside a row of A and the k slot (below 4)
// inside a lane's chunk of B rows. Rows past M read zero, B columns past N
// are clamped to column N-4 (their outputs are never stored), and A chunks
// past K are sent out of range so that they read zero, as do the B rows that
// pair with them.
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

constexpr int kTile = 128;
constexpr int RB = 8;      // 16-row MFMA blocks of the tile
constexpr int CB = 8;      // 16-column MFMA blocks of the tile
constexpr int kSets = 2;   // register sets of loads: the current group and the next
constexpr int kSlices = 16;
constexpr int kOutOfRange = 0x7fffffff;  // a per-lane offset past every descriptor

// One 128x128 tile at (m0, n0): kEdge selects the edge loads and the checked
// stores.
template <bool kEdge, int EPI>
__device__ __forceinline__ void direct128_tile(const GemmF32Args& args, int m0, int n0) {
  const int lane = threadIdx.x;
  const int g = lane >> 4;
  const int r16 = lane & 15;
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

template <int GUARD, int EPI>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_f32_direct_kernel(GemmF32Args args) {
  static_assert(GUARD == kGuardNone || GUARD == kGuardEdge, "guard");
  int tm, tn;
  tile_coords(blockIdx.x, args.tiles_m, args.tiles_n, tm, tn);
  const int m0 = __builtin_amdgcn_readfirstlane(tm * kTile);
  const int n0 = __builtin_amdgcn_readfirstlane(tn * kTile);
  if constexpr (GUARD == kGuardNone) {
    direct128_tile<false, EPI>(args, m0, n0);
  } else {
    // Edge layers: the tiles that lie inside M x N with a K of whole groups
    // take the exact tile's loads and stores; only the others pay for the
    // per-lane bounds.
    if (m0 + kTile <= args.M && n0 + kTile <= args.N && args.K % 16 == 0)
      direct128_tile<false, EPI>(args, m0, n0);
    else
      direct128_tile<true, EPI>(args, m0, n0);
  }
}

// The 64x64 tile: a workgroup of KS waves, each wave the whole tile (4x4
// blocks, 64 accumulator registers) over its share of K -- KS contiguous runs
// of 16-deep groups -- with the same fragment loads as the 128x128 tile (one
// 4-column quad of B per k slot), and the same edge handling. The KS partial tiles are then summed
// through LDS in a fixed order (wave 0 + wave 1 + ...), each wave finishing
// 4/KS of the tile's four row blocks. Groups are 64 MFMAs (~0.85 us), so loads run two groups
// ahead in three register sets. For layers with too few 128x128 tiles to fill
// the SIMDs (1024^3: 256 tiles of 64x64, K split four ways).
constexpr int kSets64 = 3;

template <int KS, int GUARD, int EPI>
__global__ void __launch_bounds__(64 * KS)
gemm_f32_direct64_kernel(GemmF32Args args) {
  static_assert(KS == 1 || KS == 4, "K split");
  static_assert(GUARD == kGuardNone || GUARD == kGuardEdge, "guard");
  constexpr bool kEdge = GUARD == kGuardEdge;
  constexpr int RB4 = 4, CB4 = 4;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4;
  const int r16 = lane & 15;
  int tm, tn;
  tile_coords(blockIdx.x, args.tiles_m, args.tiles_n, tm, tn);
  const int m0 = __builtin_amdgcn_readfirstlane(tm * 64);
  const int n0 = __builtin_amdgcn_readfirstlane(tn * 64);
  const int K = args.K;
  // The wave's groups jb .. jb + ngw - 1. Exact tiles: K is a multiple of
  // 16 * KS. Edge tiles: ceil(K / 16) groups shared as evenly as they go (a
  // wave may get none when K < 16 * KS), the last one partial.
  const int ng = (K + 15) / 16;
  const int jb = kEdge ? wave * ng / KS : wave * (K / 16 / KS);
  const int ngw = kEdge ? (wave + 1) * ng / KS - jb : K / 16 / KS;
  const int lda = (int)args.lda, ldb = (int)args.ldb;

  const i32x4 rsrc_a = buffer_rsrc(args.A + (int64_t)m0 * lda, (int64_t)(args.M - m0) * lda * 4);
  const i32x4 rsrc_b = buffer_rsrc(args.B + n0, (int64_t)K * ldb * 4 - (int64_t)n0 * 4);
  const int va = (r16 * lda + 4 * g) * 4;
  const int vb = (4 * g * ldb + 4 * r16) * 4;
  // Edge tiles, as for the 128x128 tile: per-lane row-block offsets (rows
  // past M out of range), the column quad clamped to N-4.
  int va_i[RB4];
  int vb_c = 0;
  if constexpr (kEdge) {
#pragma unroll
    for (int i = 0; i < RB4; ++i) va_i[i] = va + i * 64 * lda;
    vb_c = (4 * g * ldb + min(n0 + 4 * r16, args.N - 4) - n0) * 4;
  }

  struct Frag {
    f32x4 a[RB4];  // row block i: A[m0 + 16i + r16][16j + 4g .. +3]
    f32x4 b[4];    // k slot s: B[16j + 4g + s][n0 + 4*r16 .. +3]
  };
  auto load = [&](Frag& f, int j) __attribute__((always_inline)) {
    if constexpr (!kEdge) {
#pragma unroll
      for (int i = 0; i < RB4; ++i) f.a[i] = raw_buffer_load_f32x4(rsrc_a, va, 64 * j + i * 64 * lda, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) f.b[s] = raw_buffer_load_f32x4(rsrc_b, vb, (16 * j + s) * ldb * 4, 0);
    } else {
      // A chunks past K are sent out of range; the B rows that pair with them
      // are at or past K rows of B and read zero.
      const bool k_in = 16 * j + 4 * g < K;
#pragma unroll
      for (int i = 0; i < RB4; ++i)
        f.a[i] = raw_buffer_load_f32x4(rsrc_a, k_in ? va_i[i] : kOutOfRange, 64 * j, 0);
      const int vbj = vb_c + 16 * j * ldb * 4;
#pragma unroll
      for (int s = 0; s < 4; ++s) f.b[s] = raw_buffer_load_f32x4(rsrc_b, vbj, s * ldb * 4, 0);
    }
  };
  f32x4 acc[RB4][CB4];
#pragma unroll
  for (int i = 0; i < RB4; ++i)
#pragma unroll
    for (int c = 0; c < CB4; ++c) acc[i][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto mfmas = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < RB4; ++i)
#pragma unroll
        for (int c = 0; c < CB4; ++c)
          acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i][s], f.b[s][c], acc[i][c], 0, 0, 0);
  };
  // 8 loads over 64 MFMAs: one load per 8 MFMAs.
  auto pin = [&]() __attribute__((always_inline)) {
    static_for<8>([&](auto) __attribute__((always_inline)) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };

  // Group jb + t is computed from set t % 3 while groups jb + t + 1 and
  // jb + t + 2 are in flight; loads past the wave's last group repeat it.
  const int jl = jb + ngw - 1;
  if (ngw > 0) {
    Frag fr[kSets64];
    load(fr[0], jb);
    load(fr[1], min(jb + 1, jl));
    int t = 0;
    for (; t + kSets64 <= ngw; t += kSets64) {
      static_for<kSets64>([&](auto sc) __attribute__((always_inline)) {
        constexpr int S = decltype(sc)::value;
        load(fr[(S + 2) % kSets64], min(jb + t + S + 2, jl));
        mfmas(fr[S]);
        pin();
      });
    }
    static_for<kSets64>([&](auto sc) __attribute__((always_inline)) {
      constexpr int S = decltype(sc)::value;
      if (t + S < ngw) {
        load(fr[(S + 2) % kSets64], min(jb + t + S + 2, jl));
        mfmas(fr[S]);
      }
    });
  }

  // Lane holds rows m0 + 16i + 4g + e and columns n0 + 4*r16 .. +3 of its
  // partial tile. Sum the KS partials (wave order) for the rows this wave
  // finishes, then bias, activation and one 16-byte store per row.
  const float alpha = args.alpha;
  const int col = n0 + 4 * r16;
  f32x4 biasv = {};
  if constexpr (epi_has_bias(EPI)) {
    if (!kEdge || col < args.N) biasv = *reinterpret_cast<const f32x4*>(args.bias + col);
  }
  auto store_row = [&](int i, int e, const f32x4& sums) __attribute__((always_inline)) {
    f32x4 v;
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = apply_epilogue_f32<EPI>(sums[c], biasv[c], alpha);
    const int row = m0 + 16 * i + 4 * g + e;
    if (!kEdge || (row < args.M && col < args.N))
      __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(args.C + (int64_t)row * args.ldc + col));
  };
  if constexpr (KS == 1) {
#pragma unroll
    for (int i = 0; i < RB4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) store_row(i, e, f32x4{acc[i][0][e], acc[i][1][e], acc[i][2][e], acc[i][3][e]});
  } else {
    // [wave][row block][column block][lane] of 16-byte accumulator vectors:
    // each access moves 64 lanes x 16 contiguous bytes, no bank conflict.
    // Wave w finishes row blocks w*RB4/KS ..: for each of its blocks and
    // column blocks it reads the KS partials as vectors and sums them in
    // wave order.
    static_assert(RB4 % KS == 0, "row blocks per wave");
    __shared__ f32x4 red[KS * RB4 * CB4 * 64];
    auto slot = [&](int w, int i, int c) { return ((w * RB4 + i) * CB4 + c) * 64 + lane; };
#pragma unroll
    for (int i = 0; i < RB4; ++i)
#pragma unroll
      for (int c = 0; c < CB4; ++c) red[slot(wave, i, c)] = acc[i][c];
    __syncthreads();
    constexpr int kBlocks = RB4 / KS;  // row blocks each wave finishes
#pragma unroll
    for (int r = 0; r < kBlocks; ++r) {
      const int i = wave * kBlocks + r;
      f32x4 sums[CB4];  // [column block][e]
#pragma unroll
      for (int c = 0; c < CB4; ++c) {
        f32x4 sum = red[slot(0, i, c)];
#pragma unroll
        for (int w = 1; w < KS; ++w) {
          const f32x4 p = red[slot(w, i, c)];
#pragma unroll
          for (int e = 0; e < 4; ++e) sum[e] = __fadd_rn(sum[e], p[e]);
        }
        sums[c] = sum;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) store_row(i, e, f32x4{sums[0][e], sums[1][e], sums[2][e], sums[3][e]});
    }
  }
}

template <int KS, int GUARD>
hipError_t launch_ks64(int epi, const GemmF32Args& a, hipStream_t stream) {
  const dim3 grid(a.tiles_m * a.tiles_n);
  const dim3 block(64 * KS);
#define EDSL_DIRECT64_CASE(E)                                                              \
  case E:                                                                                  \
    hipLaunchKernelGGL((gemm_f32_direct64_kernel<KS, GUARD, E>), grid, block, 0, stream, a); \
    break;
  switch (epi) {
    EDSL_DIRECT64_CASE(epi_code(false, ACT_NONE))
    EDSL_DIRECT64_CASE(epi_code(true, ACT_NONE))
    EDSL_DIRECT64_CASE(epi_code(false, ACT_RELU))
    EDSL_DIRECT64_CASE(epi_code(true, ACT_RELU))
    EDSL_DIRECT64_CASE(epi_code(false, ACT_LEAKY))
    EDSL_DIRECT64_CASE(epi_code(true, ACT_LEAKY))
    EDSL_DIRECT64_CASE(epi_code(false, ACT_IF_RELU))
    EDSL_DIRECT64_CASE(epi_code(true, ACT_IF_RELU))
    default:
      return hipErrorInvalidValue;
  }
#undef EDSL_DIRECT64_CASE
  return hipGetLastError();
}

// The 16x16 tile for small layers (256^3: 256 tiles): a workgroup of four
// waves, each wave one 16x16 MFMA block over a quarter of K, all of its
// fragments (at most kMaxGroups16 groups of 16) loaded up front, then the
// four partial blocks summed through LDS in wave order, each wave finishing
// one of the four rows every lane holds. So the layer's MFMAs spread over
// 1024 waves, one per SIMD, and a wave waits for its loads once.
constexpr int kMaxGroups16 = 8;

template <int EPI>
__global__ void __launch_bounds__(256)
gemm_f32_direct16_kernel(GemmF32Args args) {
  constexpr int KS = 4;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4;
  const int r16 = lane & 15;
  int tm, tn;
  tile_coords(blockIdx.x, args.tiles_m, args.tiles_n, tm, tn);
  const int m0 = __builtin_amdgcn_readfirstlane(tm * 16);
  const int n0 = __builtin_amdgcn_readfirstlane(tn * 16);
  const int ngw = args.K / 16 / KS;  // groups per wave: K is a multiple of 64, at most 64 * kMaxGroups16
  const int jb = wave * ngw;
  const int lda = (int)args.lda, ldb = (int)args.ldb;
  const i32x4 rsrc_a = buffer_rsrc(args.A + (int64_t)m0 * lda, (int64_t)(args.M - m0) * lda * 4);
  const i32x4 rsrc_b = buffer_rsrc(args.B + n0, (int64_t)args.K * ldb * 4 - (int64_t)n0 * 4);
  const int va = (r16 * lda + 4 * g) * 4;      // A[m0 + r16][16j + 4g .. +3]
  const int vb = (4 * g * ldb + r16) * 4;      // B[16j + 4g + s][n0 + r16]

  f32x4 a[kMaxGroups16];
  float b[kMaxGroups16][4];
#pragma unroll
  for (int t = 0; t < kMaxGroups16; ++t) {
    if (t < ngw) {
      const int j = jb + t;
      a[t] = raw_buffer_load_f32x4(rsrc_a, va, 64 * j, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) b[t][s] = raw_buffer_load_f32(rsrc_b, vb, (16 * j + s) * ldb * 4, 0);
    }
  }
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < kMaxGroups16; ++t) {
    if (t < ngw) {
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][s], b[t][s], acc, 0, 0, 0);
    }
  }

  // Lane holds rows m0 + 4g + e, column n0 + r16. [wave][e][lane] in LDS.
  __shared__ float red[KS * 4 * 64];
#pragma unroll
  for (int e = 0; e < 4; ++e) red[(wave * 4 + e) * 64 + lane] = acc[e];
  __syncthreads();
  float sum = red[(0 * 4 + wave) * 64 + lane];
#pragma unroll
  for (int w = 1; w < KS; ++w) sum = __fadd_rn(sum, red[(w * 4 + wave) * 64 + lane]);
  const int row = m0 + 4 * g + wave;
  const int col = n0 + r16;
  const float bias = epi_has_bias(EPI) ? args.bias[col] : 0.0f;
  __builtin_nontemporal_store(apply_epilogue_f32<EPI>(sum, bias, args.alpha), args.C + (int64_t)row * args.ldc + col);
}

hipError_t launch_direct16(int epi, const GemmF32Args& a, hipStream_t stream) {
  const dim3 grid(a.tiles_m * a.tiles_n);
  const dim3 block(256);
#define EDSL_DIRECT16_CASE(E)                                                          \
  case E:                                                                              \
    hipLaunchKernelGGL((gemm_f32_direct16_kernel<E>), grid, block, 0, stream, a);     \
    break;
  switch (epi) {
    EDSL_DIRECT16_CASE(epi_code(false, ACT_NONE))
    EDSL_DIRECT16_CASE(epi_code(true, ACT_NONE))
    EDSL_DIRECT16_CASE(epi_code(false, ACT_RELU))
    EDSL_DIRECT16_CASE(epi_code(true, ACT_RELU))
    EDSL_DIRECT16_CASE(epi_code(false, ACT_LEAKY))
    EDSL_DIRECT16_CASE(epi_code(true, ACT_LEAKY))
    EDSL_DIRECT16_CASE(epi_code(false, ACT_IF_RELU))
    EDSL_DIRECT16_CASE(epi_code(true, ACT_IF_RELU))
    default:
      return hipErrorInvalidValue;
  }
#undef EDSL_DIRECT16_CASE
  return hipGetLastError();
}

// The R x C tile (16R x 16C outputs, K split over the four waves of a
// workgroup) for layers whose 64x64 tiles do not fill whole rounds of the
// CUs: 768^3 is 256 tiles of 48x48 (R = C = 3) and 1536^3 256 tiles of 96x96
// (R = C = 6), one workgroup per CU and one wave per SIMD, so every SIMD runs
// the same number of MFMAs in one round. Exact tiles take K a multiple of 16
// (at least 64); the edge twins (kEdge) take partial tiles and any K that is
// a multiple of 4, with the 128x128 edge twin's range-checked loads. Each wave computes the whole tile
// over a quarter of K with the 64x64 tile's A fragments and its loop (loads
// two 16-deep groups ahead in three register sets). B columns come in pieces
// of 64, 32 or 16 columns, read with 16-, 8- or 4-byte loads per lane and k
// slot: in a piece of width w (column blocks first .. first + w - 1) lane r16
// holds columns n0 + 16 first + w r16 + c, c < w, the c-th of them in column
// block first + c, so the lane's outputs of a row are w adjacent columns.
// The four partial tiles are summed through LDS in wave order; wave w
// finishes row 4g + w of every row block (R x C x 4 KiB of LDS: 144 KiB for
// 6 x 6).
template <int C>
struct ColPieces {
  static constexpr int n4 = C / 4, n2 = (C % 4) / 2, n1 = C % 2;
  static constexpr int count = n4 + n2 + n1;
  static constexpr int width(int p) { return p < n4 ? 4 : (p < n4 + n2 ? 2 : 1); }
  static constexpr int first(int p) {
    return p < n4 ? 4 * p : (p < n4 + n2 ? 4 * n4 + 2 * (p - n4) : 4 * n4 + 2 * n2);
  }
};

template <int W>
__device__ __forceinline__ void load_piece(float* dst, i32x4 rsrc, int voffset, int soffset) {
  if constexpr (W == 4) {
    const f32x4 v = raw_buffer_load_f32x4(rsrc, voffset, soffset, 0);
#pragma unroll
    for (int c = 0; c < 4; ++c) dst[c] = v[c];
  } else if constexpr (W == 2) {
    const f32x2 v = raw_buffer_load_f32x2(rsrc, voffset, soffset, 0);
    dst[0] = v[0];
    dst[1] = v[1];
  } else {
    dst[0] = raw_buffer_load_f32(rsrc, voffset, soffset, 0);
  }
}

template <int W>
struct VecOf;
template <>
struct VecOf<4> { using T = f32x4; };
template <>
struct VecOf<2> { using T = f32x2; };
template <>
struct VecOf<1> { using T = float; };

template <int R, int C, bool kEdge, int EPI>
__global__ void __launch_bounds__(256)
gemm_f32_direct_rc_kernel(GemmF32Args args) {
  using P = ColPieces<C>;
  constexpr int KS = 4;
  constexpr int kLoads = R + 4 * P::count;  // per group: one per row block, one per piece and k slot
  constexpr int kMfmas = 4 * R * C;         // per group
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4;
  const int r16 = lane & 15;
  int tm, tn;
  tile_coords(blockIdx.x, args.tiles_m, args.tiles_n, tm, tn);
  const int m0 = __builtin_amdgcn_readfirstlane(tm * 16 * R);
  const int n0 = __builtin_amdgcn_readfirstlane(tn * 16 * C);
  // The wave's groups jb .. jb + ngw - 1: K / 16 groups (K a multiple of 16,
  // at least 64) shared as evenly as they go, at least one per wave; edge
  // tiles: ceil(K / 16) groups, the last one partial, and a wave whose share
  // of a short K is empty skips the loop.
  const int K = args.K;
  const int ng = kEdge ? (K + 15) / 16 : K / 16;
  const int jb = wave * ng / KS;
  const int ngw = (wave + 1) * ng / KS - jb;
  const int lda = (int)args.lda, ldb = (int)args.ldb;
  const i32x4 rsrc_a = buffer_rsrc(args.A + (int64_t)m0 * lda, (int64_t)(args.M - m0) * lda * 4);
  const i32x4 rsrc_b = buffer_rsrc(args.B + n0, (int64_t)K * ldb * 4 - (int64_t)n0 * 4);
  const int va = (r16 * lda + 4 * g) * 4;  // A[m0 + 16i + r16][16j + 4g .. +3]
  int vb[P::count];                        // B[16j + 4g + s][piece columns of the lane]
  // Edge tiles, as for the 128x128 tile: per-lane row-block offsets (rows
  // past M out of range, and so are A chunks past K), each piece's columns
  // clamped to N - w (their outputs are never stored); the k row of B is in
  // the per-lane offset, so B rows past K read zero.
  int va_i[kEdge ? R : 1];
  static_for<P::count>([&](auto pc) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value;
    constexpr int W = P::width(p);
    const int col = kEdge ? min(n0 + 16 * P::first(p) + W * r16, args.N - W) : n0 + 16 * P::first(p) + W * r16;
    vb[p] = (4 * g * ldb + col - n0) * 4;
  });
  if constexpr (kEdge) {
#pragma unroll
    for (int i = 0; i < R; ++i) va_i[i] = va + i * 64 * lda;
  }

  struct Frag {
    f32x4 a[R];      // row block i: A[m0 + 16i + r16][16j + 4g .. +3]
    float b[4][C];   // k slot s, column block c
  };
  auto load = [&](Frag& f, int j) __attribute__((always_inline)) {
    if constexpr (!kEdge) {
#pragma unroll
      for (int i = 0; i < R; ++i) f.a[i] = raw_buffer_load_f32x4(rsrc_a, va, 64 * j + i * 64 * lda, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s)
        static_for<P::count>([&](auto pc) __attribute__((always_inline)) {
          constexpr int p = decltype(pc)::value;
          load_piece<P::width(p)>(&f.b[s][P::first(p)], rsrc_b, vb[p], (16 * j + s) * ldb * 4);
        });
    } else {
      const bool k_in = 16 * j + 4 * g < K;
#pragma unroll
      for (int i = 0; i < R; ++i)
        f.a[i] = raw_buffer_load_f32x4(rsrc_a, k_in ? va_i[i] : kOutOfRange, 64 * j, 0);
      const int rowj = 16 * j * ldb * 4;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        static_for<P::count>([&](auto pc) __attribute__((always_inline)) {
          constexpr int p = decltype(pc)::value;
          load_piece<P::width(p)>(&f.b[s][P::first(p)], rsrc_b, vb[p] + rowj, s * ldb * 4);
        });
    }
  };
  // The bias values of the lane's columns, loaded before the first group.
  float biasv[C];
  static_for<P::count>([&](auto pc) __attribute__((always_inline)) {
    constexpr int p = decltype(pc)::value;
    constexpr int W = P::width(p);
#pragma unroll
    for (int c = 0; c < W; ++c) biasv[P::first(p) + c] = 0.0f;
    const int col = n0 + 16 * P::first(p) + W * r16;
    if (epi_has_bias(EPI) && (!kEdge || col < args.N)) {
      const typename VecOf<W>::T v = *reinterpret_cast<const typename VecOf<W>::T*>(args.bias + col);
      if constexpr (W == 1) {
        biasv[P::first(p)] = v;
      } else {
#pragma unroll
        for (int c = 0; c < W; ++c) biasv[P::first(p) + c] = v[c];
      }
    }
  });
  f32x4 acc[R][C];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[i][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto mfmas = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < R; ++i)
#pragma unroll
        for (int c = 0; c < C; ++c)
          acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i][s], f.b[s][c], acc[i][c], 0, 0, 0);
  };
  // The group's loads spread evenly over its MFMAs.
  auto pin = [&]() __attribute__((always_inline)) {
    static_for<kLoads>([&](auto qc) __attribute__((always_inline)) {
      constexpr int q = decltype(qc)::value;
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, (q + 1) * kMfmas / kLoads - q * kMfmas / kLoads, 0);
    });
    __builtin_amdgcn_sched_barrier(0);
  };

  // Group jb + t is computed from set t % 3 while groups jb + t + 1 and
  // jb + t + 2 are in flight; loads past the wave's last group repeat it.
  const int jl = jb + ngw - 1;
  if (!kEdge || ngw > 0) {
    Frag fr[kSets64];
    load(fr[0], jb);
    load(fr[1], min(jb + 1, jl));
    int t = 0;
    for (; t + kSets64 <= ngw; t += kSets64) {
      static_for<kSets64>([&](auto sc) __attribute__((always_inline)) {
        constexpr int S = decltype(sc)::value;
        load(fr[(S + 2) % kSets64], min(jb + t + S + 2, jl));
        mfmas(fr[S]);
        pin();
      });
    }
    static_for<kSets64>([&](auto sc) __attribute__((always_inline)) {
      constexpr int S = decltype(sc)::value;
      if (t + S < ngw) {
        load(fr[(S + 2) % kSets64], min(jb + t + S + 2, jl));
        mfmas(fr[S]);
      }
    });
  }

  // LDS [wave][row block][e][column block][lane]: per (wave, i, e) the lane's
  // w adjacent columns of each piece as one vector, 64 lanes contiguous.
  __shared__ float red[KS * R * 4 * C * 64];
  auto base = [&](int w, int i, int e) { return ((w * R + i) * 4 + e) * C * 64; };
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      static_for<P::count>([&](auto pc) __attribute__((always_inline)) {
        constexpr int p = decltype(pc)::value;
        constexpr int W = P::width(p);
        constexpr int c0 = P::first(p);
        float* dst = red + base(wave, i, e) + c0 * 64 + lane * W;
        if constexpr (W == 4) {
          *reinterpret_cast<f32x4*>(dst) = f32x4{acc[i][c0][e], acc[i][c0 + 1][e], acc[i][c0 + 2][e], acc[i][c0 + 3][e]};
        } else if constexpr (W == 2) {
          *reinterpret_cast<f32x2*>(dst) = f32x2{acc[i][c0][e], acc[i][c0 + 1][e]};
        } else {
          *dst = acc[i][c0][e];
        }
      });
  __syncthreads();
  const float alpha = args.alpha;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int row = m0 + 16 * i + 4 * g + wave;
    static_for<P::count>([&](auto pc) __attribute__((always_inline)) {
      constexpr int p = decltype(pc)::value;
      constexpr int W = P::width(p);
      constexpr int c0 = P::first(p);
      using V = typename VecOf<W>::T;
      V sum = *reinterpret_cast<const V*>(red + base(0, i, wave) + c0 * 64 + lane * W);
#pragma unroll
      for (int w = 1; w < KS; ++w) {
        const V part = *reinterpret_cast<const V*>(red + base(w, i, wave) + c0 * 64 + lane * W);
        if constexpr (W == 1) {
          sum = __fadd_rn(sum, part);
        } else {
#pragma unroll
          for (int c = 0; c < W; ++c) sum[c] = __fadd_rn(sum[c], part[c]);
        }
      }
      V out;
      if constexpr (W == 1) {
        out = apply_epilogue_f32<EPI>(sum, biasv[c0], alpha);
      } else {
#pragma unroll
        for (int c = 0; c < W; ++c) out[c] = apply_epilogue_f32<EPI>(sum[c], biasv[c0 + c], alpha);
      }
      const int col = n0 + 16 * c0 + W * r16;
      if (!kEdge || (row < args.M && col < args.N))
        __builtin_nontemporal_store(out, reinterpret_cast<V*>(args.C + (int64_t)row * args.ldc + col));
    });
  }
}

template <int R, int C, bool kEdge = false>
hipError_t launch_rc(int epi, const GemmF32Args& a, hipStream_t stream) {
  const dim3 grid(a.tiles_m * a.tiles_n);
  const dim3 block(256);
#define EDSL_DIRECT_RC_CASE(E)                                                                    \
  case E:                                                                                         \
    hipLaunchKernelGGL((gemm_f32_direct_rc_kernel<R, C, kEdge, E>), grid, block, 0, stream, a);  \
    break;
  switch (epi) {
    EDSL_DIRECT_RC_CASE(epi_code(false, ACT_NONE))
    EDSL_DIRECT_RC_CASE(epi_code(true, ACT_NONE))
    EDSL_DIRECT_RC_CASE(epi_code(false, ACT_RELU))
    EDSL_DIRECT_RC_CASE(epi_code(true, ACT_RELU))
    EDSL_DIRECT_RC_CASE(epi_code(false, ACT_LEAKY))
    EDSL_DIRECT_RC_CASE(epi_code(true, ACT_LEAKY))
    EDSL_DIRECT_RC_CASE(epi_code(false, ACT_IF_RELU))
    EDSL_DIRECT_RC_CASE(epi_code(true, ACT_IF_RELU))
    default:
      return hipErrorInvalidValue;
  }
#undef EDSL_DIRECT_RC_CASE
  return hipGetLastError();
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

namespace {
// Shapes, strides and alignment every direct tile assumes (the planner only
// picks one for such layers; checked again here because a wrong launch reads
// out of bounds).
bool direct_operands_ok(int epi, const GemmF32Args& a) {
  if (a.M < 1 || a.N < 4 || a.K < 4 || a.N % 4 || a.K % 4) return false;
  if (a.lda < a.K || a.ldb < a.N || a.ldc < a.N || a.lda % 4 || a.ldb % 4 || a.ldc % 4) return false;
  const uintptr_t bias_bits = epi_has_bias(epi) ? (uintptr_t)a.bias : 0;
  if (((uintptr_t)a.A | (uintptr_t)a.B | (uintptr_t)a.C | bias_bits) % 16) return false;
  if (epi_has_bias(epi) && a.bias == nullptr) return false;
  return gemm_f32_direct_offsets_fit(a.K, a.lda, a.ldb);
}
}  // namespace

hipError_t launch_gemm_f32_direct(int guard, int epi, GemmF32Args a, hipStream_t stream) {
  if (!direct_operands_ok(epi, a)) return hipErrorInvalidValue;
  if (a.tiles_m != (a.M + kTile - 1) / kTile || a.tiles_n != (a.N + kTile - 1) / kTile) return hipErrorInvalidValue;
  if (guard == kGuardNone) {
    if (a.M % kTile || a.N % kTile || a.K % 16) return hipErrorInvalidValue;
    return launch_guard<kGuardNone>(epi, a, stream);
  }
  if (guard == kGuardEdge) return launch_guard<kGuardEdge>(epi, a, stream);
  return hipErrorInvalidValue;
}

hipError_t launch_gemm_f32_direct64(int ksplit, int guard, int epi, GemmF32Args a, hipStream_t stream) {
  if (!direct_operands_ok(epi, a)) return hipErrorInvalidValue;
  if (a.tiles_m != (a.M + 63) / 64 || a.tiles_n != (a.N + 63) / 64) return hipErrorInvalidValue;
  if (guard == kGuardNone) {
    if (a.M % 64 || a.N % 64 || a.K % (16 * ksplit)) return hipErrorInvalidValue;
    if (ksplit == 1) return launch_ks64<1, kGuardNone>(epi, a, stream);
    if (ksplit == 4) return launch_ks64<4, kGuardNone>(epi, a, stream);
  } else if (guard == kGuardEdge && ksplit == 4) {
    return launch_ks64<4, kGuardEdge>(epi, a, stream);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm_f32_direct16(int epi, GemmF32Args a, hipStream_t stream) {
  if (!direct_operands_ok(epi, a)) return hipErrorInvalidValue;
  if (a.M % 16 || a.N % 16 || a.K % 64 || a.K > 64 * kMaxGroups16) return hipErrorInvalidValue;
  if (a.tiles_m != a.M / 16 || a.tiles_n != a.N / 16) return hipErrorInvalidValue;
  return launch_direct16(epi, a, stream);
}

hipError_t launch_gemm_f32_direct_rc(int r, int c, int guard, int epi, GemmF32Args a, hipStream_t stream) {
  if (!direct_operands_ok(epi, a)) return hipErrorInvalidValue;
  if (r < 1 || c < 1) return hipErrorInvalidValue;
  if (a.tiles_m != (a.M + 16 * r - 1) / (16 * r) || a.tiles_n != (a.N + 16 * c - 1) / (16 * c)) return hipErrorInvalidValue;
  if (guard == kGuardEdge) {  // any M; N and K multiples of 4 (direct_operands_ok)
    if (r == 2 && c == 2) return launch_rc<2, 2, true>(epi, a, stream);
    if (r == 3 && c == 3) return launch_rc<3, 3, true>(epi, a, stream);
    if (r == 4 && c == 4) return launch_rc<4, 4, true>(epi, a, stream);
    if (r == 5 && c == 5) return launch_rc<5, 5, true>(epi, a, stream);
    if (r == 6 && c == 6) return launch_rc<6, 6, true>(epi, a, stream);
    return hipErrorInvalidValue;
  }
  if (guard != kGuardNone || a.M % (16 * r) || a.N % (16 * c) || a.K % 16 || a.K < 64) return hipErrorInvalidValue;
  if (r == 2 && c == 2) return launch_rc<2, 2>(epi, a, stream);
  if (r == 3 && c == 3) return launch_rc<3, 3>(epi, a, stream);
  if (r == 5 && c == 5) return launch_rc<5, 5>(epi, a, stream);
  if (r == 6 && c == 6) return launch_rc<6, 6>(epi, a, stream);
  if (r == 3 && c == 6) return launch_rc<3, 6>(epi, a, stream);
  if (r == 6 && c == 3) return launch_rc<6, 3>(epi, a, stream);
  if (r == 4 && c == 4) return launch_rc<4, 4>(epi, a, stream);
  return hipErrorInvalidValue;
}

}  // namespace edsl
