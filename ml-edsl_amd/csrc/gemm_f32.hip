// fp32 dense layer / matmul on gfx950 matrix cores.
//
// C[M,N] = epilogue(A[M,K] x B[K,N] (+ bias[N])), fp32 accumulate.
//
// This realises, as one kernel, the reference's fill + linalg.matmul + bias
// generic + ReLU generic chain (reference cpp/src/builders/LinalgBuilder.cpp:106-139,
// 180-239, 301-339), which the reference GPU lowering runs as three kernels
// (reference cpp/src/MLIRLowering.cpp:495-518): the zero fill becomes the
// register-zeroed accumulator, and bias + activation run on the accumulator
// registers before the one store of C.
//
// Design (per workgroup, one BM x BN output tile):
//  * K is walked in BK-deep steps; A and B tiles are staged in LDS, double
//    buffered, with the next step's global loads (16-byte, coalesced) issued
//    before the current step's MFMAs and written to the other LDS buffer after.
//  * v_mfma_f32_32x32x2_f32: lane l supplies A[row l%32][k-slot l/32] and
//    B[k-slot l/32][col l%32]. A lane reads 4 consecutive k of an A row with one
//    ds_read_b128, and for each of those k one ds_read_b{32,64,128} of CP
//    consecutive B columns. The two lane halves take k = 8j+s and 8j+4+s for
//    MFMA step s, so the same k pairs A and B. Column phase c of a wave tile
//    therefore holds output columns wn0 + CP*(l%32) + c, which gives each lane
//    CP consecutive columns in the epilogue: one vector store per row.
//  * A tiles are stored row-major in LDS with the 16-byte chunk index XOR-ed by
//    a row hash, so the 16 lanes of a ds_read_b128 phase hit distinct banks.
//  * Workgroups map to tiles XCD-aware (common.hpp: tile_coords).
//  * C is written with non-temporal stores.
#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>
#include <utility>

namespace edsl {
namespace {

template <int KCH>
__device__ __forceinline__ int a_swizzle(int row) {
  // A row holds KCH 16-byte chunks; the LDS has 64 four-byte banks (one
  // 256-byte bank line), and one ds_read_b128 phase serves 16 lanes, here 16
  // consecutive rows at one chunk index. Fewer than 16 chunks: 16/KCH rows
  // share a bank line, so rows 16/KCH apart rotate the chunk; 16 or more:
  // XOR with the row index (mod KCH). Either way the 16 rows land on distinct
  // 16-byte bank groups (SQ_LDS_BANK_CONFLICT reads 0 for the 256x256x16
  // tile, 1.6 cycles per LDS instruction with a 32-bank layout).
  if constexpr (KCH >= 16) return row % KCH;
  else return (row / (16 / KCH)) % KCH;
}

template <int CP>
__device__ __forceinline__ void load_b_frag(const float* p, float (&v)[CP]) {
  if constexpr (CP == 4) {
    const f32x4 t = *reinterpret_cast<const f32x4*>(p);
    v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
  } else if constexpr (CP == 2) {
    const f32x2 t = *reinterpret_cast<const f32x2*>(p);
    v[0] = t[0]; v[1] = t[1];
  } else {
    v[0] = *p;
  }
}

template <int N>
using Ic = std::integral_constant<int, N>;

// f(Ic<0>{}), f(Ic<1>{}), ..., f(Ic<N-1>{}) in order.
template <typename F, int... S>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, S...>) {
  (f(Ic<S>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// GUARD selects the bounds handling:
//  kGuardNone: M, N, K are multiples of the tile, operands 16-byte aligned.
//  kGuardEdge: partial tiles at the M, N and K edges; operands 16-byte aligned
//    with row strides, N and K multiples of 4. Loads stay 16-byte vectors at
//    clamped addresses: A rows past M read row M-1 and B columns past N read
//    columns N-4.., which only feed outputs that are never stored (the clamps
//    are loop-invariant). The K loop runs the whole BK steps; a partial last
//    step follows it once, with loads past K skipped and zero. Stores are
//    masked per vector (N % 4 == 0, so a vector of CP <= 4 columns is all in
//    or all out).
//  kGuardScalar: as kGuardEdge (whole K steps in the loop, then the partial
//    step; rows past M read row M-1, columns past N read column N-1), with
//    4-byte loads and stores: rows of any alignment, K and N of any value.
//    A chunk's 4 k of an A row are consecutive (one address, immediate
//    offsets); B columns are clamped only in tiles that reach past N.
//  kGuardAll: any shape and alignment; element-wise checked scalar loads/stores.
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int WAVES_K, int PF, int EPI, int GUARD,
          int SCHED = 0>
__global__ void __launch_bounds__(WAVES_M * WAVES_N * WAVES_K * 64)
gemm_f32_kernel(GemmF32Args args) {
  constexpr int NT = WAVES_M * WAVES_N * WAVES_K * 64;
  constexpr int WMN = WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M;
  constexpr int WN = BN / WAVES_N;
  constexpr int CP = WN / 32;
  constexpr int RB = WM / 32;
  constexpr int KCH = BK / 4;
  static_assert(WM % 32 == 0, "wave tile rows must be a multiple of 32");
  static_assert(WN == 32 * CP && (CP == 1 || CP == 2 || CP == 4), "wave tile cols");
  static_assert(BK % 8 == 0 && KCH <= 32 && (KCH & (KCH - 1)) == 0, "BK");
  static_assert((BK / 8) % WAVES_K == 0, "waves splitting K need equal shares of a K step");
  constexpr int JP = BK / 8 / WAVES_K;  // 8-k groups of a K step per wave
  constexpr int A_F4 = BM * KCH;
  constexpr int B_F4 = BK * BN / 4;
  static_assert(A_F4 % NT == 0 && B_F4 % NT == 0, "tile loads must divide evenly");
  constexpr int A_LD = A_F4 / NT;
  constexpr int B_LD = B_F4 / NT;

  // SCHED 0: a K step's LDS stores follow its MFMAs. SCHED 1 (tiles with
  // loads several steps ahead): the next step's LDS stores are issued right
  // after the step's first fragment reads, ahead of its MFMAs, so the LDS
  // writes them while the matrix cores run (c2 1024^3: 23.4-23.5 -> 23.0-23.1
  // us on one box).
  static_assert(SCHED == 0 || SCHED == 1, "schedule");
  static_assert(SCHED == 0 || (PF >= 2 && GUARD != kGuardAll), "schedule 1: prefetching vector tiles");
  __shared__ f32x4 sA[2][A_F4];
  __shared__ float sB[2][BK * BN];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_k = wave / WMN;
  const int wave_m = (wave % WMN) / WAVES_N;
  const int wave_n = wave % WAVES_N;
  int tm, tn;
  tile_coords(blockIdx.x, args.tiles_m, args.tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int M = args.M, N = args.N, K = args.K;

  static_assert(PF >= 1 && PF <= 4, "global prefetch depth");
  f32x4 ra[PF][A_LD];
  f32x4 rb[PF][B_LD];

  // Register set S receives the global tile loads of one K step. With the
  // edge guard the K loop runs whole steps only (`tail` false: no check in
  // k); a partial last step is loaded once, after the loop, with `tail` true.
  auto load_global = [&](auto set, int k0, auto tail) {
    constexpr int S = decltype(set)::value;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / KCH;
      const int q = idx % KCH;
      const int gm = m0 + r;
      const int gk = k0 + 4 * q;
      if constexpr (GUARD == kGuardNone) {
        ra[S][i] = *reinterpret_cast<const f32x4*>(args.A + (int64_t)gm * args.lda + gk);
      } else if constexpr (GUARD == kGuardEdge) {
        const float* src = args.A + (int64_t)min(gm, M - 1) * args.lda + gk;
        if constexpr (decltype(tail)::value) {
          f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
          if (gk < K) v = *reinterpret_cast<const f32x4*>(src);
          ra[S][i] = v;
        } else {
          ra[S][i] = *reinterpret_cast<const f32x4*>(src);
        }
      } else if constexpr (GUARD == kGuardScalar) {
        const float* src = args.A + (int64_t)min(gm, M - 1) * args.lda + gk;
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (decltype(tail)::value) v[e] = gk + e < K ? src[e] : 0.0f;
          else v[e] = src[e];
        }
        ra[S][i] = v;
      } else {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (gm < M && gk + e < K) ? args.A[(int64_t)gm * args.lda + gk + e] : 0.0f;
        ra[S][i] = v;
      }
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / (BN / 4);
      const int c = 4 * (idx % (BN / 4));
      const int gk = k0 + r;
      const int gn = n0 + c;
      if constexpr (GUARD == kGuardNone) {
        rb[S][i] = *reinterpret_cast<const f32x4*>(args.B + (int64_t)gk * args.ldb + gn);
      } else if constexpr (GUARD == kGuardEdge) {
        const float* src = args.B + (int64_t)gk * args.ldb + min(gn, N - 4);
        if constexpr (decltype(tail)::value) {
          f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
          if (gk < K) v = *reinterpret_cast<const f32x4*>(src);
          rb[S][i] = v;
        } else {
          rb[S][i] = *reinterpret_cast<const f32x4*>(src);
        }
      } else if constexpr (GUARD == kGuardScalar) {
        const bool in_k = !decltype(tail)::value || gk < K;
        const float* src = args.B + (int64_t)(in_k ? gk : K - 1) * args.ldb;
        f32x4 v;
        if (n0 + BN <= N) {  // uniform: the tile lies inside N
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = src[gn + e];
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = src[min(gn + e, N - 1)];
        }
        if constexpr (decltype(tail)::value) {
          if (!in_k) v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        rb[S][i] = v;
      } else {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (gk < K && gn + e < N) ? args.B[(int64_t)gk * args.ldb + gn + e] : 0.0f;
        rb[S][i] = v;
      }
    }
  };

  auto store_lds = [&](auto set, int buf) {
    constexpr int S = decltype(set)::value;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / KCH;
      const int q = idx % KCH;
      sA[buf][r * KCH + (q ^ a_swizzle<KCH>(r))] = ra[S][i];
    }
#pragma unroll
    for (int i = 0; i < B_LD; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / (BN / 4);
      const int c = 4 * (idx % (BN / 4));
      *reinterpret_cast<f32x4*>(&sB[buf][r * BN + c]) = rb[S][i];
    }
  };

  f32x16 acc[RB][CP];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int c = 0; c < CP; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][c][r] = 0.0f;

  const int half = lane >> 5;
  const int l32 = lane & 31;

  // The epilogue's bias values (columns col0 + c, c < CP), loaded before the
  // first K step's tile so that their latency hides behind it rather than
  // adding to the epilogue's.
  const int col0 = n0 + wave_n * WN + CP * l32;
  float bvals[CP];
#pragma unroll
  for (int c = 0; c < CP; ++c) bvals[c] = 0.0f;
  if constexpr (epi_has_bias(EPI)) {
    if constexpr (GUARD == kGuardNone) {
      load_b_frag<CP>(args.bias + col0, bvals);
    } else if constexpr (GUARD == kGuardEdge) {
      if (col0 < N) load_b_frag<CP>(args.bias + col0, bvals);
    } else {
#pragma unroll
      for (int c = 0; c < CP; ++c) bvals[c] = (col0 + c < N) ? args.bias[col0 + c] : 0.0f;
    }
  }

  // A wave raises its issue priority while it reads fragments and runs its
  // MFMAs, so waves with MFMAs ready win issue over waves issuing loads or
  // LDS stores (same box: c3 88.2 -> 88.5-88.8 % of peak, the 8-way c3
  // column shard +2.7 %, c2 unchanged).
  auto compute = [&](int buf) {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int jj = 0; jj < JP; ++jj) {
      const int j = wave_k * JP + jj;
      f32x4 a[RB];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int row = wave_m * WM + i * 32 + l32;
        const int q = 2 * j + half;
        a[i] = sA[buf][row * KCH + (q ^ a_swizzle<KCH>(row))];
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int k = 8 * j + 4 * half + s;
        float bv[CP];
        load_b_frag<CP>(&sB[buf][k * BN + wave_n * WN + CP * l32], bv);
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int c = 0; c < CP; ++c)
            acc[i][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], bv[c], acc[i][c], 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // SCHED 1: as compute(), with mid() issued right after the first 8-k
  // group's fragment reads.
  auto compute_mid = [&](int buf, auto&& mid) {
    __builtin_amdgcn_s_setprio(1);
    static_for<JP>([&](auto jjc) {
      constexpr int jj = decltype(jjc)::value;
      const int j = wave_k * JP + jj;
      f32x4 a[RB];
      float bv[4][CP];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int row = wave_m * WM + i * 32 + l32;
        const int q = 2 * j + half;
        a[i] = sA[buf][row * KCH + (q ^ a_swizzle<KCH>(row))];
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) load_b_frag<CP>(&sB[buf][(8 * j + 4 * half + s) * BN + wave_n * WN + CP * l32], bv[s]);
      if constexpr (jj == 0) {
        __builtin_amdgcn_sched_barrier(0);
        mid();
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
          for (int c = 0; c < CP; ++c)
            acc[i][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], bv[s][c], acc[i][c], 0, 0, 0);
    });
    __builtin_amdgcn_s_setprio(0);
  };

  // K steps of the main loop: all of them, or with the edge guard the whole
  // ones only (the partial step follows the loop).
  constexpr bool kPartialStep = GUARD == kGuardEdge || GUARD == kGuardScalar;
  const int nk = kPartialStep ? K / BK : (K + BK - 1) / BK;
  const std::false_type body{};
  if constexpr (PF == 1) {
    if (nk > 0) {
      load_global(Ic<0>{}, 0, body);
      store_lds(Ic<0>{}, 0);
      __syncthreads();
      for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) load_global(Ic<0>{}, (kt + 1) * BK, body);
        compute(buf);
        if (more) store_lds(Ic<0>{}, buf ^ 1);
        __syncthreads();
      }
    }
  } else if (nk > 0) {
    // PF K steps of global loads in flight, in a ring of PF register sets
    // (step s lives in set s % PF): while step kt is computed from LDS buffer
    // kt&1, step kt+1 (loaded PF-1 iterations earlier) goes to the other LDS
    // buffer and step kt+PF is loaded into set kt % PF, whose step went to the
    // LDS one iteration earlier. At depth 4, when PF divides the step count,
    // the last PF steps, already loaded, run without loads. Otherwise the
    // loads past the last step repeat the last step (in bounds, never used),
    // so the body has no branch and its wait counts stay exact.
    auto prologue = [&](auto set) {
      constexpr int S = decltype(set)::value;
      load_global(Ic<S>{}, min(S, nk - 1) * BK, body);
    };
    static_for<PF>(prologue);
    store_lds(Ic<0>{}, 0);
    __syncthreads();
    auto step = [&](auto cur, int kt) {
      constexpr int C = decltype(cur)::value;
      load_global(Ic<C>{}, min(kt + PF, nk - 1) * BK, body);
      // Keep the loads ahead of this step's MFMAs (the scheduler would
      // otherwise sink them and shorten their lead).
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (SCHED == 1) {
        // LDS buffer (kt + 1) & 1 was last read before the previous barrier.
        compute_mid(kt & 1, [&] { store_lds(Ic<(C + 1) % PF>{}, (kt + 1) & 1); });
      } else {
        compute(kt & 1);
        __builtin_amdgcn_sched_barrier(0);
        store_lds(Ic<(C + 1) % PF>{}, (kt + 1) & 1);
      }
      __syncthreads();
    };
    int kt = 0;
    // At depth 4 the repeated loads are 4 of every nk + 4 (1/9 at C2's 32
    // steps), and a tail without them measured 2% faster there. At depth 2
    // (2 of 66 at the 8-way C3 column shard, two workgroups per CU) the tail
    // measured 1-4% slower, so that depth keeps the repeated loads.
    if (PF >= 4 && nk % PF == 0) {
      // Every load of the loop is in range, and the last PF steps (already
      // loaded) run without loads: no step is fetched twice.
      for (; kt + PF < nk; kt += PF) {
        static_for<PF>([&](auto s) { step(s, kt + decltype(s)::value); });
      }
      static_for<PF>([&](auto s) {
        constexpr int C = decltype(s)::value;
        if constexpr (SCHED == 1 && C + 1 < PF) {
          compute_mid((kt + C) & 1, [&] { store_lds(Ic<C + 1>{}, (kt + C + 1) & 1); });
        } else {
          compute((kt + C) & 1);
        }
        if constexpr (SCHED != 1 && C + 1 < PF) {
          __builtin_amdgcn_sched_barrier(0);
          store_lds(Ic<C + 1>{}, (kt + C + 1) & 1);
        }
        // Also after the last step: the K-split reduction below reuses the
        // A tile's LDS.
        __syncthreads();
      });
    } else {
      for (; kt + PF <= nk; kt += PF) {
        static_for<PF>([&](auto s) { step(s, kt + decltype(s)::value); });
      }
      static_for<PF>([&](auto s) {
        if (kt + decltype(s)::value < nk) step(s, kt + decltype(s)::value);
      });
    }
  }
  if constexpr (kPartialStep) {
    // The partial last K step (K % BK != 0), zero past K. Every path above
    // ended with a barrier, so LDS buffer nk & 1 is free.
    if (nk * BK < K) {
      load_global(Ic<0>{}, nk * BK, std::true_type{});
      store_lds(Ic<0>{}, nk & 1);
      __syncthreads();
      compute(nk & 1);
      __syncthreads();
    }
  }

  // Waves that split K add their partial tiles into wave group 0 through
  // LDS, in wave order. The K loop ended with a barrier, so the A tile's LDS
  // is free and holds the partials when it is large enough.
  if constexpr (WAVES_K > 1) {
    using Red = f32x4[WAVES_K - 1][WMN][RB * CP * 4][64];
    Red* red_p;
    if constexpr (sizeof(Red) <= sizeof(sA)) {
      red_p = reinterpret_cast<Red*>(&sA[0][0]);
    } else {
      __shared__ Red red_own;
      red_p = &red_own;
    }
    Red& red = *red_p;
    if (wave_k > 0) {
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int c = 0; c < CP; ++c)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            red[wave_k - 1][wave % WMN][(i * CP + c) * 4 + q][lane] =
                f32x4{acc[i][c][4 * q], acc[i][c][4 * q + 1], acc[i][c][4 * q + 2], acc[i][c][4 * q + 3]};
    }
    __syncthreads();
    if (wave_k > 0) return;
#pragma unroll
    for (int w = 0; w < WAVES_K - 1; ++w)
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int c = 0; c < CP; ++c)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 t = red[w][wave % WMN][(i * CP + c) * 4 + q][lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][c][4 * q + e] += t[e];
          }
  }

  // Epilogue: lane holds rows rbase + 8*(r/4) + 4*half + r%4 of each 32-row
  // block and columns col0 + c, c < CP.
  const float alpha = args.alpha;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wave_m * WM + i * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
      float v[CP];
#pragma unroll
      for (int c = 0; c < CP; ++c) v[c] = apply_epilogue_f32<EPI>(acc[i][c][r], bvals[c], alpha);
      float* dst = args.C + (int64_t)row * args.ldc + col0;
      if constexpr (GUARD == kGuardNone || GUARD == kGuardEdge) {
        if (GUARD == kGuardNone || (row < M && col0 < N)) {
          // Non-temporal: C is not read again by this kernel (c2 23.0 ->
          // 22.6 us on one box; c1, c3 and the c3 column shard unchanged).
          if constexpr (CP == 4) {
            __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4*>(dst));
          } else if constexpr (CP == 2) {
            __builtin_nontemporal_store(f32x2{v[0], v[1]}, reinterpret_cast<f32x2*>(dst));
          } else {
            __builtin_nontemporal_store(v[0], dst);
          }
        }
      } else if constexpr (GUARD == kGuardScalar) {
        if (row < M) {
#pragma unroll
          for (int c = 0; c < CP; ++c)
            if (col0 + c < N) __builtin_nontemporal_store(v[c], dst + c);
        }
      } else {
        if (row < M) {
#pragma unroll
          for (int c = 0; c < CP; ++c)
            if (col0 + c < N) dst[c] = v[c];
        }
      }
    }
  }
}


template <int BM, int BN, int BK, int WMW, int WNW, int WKW, int GUARD, int PF = 1, int SCHED = 0>
hipError_t launch_cfg(int epi, const GemmF32Args& a, hipStream_t stream) {
  const dim3 grid(a.tiles_m * a.tiles_n);
  const dim3 block(WMW * WNW * WKW * 64);
#define EDSL_F32_CASE(E)                                                                           \
  case E:                                                                                          \
    hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, BK, WMW, WNW, WKW, PF, E, GUARD, SCHED>), grid, block, 0, \
                       stream, a);                                                                 \
    break;
  switch (epi) {
    EDSL_F32_CASE(epi_code(false, ACT_NONE))
    EDSL_F32_CASE(epi_code(true, ACT_NONE))
    EDSL_F32_CASE(epi_code(false, ACT_RELU))
    EDSL_F32_CASE(epi_code(true, ACT_RELU))
    EDSL_F32_CASE(epi_code(false, ACT_LEAKY))
    EDSL_F32_CASE(epi_code(true, ACT_LEAKY))
    EDSL_F32_CASE(epi_code(false, ACT_IF_RELU))
    EDSL_F32_CASE(epi_code(true, ACT_IF_RELU))
    default:
      return hipErrorInvalidValue;
  }
#undef EDSL_F32_CASE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_f32(int cfg, int epi, GemmF32Args a, hipStream_t stream) {
  switch (cfg) {
    case kF32Guard64: return launch_cfg<64, 64, 16, 2, 2, 1, kGuardAll>(epi, a, stream);
    case kF32T32: return launch_cfg<32, 32, 64, 1, 1, 4, kGuardNone, 4>(epi, a, stream);
    case kF32T32Edge: return launch_cfg<32, 32, 64, 1, 1, 4, kGuardEdge, 4>(epi, a, stream);
    case kF32T32Any: return launch_cfg<32, 32, 64, 1, 1, 4, kGuardScalar, 4>(epi, a, stream);
    case kF32T64Any: return launch_cfg<64, 64, 32, 2, 2, 2, kGuardScalar, 4, 1>(epi, a, stream);
    case kF32T64K2Any: return launch_cfg<64, 64, 64, 2, 2, 2, kGuardScalar, 2>(epi, a, stream);
    case kF32T256Any: return launch_cfg<256, 256, 16, 4, 4, 1, kGuardScalar>(epi, a, stream);
    case kF32M16_128: return launch_gemm_f32_m16(0, kGuardNone, epi, a, stream);
    case kF32M16_128Edge: return launch_gemm_f32_m16(0, kGuardEdge, epi, a, stream);
    case kF32M16_128Any: return launch_gemm_f32_m16(0, kGuardScalar, epi, a, stream);
    case kF32M16_64: return launch_gemm_f32_m16(1, kGuardNone, epi, a, stream);
    case kF32M16_64Edge: return launch_gemm_f32_m16(1, kGuardEdge, epi, a, stream);
    case kF32M16_128x256: return launch_gemm_f32_m16(2, kGuardNone, epi, a, stream);
    case kF32M16_128x256Edge: return launch_gemm_f32_m16(2, kGuardEdge, epi, a, stream);
    case kF32M16_128W8: return launch_gemm_f32_m16(3, kGuardNone, epi, a, stream);
    case kF32M16_128W8Edge: return launch_gemm_f32_m16(3, kGuardEdge, epi, a, stream);
    case kF32Direct128: return launch_gemm_f32_direct(kGuardNone, epi, a, stream);
    case kF32Direct128Edge: return launch_gemm_f32_direct(kGuardEdge, epi, a, stream);
    case kF32Direct64: return launch_gemm_f32_direct64(1, kGuardNone, epi, a, stream);
    case kF32Direct64K4: return launch_gemm_f32_direct64(4, kGuardNone, epi, a, stream);
    case kF32Direct64K4Edge: return launch_gemm_f32_direct64(4, kGuardEdge, epi, a, stream);
    case kF32Direct16K4: return launch_gemm_f32_direct16(epi, a, stream);
    case kF32DirectRC2x2: return launch_gemm_f32_direct_rc(2, 2, kGuardNone, epi, a, stream);
    case kF32DirectRC3x3: return launch_gemm_f32_direct_rc(3, 3, kGuardNone, epi, a, stream);
    case kF32DirectRC5x5: return launch_gemm_f32_direct_rc(5, 5, kGuardNone, epi, a, stream);
    case kF32DirectRC6x6: return launch_gemm_f32_direct_rc(6, 6, kGuardNone, epi, a, stream);
    case kF32DirectRC3x6: return launch_gemm_f32_direct_rc(3, 6, kGuardNone, epi, a, stream);
    case kF32DirectRC6x3: return launch_gemm_f32_direct_rc(6, 3, kGuardNone, epi, a, stream);
    case kF32DirectRC4x4: return launch_gemm_f32_direct_rc(4, 4, kGuardNone, epi, a, stream);
    case kF32DirectRC2x2Edge: return launch_gemm_f32_direct_rc(2, 2, kGuardEdge, epi, a, stream);
    case kF32DirectRC3x3Edge: return launch_gemm_f32_direct_rc(3, 3, kGuardEdge, epi, a, stream);
    case kF32DirectRC4x4Edge: return launch_gemm_f32_direct_rc(4, 4, kGuardEdge, epi, a, stream);
    case kF32DirectRC5x5Edge: return launch_gemm_f32_direct_rc(5, 5, kGuardEdge, epi, a, stream);
    case kF32DirectRC6x6Edge: return launch_gemm_f32_direct_rc(6, 6, kGuardEdge, epi, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace edsl
