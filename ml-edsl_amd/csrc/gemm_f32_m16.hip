// fp32 dense layer / matmul on 16x16 MFMA blocks, one or two waves per SIMD.
//
// C[M,N] = epilogue(A[M,K] x B[K,N] (+ bias[N])) -- the same op as the
// 32x32-block tiles of gemm_f32.hip (reference
// cpp/src/builders/LinalgBuilder.cpp:106-139, 180-239, 301-339), for
// 16-byte aligned operands (edge twins for partial tiles, and an any-shape
// twin of the 128x128 tile with 4-byte accesses).
//
// Design (per workgroup, one output tile; the layouts are listed below):
//  * v_mfma_f32_16x16x4_f32: lane l supplies A[row l%16][k-slot l/16] and
//    B[k-slot l/16][col l%16] and receives rows 4*(l/16)..+3 of column l%16.
//    A 64x64 wave tile is 4x4 such blocks: 16 independent accumulators, so the
//    matrix core never waits on a result and the wave has room to issue its
//    LDS reads, global loads and LDS stores between MFMAs.
//  * Lane group g = l/16 owns k = 16j + 4g .. 16j + 4g + 3 of each 16-deep
//    group j: one ds_read_b128 of its A row per row block gives the four
//    k-slots of four MFMA steps, and for each of those k one ds_read_b128 (or
//    b64) of CB consecutive B columns gives the B operand of the CB column
//    blocks. Column block c therefore holds output columns wn0 + CB*(l%16) + c:
//    each lane ends with CB consecutive columns of a row, one vector store.
//  * LDS is double buffered; the global loads run PF K steps ahead in a ring
//    of register sets; each step's last group of MFMAs is issued after the
//    barrier that ends the step, behind the next step's loads and first
//    fragment reads; scheduling group barriers spread each group's fragment
//    reads, the global loads and the LDS stores over the MFMAs.
//  * A rows are stored with the 16-byte chunk index XOR-ed by a row hash so
//    that the 16 lanes of a ds_read_b128 phase hit distinct banks; B rows are
//    read 256 contiguous bytes per phase.
//  * Workgroups map to tiles XCD-aware (common.hpp: tile_coords); C is written
//    with non-temporal stores.
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

// 16-byte chunk position of chunk q in A row `row` (KCH chunks per row): the
// 16 rows a ds_read_b128 phase reads at one chunk index land on 16 distinct
// 16-byte bank groups of the 256-byte bank line.
template <int KCH>
__device__ __forceinline__ int a_slot(int row, int q) {
  if constexpr (KCH >= 16) return q ^ (row % KCH);
  else return q ^ ((row / (16 / KCH)) % KCH);
}

constexpr int PF = 2;    // K steps of global loads in flight

// Tile layouts (WM x WN waves over the tile):
//  kLarge: 128x128 tile, 2x2 waves of 64x64 (4x4 MFMA blocks), 32-deep K steps,
//          two workgroups per CU;
//  kSmall: 64x64 tile, 2x2 waves of 32x32 (2x2 MFMA blocks), 64-deep K steps,
//          for shapes whose 128x128 tiles would leave CUs idle (1024^3:
//          256 tiles of 64x64);
//  kWide:  128x256 tile, 2x4 waves of 64x64, 32-deep K steps, one workgroup
//          of eight waves per CU (96 KiB of LDS);
//  kLarge8: 128x128 tile, 2x4 waves of 64x32, 32-deep K steps, for exactly
//          one tile per CU (two waves per SIMD).
enum : int { kLarge = 0, kSmall = 1, kWide = 2, kLarge8 = 3 };
template <int L> struct Layout;
template <> struct Layout<kLarge> {
  static constexpr int BM = 128, BN = 128, BK = 32, WM = 2, WN = 2;
};
template <> struct Layout<kSmall> {
  static constexpr int BM = 64, BN = 64, BK = 64, WM = 2, WN = 2;
};
template <> struct Layout<kWide> {
  static constexpr int BM = 128, BN = 256, BK = 32, WM = 2, WN = 4;
};
template <> struct Layout<kLarge8> {
  static constexpr int BM = 128, BN = 128, BK = 32, WM = 2, WN = 4;
};

template <int N> struct VecT;
template <> struct VecT<2> { using type = f32x2; };
template <> struct VecT<4> { using type = f32x4; };

// n items spread over `slices` slices: the count of slice t.
constexpr int share(int n, int slices, int t) { return n / slices + (t < n % slices ? 1 : 0); }

// GUARD: kGuardNone (M, N multiples of the tile, K of BK), kGuardEdge (partial
// tiles and a partial last K step; 16-byte aligned rows, N and K multiples of
// 4) or kGuardScalar (any shape and alignment). The edge twin clamps the
// tile's rows past M to row M-1 and its columns past N to N-4
// (loop-invariant; those outputs are never stored), runs the whole K steps
// through the same pipeline, then the partial step once with loads past K
// skipped and zero, and stores only inside M x N. The any-shape twin does the
// same with 4-byte loads and stores: a 16-byte chunk of an A row is four
// loads at one address with immediate offsets, B columns past N read column
// N-1, and the partial step zeroes each element past K.
template <int L, int GUARD, int EPI>
__global__ void __launch_bounds__(Layout<L>::WM * Layout<L>::WN * 64, 2)
gemm_f32_m16_kernel(GemmF32Args args) {
  constexpr int kThreads = Layout<L>::WM * Layout<L>::WN * 64;
  constexpr bool kScalar = GUARD == kGuardScalar;
  constexpr bool kEdge = GUARD == kGuardEdge || kScalar;  // partial tiles and K step
  static_assert(GUARD == kGuardNone || GUARD == kGuardEdge || kScalar, "guard");
  constexpr int kBM = Layout<L>::BM;
  constexpr int kBN = Layout<L>::BN;
  constexpr int BK = Layout<L>::BK;
  constexpr int RB = kBM / Layout<L>::WM / 16;  // 16-row MFMA blocks of a wave tile
  constexpr int CB = kBN / Layout<L>::WN / 16;  // 16-column MFMA blocks of a wave tile
  constexpr int KCH = BK / 4;        // 16-byte chunks of an A row
  constexpr int G = BK / 16;         // 16-deep groups of a K step
  constexpr int A_F4 = kBM * KCH;
  constexpr int B_F4 = BK * kBN / 4;
  constexpr int A_LD = A_F4 / kThreads;
  constexpr int B_LD = B_F4 / kThreads;
  constexpr int NW = A_LD + B_LD;    // global loads, and LDS stores, of one K step per lane
  constexpr int NR = RB + 4;         // fragment reads of one group
  constexpr int NM = 4 * RB * CB;    // MFMAs of one group
  using bvec = typename VecT<CB>::type;
  static_assert(BK % 16 == 0 && KCH <= 32 && G % 2 == 0, "BK");
  static_assert(A_F4 % kThreads == 0 && B_F4 % kThreads == 0, "tile loads must divide evenly");
  static_assert(PF == 2, "prefetch depth");
  __shared__ f32x4 sA[2][A_F4];
  __shared__ __attribute__((aligned(16))) float sB[2][BK * kBN];  // 16-byte rows: f32x4 stores and reads

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wt = wave % (Layout<L>::WM * Layout<L>::WN);  // the wave's tile
  const int g = lane >> 4;
  const int r16 = lane & 15;
  const int wm0 = (wt / Layout<L>::WN) * (kBM / Layout<L>::WM);
  const int wn0 = (wt % Layout<L>::WN) * (kBN / Layout<L>::WN);
  int tm, tn;
  tile_coords(blockIdx.x, args.tiles_m, args.tiles_n, tm, tn);
  const int m0 = tm * kBM;
  const int n0 = tn * kBN;
  const int nk = args.K / BK;

  const float* a_src[A_LD];
  int a_dst[A_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int idx = tid + i * kThreads;
    const int r = idx / KCH;
    const int q = idx % KCH;
    a_src[i] = args.A + (int64_t)(kEdge ? min(m0 + r, args.M - 1) : m0 + r) * args.lda + 4 * q;
    a_dst[i] = r * KCH + a_slot<KCH>(r, q);
  }
  const float* b_src[B_LD];
  int b_dst[B_LD];
  // A lane's B chunks all start at the same column (kThreads is a multiple of
  // the kBN/4 lanes that cover a row).
  static_assert(kThreads % (kBN / 4) == 0, "B chunk columns");
  const int b_col = n0 + 4 * (tid % (kBN / 4));
#pragma unroll
  for (int i = 0; i < B_LD; ++i) {
    const int idx = tid + i * kThreads;
    const int r = idx / (kBN / 4);
    const int c = 4 * (idx % (kBN / 4));
    b_src[i] = args.B + (int64_t)r * args.ldb + (kScalar ? 0 : kEdge ? min(n0 + c, args.N - 4) : n0 + c);
    b_dst[i] = r * kBN + c;
  }
  // Any-shape twin: element e of a lane's B chunk, column min(b_col + e, N-1).
  auto b_elem = [&](int i, int64_t row_off, int e) -> float {
    return b_src[i][row_off + min(b_col + e, args.N - 1)];
  };

  f32x4 ra[PF][A_LD];
  f32x4 rb[PF][B_LD];
  auto load_global = [&](auto set, int kt) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    const int k0 = kt * BK;
    if constexpr (kScalar) {
#pragma unroll
      for (int i = 0; i < A_LD; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) ra[S][i][e] = a_src[i][k0 + e];
#pragma unroll
      for (int i = 0; i < B_LD; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) rb[S][i][e] = b_elem(i, (int64_t)k0 * args.ldb, e);
    } else {
#pragma unroll
      for (int i = 0; i < A_LD; ++i) ra[S][i] = *reinterpret_cast<const f32x4*>(a_src[i] + k0);
#pragma unroll
      for (int i = 0; i < B_LD; ++i)
        rb[S][i] = *reinterpret_cast<const f32x4*>(b_src[i] + (int64_t)k0 * args.ldb);
    }
  };
  auto store_lds = [&](auto set, int buf) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
#pragma unroll
    for (int i = 0; i < A_LD; ++i) sA[buf][a_dst[i]] = ra[S][i];
#pragma unroll
    for (int i = 0; i < B_LD; ++i) *reinterpret_cast<f32x4*>(&sB[buf][b_dst[i]]) = rb[S][i];
  };

  // The epilogue's bias values, loaded before the first K step's tile so
  // that their latency hides behind it.
  const int col0 = n0 + wn0 + CB * r16;
  bvec biasv = {};
  if constexpr (epi_has_bias(EPI)) {
    if constexpr (kScalar) {
#pragma unroll
      for (int c = 0; c < CB; ++c) biasv[c] = col0 + c < args.N ? args.bias[col0 + c] : 0.0f;
    } else if (!kEdge || col0 < args.N) {
      biasv = *reinterpret_cast<const bvec*>(args.bias + col0);
    }
  }

  f32x4 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int c = 0; c < CB; ++c) acc[i][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  struct Frag {
    f32x4 a[RB];  // row block i: A[wm0 + 16i + r16][16j + 4g .. +3]
    bvec b[4];    // step s: B[16j + 4g + s][wn0 + CB*r16 .. +CB-1]
  };
  auto read_frag = [&](int buf, int j, Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int row = wm0 + 16 * i + r16;
      f.a[i] = sA[buf][row * KCH + a_slot<KCH>(row, 4 * j + g)];
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // The element offset is a multiple of CB floats. With four columns per
      // block, stating that alignment keeps every read a ds_read_b128: some
      // were split into ds_read2_b32 pairs, whose 4-byte lanes conflict in the
      // LDS banks (4096^3: 37.7M conflict cycles per launch, now 0; 0.3-0.8 %
      // faster). The two-column layouts measured 2-3 % slower with it (all
      // their reads became ds_read2_b64) and keep the 4-byte alignment the
      // compiler infers from the float array.
      if constexpr (CB == 4)
        f.b[s] = *static_cast<const bvec*>(
            __builtin_assume_aligned(&sB[buf][(16 * j + 4 * g + s) * kBN + wn0 + CB * r16], 16));
      else
        f.b[s] = *reinterpret_cast<const bvec*>(&sB[buf][(16 * j + 4 * g + s) * kBN + wn0 + CB * r16]);
    }
  };
  auto mfmas = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int c = 0; c < CB; ++c)
          acc[i][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i][s], f.b[s][c], acc[i][c], 0, 0, 0);
  };

  // The instruction order inside each group's MFMAs is pinned with
  // scheduling group barriers: the next group's fragment reads spread over
  // the MFMAs (the compiler otherwise sinks the reads to just before their
  // first use, and every group starts with an LDS wait), with the global
  // loads or the LDS stores of the step between them. Same box, 4096^3:
  // 965 us, against 981 us with each group's reads issued as one burst and
  // 986 us for the 256x256 tile of gemm_f32.hip; the same reads and stores
  // in the first half of the group measured 980 us.
  constexpr int kSlices = NM < 8 ? NM : 8;
  // Slices that take the fragment reads: all of them, except for the one-wave
  // 64x64 tile, whose groups are only 16 MFMAs long: there the reads go in the
  // first half, so that they have landed when the next group starts (5120^3
  // 2013 -> 1943 us, 4096x4096x512 134.5 -> 130.3 us, 3072^3 443.6 -> 430.5 us;
  // the same for the 64-MFMA groups of the 128x256 tile measured 2 % slower).
  constexpr int kReadSlices = L == kSmall ? kSlices / 2 : kSlices;
  auto pin = [&](auto vmem, auto stores) __attribute__((always_inline)) {
    constexpr int V = decltype(vmem)::value, W = decltype(stores)::value;
    static_for<kSlices>([&](auto tc) __attribute__((always_inline)) {
      constexpr int t = decltype(tc)::value;
      if constexpr (share(V, kSlices, t) > 0) __builtin_amdgcn_sched_group_barrier(0x020, share(V, kSlices, t), 0);
      if constexpr (t < kReadSlices && share(NR, kReadSlices, t) > 0)
        __builtin_amdgcn_sched_group_barrier(0x100, share(NR, kReadSlices, t), 0);
      constexpr int m = share(NM, kSlices, t);
      if constexpr (share(W, kSlices, t) > 0) {
        __builtin_amdgcn_sched_group_barrier(0x008, m / 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, share(W, kSlices, t), 0);
        __builtin_amdgcn_sched_group_barrier(0x008, m - m / 2, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x008, m, 0);
      }
    });
    __builtin_amdgcn_sched_barrier(0);
  };

  // Each K step's last group of MFMAs is issued after the barrier that ends
  // the step, behind the next step's global loads and first fragment reads,
  // so the matrix core has work while those are in flight. Groups alternate
  // between the fragment sets f0 and f1 (G is even, so a step's last group
  // is in f1). The first step is peeled: it has no earlier group to finish.
  Frag f0, f1;

  if (nk > 0) {
    // PF K steps of global loads in flight, in a ring of PF register sets
    // (step s lives in set s % PF). While step kt is computed from LDS buffer
    // kt & 1, step kt + 1 goes to the other buffer and step kt + PF is loaded
    // into the set step kt left. Loads past the last step repeat the last
    // step (in bounds, never used), so the loop body has no branch.
    static_for<PF>([&](auto s) { load_global(s, min((int)decltype(s)::value, nk - 1)); });
    store_lds(Ic<0>{}, 0);
    __syncthreads();
    auto step = [&](auto cur, int kt, auto first) __attribute__((always_inline)) {
      constexpr int C = decltype(cur)::value;
      const int buf = kt & 1;
      load_global(Ic<C>{}, min(kt + PF, nk - 1));
      read_frag(buf, 0, f0);
      if constexpr (!decltype(first)::value) mfmas(f1);  // the previous step's last group
      pin(Ic<(kScalar ? 4 : 1) * NW>{}, Ic<0>{});
      static_for<G - 1>([&](auto jc) __attribute__((always_inline)) {
        constexpr int j = decltype(jc)::value;
        if constexpr (j % 2 == 0) {
          read_frag(buf, j + 1, f1);
          mfmas(f0);
        } else {
          read_frag(buf, j + 1, f0);
          mfmas(f1);
        }
        // The next step's LDS stores go with the first group (LDS buffer
        // buf ^ 1 was last read before the previous barrier).
        if constexpr (j == 0) {
          store_lds(Ic<(C + 1) % PF>{}, buf ^ 1);
          pin(Ic<0>{}, Ic<NW>{});
        } else {
          pin(Ic<0>{}, Ic<0>{});
        }
      });
      __syncthreads();
    };
    // Step kt uses register set kt % PF; after the peeled step 0 every
    // block of PF steps starts at kt = 1 (mod PF).
    step(Ic<0>{}, 0, Ic<1>{});
    int kt = 1;
    for (; kt + PF <= nk; kt += PF)
      static_for<PF>([&](auto s) { step(Ic<(decltype(s)::value + 1) % PF>{}, kt + decltype(s)::value, Ic<0>{}); });
    static_for<PF>([&](auto s) {
      if (kt + decltype(s)::value < nk) step(Ic<(decltype(s)::value + 1) % PF>{}, kt + decltype(s)::value, Ic<0>{});
    });
    mfmas(f1);
  }

  if constexpr (kEdge) {
    // The partial last K step, zero past K, through LDS buffer 0 (every
    // wave's last fragment reads came before the loop's last barrier).
    const int k0 = nk * BK;
    if (k0 < args.K) {
#pragma unroll
      for (int i = 0; i < A_LD; ++i) {
        const int q = (tid + i * kThreads) % KCH;
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (kScalar) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (k0 + 4 * q + e < args.K) v[e] = a_src[i][k0 + e];
        } else if (k0 + 4 * q < args.K) {
          v = *reinterpret_cast<const f32x4*>(a_src[i] + k0);
        }
        ra[0][i] = v;
      }
#pragma unroll
      for (int i = 0; i < B_LD; ++i) {
        const int r = (tid + i * kThreads) / (kBN / 4);
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        if (k0 + r < args.K) {
          if constexpr (kScalar) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = b_elem(i, (int64_t)k0 * args.ldb, e);
          } else {
            v = *reinterpret_cast<const f32x4*>(b_src[i] + (int64_t)k0 * args.ldb);
          }
        }
        rb[0][i] = v;
      }
      store_lds(Ic<0>{}, 0);
      __syncthreads();
      static_for<G>([&](auto jc) __attribute__((always_inline)) {
        read_frag(0, decltype(jc)::value, f0);
        mfmas(f0);
      });
    }
  }

  // Epilogue: lane holds rows wm0 + 16i + 4g + e and columns col0 .. col0+CB-1.
  const float alpha = args.alpha;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = m0 + wm0 + 16 * i + 4 * g + e;
      bvec v;
#pragma unroll
      for (int c = 0; c < CB; ++c) v[c] = apply_epilogue_f32<EPI>(acc[i][c][e], biasv[c], alpha);
      float* dst = args.C + (int64_t)row * args.ldc + col0;
      if constexpr (kScalar) {
        if (row < args.M) {
#pragma unroll
          for (int c = 0; c < CB; ++c)
            if (col0 + c < args.N) __builtin_nontemporal_store(v[c], dst + c);
        }
      } else if (!kEdge || (row < args.M && col0 < args.N)) {
        __builtin_nontemporal_store(v, reinterpret_cast<bvec*>(dst));
      }
    }
  }
}

}  // namespace

namespace {
template <int L, int GUARD>
hipError_t launch_layout(int epi, const GemmF32Args& a, hipStream_t stream) {
  constexpr int BM = Layout<L>::BM, BN = Layout<L>::BN, BK = Layout<L>::BK;
  if (GUARD == kGuardNone) {
    if (a.M % BM || a.N % BN || a.K <= 0 || a.K % BK) return hipErrorInvalidValue;
  } else if (GUARD == kGuardEdge) {
    if (a.M < 1 || a.N < 4 || a.K < 4 || a.N % 4 || a.K % 4) return hipErrorInvalidValue;
  } else if (a.M < 1 || a.N < 1 || a.K < 1) {
    return hipErrorInvalidValue;
  }
  if (a.tiles_m != (a.M + BM - 1) / BM || a.tiles_n != (a.N + BN - 1) / BN) return hipErrorInvalidValue;
  const dim3 grid(a.tiles_m * a.tiles_n);
  const dim3 block(Layout<L>::WM * Layout<L>::WN * 64);
#define EDSL_M16_CASE(E)                                                                \
  case E:                                                                               \
    hipLaunchKernelGGL((gemm_f32_m16_kernel<L, GUARD, E>), grid, block, 0, stream, a);  \
    break;
  switch (epi) {
    EDSL_M16_CASE(epi_code(false, ACT_NONE))
    EDSL_M16_CASE(epi_code(true, ACT_NONE))
    EDSL_M16_CASE(epi_code(false, ACT_RELU))
    EDSL_M16_CASE(epi_code(true, ACT_RELU))
    EDSL_M16_CASE(epi_code(false, ACT_LEAKY))
    EDSL_M16_CASE(epi_code(true, ACT_LEAKY))
    EDSL_M16_CASE(epi_code(false, ACT_IF_RELU))
    EDSL_M16_CASE(epi_code(true, ACT_IF_RELU))
    default:
      return hipErrorInvalidValue;
  }
#undef EDSL_M16_CASE
  return hipGetLastError();
}
}  // namespace

hipError_t launch_gemm_f32_m16(int layout, int guard, int epi, GemmF32Args a, hipStream_t stream) {
  switch (layout * 4 + guard) {
    case kLarge * 4 + kGuardNone: return launch_layout<kLarge, kGuardNone>(epi, a, stream);
    case kLarge * 4 + kGuardEdge: return launch_layout<kLarge, kGuardEdge>(epi, a, stream);
    case kLarge * 4 + kGuardScalar: return launch_layout<kLarge, kGuardScalar>(epi, a, stream);
    case kSmall * 4 + kGuardNone: return launch_layout<kSmall, kGuardNone>(epi, a, stream);
    case kSmall * 4 + kGuardEdge: return launch_layout<kSmall, kGuardEdge>(epi, a, stream);
    case kWide * 4 + kGuardNone: return launch_layout<kWide, kGuardNone>(epi, a, stream);
    case kWide * 4 + kGuardEdge: return launch_layout<kWide, kGuardEdge>(epi, a, stream);
    case kLarge8 * 4 + kGuardNone: return launch_layout<kLarge8, kGuardNone>(epi, a, stream);
    case kLarge8 * 4 + kGuardEdge: return launch_layout<kLarge8, kGuardEdge>(epi, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace edsl
