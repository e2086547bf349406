// fp32 dense layer for small M (M <= 64): a weight-streaming kernel.
//
// Y[M,N] = epilogue(X[M,K] x W[K,N] (+ bias[N])) -- the same op as the tiled
// kernel (reference cpp/src/builders/LinalgBuilder.cpp:106-139, 180-239,
// 301-339), shaped for the HBM-bound case where W dominates the traffic
// (M=16, K=N=8192: W is 256 MiB, X and Y 512 KiB each).
//
// Every W element is read from HBM exactly once and used for all M rows at
// once on the matrix cores:
//  * v_mfma_f32_16x16x4_f32: lane l supplies X[row l%16][k-slot l/16] and
//    W[k-slot l/16][col l%16]. Lane group g = l/16 owns the k rows
//    k0+4g .. k0+4g+3 of each 16-row step: it loads those 4 k of its X row
//    with one 16-byte load and, for each k, CPL consecutive W columns with one
//    4*CPL-byte load. MFMA (step s, column phase c) pairs X[.][k0+4g+s] with
//    W[k0+4g+s][n0 + CPL*(l%16) + c], so lane l%16 accumulates columns
//    n0 + CPL*(l%16) + c: a wave owns 16*CPL columns and stores CPL per row.
//  * A workgroup is NW waves (4 for one row block, 8 for more) covering
//    `cols` adjacent columns: WN waves side by side (cols = 16*CPL*WN), and
//    WK = NW/WN waves splitting the workgroup's K range. The WK slices are
//    summed in LDS, in wave order. Fewer waves per CU keep fewer HBM rows
//    open at once: 16-wave workgroups were 2-3 % slower at M=16, K=N=8192,
//    6-10 % at M=48-64 and 10 % on realigned rows (16x8192x8191).
//  * Wider column blocks read longer row runs but give fewer workgroups;
//    they split K over `ksplit` workgroups to fill the chip. Each writes its
//    partial tile, and a second small kernel sums the partials in split order
//    and applies bias and activation. (A "last workgroup to arrive reduces"
//    variant, with the partials exchanged through agent-scope atomics, was
//    measured: it costs as much as the extra launch, so it is not used.)
//  * Each K slice starts its walk at a hashed offset (wrapping), so the rows
//    in flight at any moment are spread over the matrix and over the HBM
//    channels instead of every wave hitting the same few rows. Waves side by
//    side share the offset, so a workgroup reads WN*16*CPL*4 contiguous bytes
//    of a row at a time (a per-wave offset was ~2 % slower at M=16).
//  * W registers are reloaded one at a time right after the MFMAs that read
//    them, so a wave's loads stay in flight while it computes.
//    A wave that drained its loads before every batch of MFMAs streamed
//    ~1.5 us slower at M=16, K=N=8192 (~42.7 vs ~41.2 us for the main kernel).
// The summation order is fixed by the shape and the configuration, so
// results are deterministic.
#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace edsl {
namespace {

typedef float f32x3 __attribute__((ext_vector_type(3)));

// Waves per workgroup for MB row blocks of 16 and WN waves side by side.
constexpr int waves_per_wg(int mb, int wn) { return (mb == 1 ? 4 : 8) > wn ? (mb == 1 ? 4 : 8) : wn; }
constexpr int kMaxSplit = 16;
constexpr int kMaxTail = 16;  // rows of the K tail (GemvF32Args::k_end - K)

__device__ __forceinline__ float epilogue_rt(float acc, float b, float alpha, int epi) {
  switch (epi) {
    case epi_code(false, ACT_NONE): return apply_epilogue_f32<epi_code(false, ACT_NONE)>(acc, b, alpha);
    case epi_code(true, ACT_NONE): return apply_epilogue_f32<epi_code(true, ACT_NONE)>(acc, b, alpha);
    case epi_code(false, ACT_RELU): return apply_epilogue_f32<epi_code(false, ACT_RELU)>(acc, b, alpha);
    case epi_code(true, ACT_RELU): return apply_epilogue_f32<epi_code(true, ACT_RELU)>(acc, b, alpha);
    case epi_code(false, ACT_LEAKY): return apply_epilogue_f32<epi_code(false, ACT_LEAKY)>(acc, b, alpha);
    case epi_code(true, ACT_LEAKY): return apply_epilogue_f32<epi_code(true, ACT_LEAKY)>(acc, b, alpha);
    case epi_code(false, ACT_IF_RELU): return apply_epilogue_f32<epi_code(false, ACT_IF_RELU)>(acc, b, alpha);
    default: return apply_epilogue_f32<epi_code(true, ACT_IF_RELU)>(acc, b, alpha);
  }
}

// XV: X rows are 16-byte aligned (row stride % 4 == 0) and are read with one
// 16-byte load per row block and step; otherwise with four 4-byte loads
// (X is small and read from the caches, so this costs little against W).
// WM (GemvF32Args::w_mode): kWVector -- W, Y and the bias are 16-byte
// aligned, their row strides and N multiples of 4: a lane's CPL columns are
// one vector load or store, all in or all out of range. Otherwise Y and the
// bias are 4-byte accesses and columns past N are not stored; W is read
// either with a 4-byte load per column (kWScalar; columns past N read column
// N - 1) or, for CPL = 4, realigned (kWRealign): the lane's 4 columns lie in
// two neighbouring 16-byte chunks of the row, loaded whole (the second mostly
// by the neighbouring lane), and a select by the row's offset within its
// chunk picks them; the caller leaves the last row of W to the K tail.
template <int MB, int CPL, int WN, bool XV, int WM>
__global__ void __launch_bounds__(waves_per_wg(MB, WN) * 64)
gemv_f32_kernel(GemvF32Args a, int epi) {
  using vec = typename std::conditional<CPL == 4, f32x4, f32x2>::type;
  constexpr int NW = waves_per_wg(MB, WN);
  static_assert(NW % WN == 0, "waves side by side must divide the workgroup");
  constexpr int WK = NW / WN;
  constexpr int kWaveCols = 16 * CPL;
  constexpr int kGroupCols = kWaveCols * WN;
  // 16-row steps per loop iteration: 8 W loads in flight per lane for one row
  // block, 4 for more. Two row blocks measured faster with one step than with
  // two (M = 32: 21.4 vs 23.5 us at K = N = 4096, 56.5 vs 59.9 us at 8192), and
  // three or four need the registers for their accumulators. Four steps (16
  // loads per lane) with one row block measured no faster, also where each
  // wave's K slice is short (the c4 column shard: 11.3-11.5 against 11.0-11.2 us).
  constexpr int kU = MB == 1 ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wn = wave % WN;
  const int wk = wave / WN;
  const int groups = (a.N + kGroupCols - 1) / kGroupCols;  // the last may be partial
  const int g = blockIdx.x % groups;
  const int split = blockIdx.x / groups;
  const int n0 = g * kGroupCols + kWaveCols * wn;
  // K, in 16-row chunks, is spread as evenly as possible over the ksplit x WK
  // slices: slice i = split * WK + wk takes chunks [i*C/S, (i+1)*C/S). When S
  // divides C every slice has the same length.
  const int chunks = a.K / 16;
  const int nslices = a.ksplit * WK;
  const int slice = split * WK + wk;
  const int kbeg = 16 * (int)((int64_t)slice * chunks / nslices);
  const int kwave = 16 * (int)((int64_t)(slice + 1) * chunks / nslices) - kbeg;  // multiple of 16
  const int li = lane & 15;
  const int lg = lane >> 4;

  f32x4 acc[MB][CPL];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[mb][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int64_t ldw = a.ldw;
  // kWVector: lanes whose columns lie past N (a partial last column block)
  // read the last CPL columns instead; their results are never stored. N % 4
  // == 0, so a lane's CPL columns are all in or all out. kWScalar: wbase is
  // the row start and cofs the lane's columns, each clamped to N - 1.
  static_assert(WM != kWRealign || CPL == 4, "realigned W rows need 4 columns per lane");
  // Realigned rows: every lane's column offset and every step's row offset
  // within the wave's slice are multiples of 4, so the offset of a row within
  // its 16-byte chunk depends only on the row's slot s = q % 4 in the step:
  // dsh[s], the same for every lane and step.
  //
  // A lane loads one chunk per row, the one holding its first column. The next chunk, which holds the rest, is
  // its right neighbour's, taken with a row shift (lanes 16g .. 16g+15 share
  // a row); only lane 16g+15 has no neighbour and loads it as well (the other
  // lanes masked off; 12 bytes, the most it needs). Both are kept until just
  // before the MFMAs that read them, so a wave's loads stay in flight. Lanes
  // wholly past N read the chunk at r4 = N rounded up to 4, the one after the
  // last lane that holds a column below N, so that its neighbour finds the
  // right chunk there. Every chunk loaded holds a column below N of its row or
  // one of the next row's first elements (the caller leaves the last row of W
  // to the K tail), so no load leaves the matrix's pages.
  constexpr bool kDefer = WM == kWRealign;
  const int col_lane = n0 + CPL * li;
  const int r4 = (a.N + 3) & ~3;
  const int col_w = WM == kWVector ? min(col_lane, a.N - CPL) : kDefer ? min(col_lane, r4) : 0;
  const float* wbase = a.W + (int64_t)(kbeg + 4 * lg) * ldw + col_w;
  int cofs[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) cofs[c] = min(col_lane + c, a.N - 1);
  int dsh[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    dsh[s] = (int)(((reinterpret_cast<uintptr_t>(a.W) >> 2) + (uint64_t)s * (uint64_t)ldw) & 3);
  // Lane 16g+15 loads its second chunk when it holds a column below N.
  const bool own_next = li == 15 && col_lane < a.N;
  // Elements d .. d+3 (d = dsh[s]) of the lane's chunk c0 and the next one.
  // The row shift runs on every lane (a lane masked off would read as
  // invalid to its neighbour); the selects follow.
  auto realign = [&](const f32x4& c0, const f32x3& own, int s) {
    auto shl1 = [](float v) {  // lane i <- lane i + 1 of its row of 16
      return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x101, 0xf, 0xf, false));
    };
    const f32x3 next{shl1(c0[0]), shl1(c0[1]), shl1(c0[2])};
    const f32x3 c1 = li == 15 ? own : next;
    const bool b0 = dsh[s] & 1, b1 = dsh[s] & 2;
    const float t0 = b0 ? c0[1] : c0[0], t1 = b0 ? c0[2] : c0[1], t2 = b0 ? c0[3] : c0[2];
    const float t3 = b0 ? c1[0] : c0[3], t4 = b0 ? c1[1] : c1[0], t5 = b0 ? c1[2] : c1[1];
    return f32x4{b1 ? t2 : t0, b1 ? t3 : t1, b1 ? t4 : t2, b1 ? t5 : t3};
  };
  // The second chunk is loaded as 12 bytes, so no register of an outstanding
  // load is dead (a dead one is reused as a temporary, and the wave then
  // waits for the load before the temporary is written).
  struct Chunks { f32x4 c0; f32x3 c1; };
  using wreg = typename std::conditional<kDefer, Chunks, vec>::type;
  auto load_row = [&](const float* row, int s) {
    if constexpr (WM == kWVector) {
      return __builtin_nontemporal_load(reinterpret_cast<const vec*>(row));
    } else if constexpr (kDefer) {
      const f32x4* p0 = reinterpret_cast<const f32x4*>(row - dsh[s]);
      Chunks r;
      r.c0 = __builtin_nontemporal_load(p0);
      r.c1 = f32x3{0.0f, 0.0f, 0.0f};
      if (own_next && dsh[s] != 0) r.c1 = __builtin_nontemporal_load(reinterpret_cast<const f32x3*>(p0 + 1));
      return r;
    } else {
      vec v;
#pragma unroll
      for (int c = 0; c < CPL; ++c) v[c] = __builtin_nontemporal_load(row + cofs[c]);
      return v;
    }
  };
  // Rows of X past M read row 0 instead: MFMA output row i depends only on
  // A row i, and those output rows are never stored.
  const float* xp[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = 16 * mb + li;
    xp[mb] = a.X + (int64_t)(row < a.M ? row : 0) * a.ldx + kbeg + 4 * lg;
  }

  // One step = 16 rows of the wave's K slice: per lane 4 W loads of CPL
  // columns (register q = 4u + s holds row 16u + s of the step) and one X load
  // per row block.
  auto load_w = [&](auto& w, int k) {
    constexpr int U = sizeof(w) / sizeof(w[0]) / 4;
    const float* wp = wbase + (int64_t)k * ldw;
#pragma unroll
    for (int q = 0; q < 4 * U; ++q) w[q] = load_row(wp + (int64_t)(16 * (q / 4) + q % 4) * ldw, q % 4);
  };
  auto load_x = [&](auto& x, int k) {
    constexpr int U = sizeof(x) / sizeof(x[0]);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const float* p = xp[mb] + k + 16 * u;
        if constexpr (XV)
          x[u][mb] = *reinterpret_cast<const f32x4*>(p);
        else
          x[u][mb] = f32x4{p[0], p[1], p[2], p[3]};
      }
  };
  auto mfma_q = [&](const f32x4 (&xu)[MB], int s, const wreg& wr) {
    vec wq;
    if constexpr (kDefer)
      wq = realign(wr.c0, wr.c1, s);
    else
      wq = wr;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int c = 0; c < CPL; ++c)
        acc[mb][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(xu[mb][s], wq[c], acc[mb][c], 0, 0, 0);
  };

  // Main iterations of kU steps, walked from a hashed start. The loads are a
  // rotating pipeline: as soon as the MFMAs of W register q have been issued,
  // q is reloaded with the next iteration's row, so every wave keeps its 4*kU
  // W loads in flight while it computes instead of draining them before each
  // iteration. (The scheduling barrier keeps the compiler from sinking the
  // reloads to the end of the iteration.) For three or four row blocks this
  // also measured faster than loading, waiting and computing one iteration at
  // a time: at K = N = 8192, M = 48 80.5 vs 91.6 us and M = 64 104 vs 115 us
  // (M = 64 with 4 columns per lane uses all 128 registers and 8-16 bytes of
  // scratch); at K = N = 4096 the two measure the same.
  const int nit = kwave / (16 * kU);
  const int r0 = nit > 0 ? (int)(((unsigned)blockIdx.x * 2654435761u >> 8) + (unsigned)wk * 977u) % nit : 0;
  if (nit > 0) {
    wreg w[4 * kU];
    f32x4 x[kU][MB], xn[kU][MB];
    int it = r0;
    load_x(x, it * 16 * kU);
    load_w(w, it * 16 * kU);
    for (int i = 1; i < nit; ++i) {
      int itn = it + 1;
      if (itn >= nit) itn = 0;
      const int kn = itn * 16 * kU;
      load_x(xn, kn);
      const float* wp = wbase + (int64_t)kn * ldw;
#pragma unroll
      for (int q = 0; q < 4 * kU; ++q) {
        mfma_q(x[q / 4], q % 4, w[q]);
        w[q] = load_row(wp + (int64_t)(16 * (q / 4) + q % 4) * ldw, q % 4);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int u = 0; u < kU; ++u)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) x[u][mb] = xn[u][mb];
      it = itn;
    }
#pragma unroll
    for (int q = 0; q < 4 * kU; ++q) mfma_q(x[q / 4], q % 4, w[q]);
  }
  // Remaining single steps (kwave not a multiple of 16*kU).
  for (int k = nit * 16 * kU; k < kwave; k += 16) {
    wreg w[4];
    f32x4 x[1][MB];
    load_x(x, k);
    load_w(w, k);
#pragma unroll
    for (int q = 0; q < 4; ++q) mfma_q(x[0], q, w[q]);
  }

  // Sum the WK K-slices of each column block in wave order, one row block at
  // a time to bound LDS.
  __shared__ f32x4 red[WK > 1 ? WK - 1 : 1][WN][CPL][64];
  if constexpr (WK > 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      if (wk > 0) {
#pragma unroll
        for (int c = 0; c < CPL; ++c) red[wk - 1][wn][c][lane] = acc[mb][c];
      }
      __syncthreads();
      if (wk == 0) {
#pragma unroll
        for (int w = 0; w < WK - 1; ++w)
#pragma unroll
          for (int c = 0; c < CPL; ++c) acc[mb][c] += red[w][wn][c][lane];
      }
      __syncthreads();
    }
    if (wk != 0) return;
  }

  // Lane holds rows 16*mb + 4*lg + r and columns n0 + CPL*li + c.
  const int col = n0 + CPL * li;
  if (col >= a.N) return;
  if (a.ksplit == 1) {
    vec bv;
#pragma unroll
    for (int c = 0; c < CPL; ++c) bv[c] = 0.0f;
    if (epi_has_bias(epi)) {
      if constexpr (WM == kWVector) {
        bv = *reinterpret_cast<const vec*>(a.bias + col);
      } else {
#pragma unroll
        for (int c = 0; c < CPL; ++c) bv[c] = col + c < a.N ? a.bias[col + c] : 0.0f;
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mb + 4 * lg + r;
        if (row < a.M) {
          vec y;
#pragma unroll
          for (int c = 0; c < CPL; ++c) y[c] = epilogue_rt(acc[mb][c][r], bv[c], a.alpha, epi);
          float* dst = a.Y + (int64_t)row * a.ldy + col;
          if constexpr (WM == kWVector) {
            *reinterpret_cast<vec*>(dst) = y;
          } else {
#pragma unroll
            for (int c = 0; c < CPL; ++c)
              if (col + c < a.N) dst[c] = y[c];
          }
        }
      }
    return;
  }
  const int prow = 16 * MB;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * mb + 4 * lg + r;
      if (row < a.M) {
        vec p;
#pragma unroll
        for (int c = 0; c < CPL; ++c) p[c] = acc[mb][c][r];
        *reinterpret_cast<vec*>(a.partials + ((int64_t)split * prow + row) * a.ldp + col) = p;
      }
    }
}

// Y[m, 4j..4j+3] = epilogue(sum over splits s = 0..ksplit-1, in order, plus
// the K tail rows).
// All split loads are issued before the first add so their latencies overlap.
// WV as for gemv_f32_kernel: otherwise the bias, the tail rows of W and Y
// are 4-byte accesses, columns past N neither read nor written. The partials
// always have an aligned row pitch (ldp, a multiple of 4).
// One wave per workgroup spreads the reduction over more CUs than 256-thread
// workgroups (the c4 column shard: 16 workgroups of 256 threads); measured
// 0.2 us faster per layer at c4 and at its column shard.
template <bool WV>
__global__ void __launch_bounds__(64) gemv_reduce_kernel(GemvF32Args a, int epi, int prow) {
  const int64_t idx = (int64_t)blockIdx.x * 64 + threadIdx.x;  // over M * ceil(N/4)
  const int n4 = (a.N + 3) / 4;
  if (idx >= (int64_t)a.M * n4) return;
  const int row = (int)(idx / n4);
  const int col = 4 * (int)(idx % n4);
  f32x4 v[kMaxSplit];
#pragma unroll
  for (int sp = 0; sp < kMaxSplit; ++sp)
    if (sp < a.ksplit)
      v[sp] = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4*>(a.partials + ((int64_t)sp * prow + row) * a.ldp + col));
  f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
  if (epi_has_bias(epi)) {
    if constexpr (WV) {
      bv = *reinterpret_cast<const f32x4*>(a.bias + col);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) bv[c] = col + c < a.N ? a.bias[col + c] : 0.0f;
    }
  }
  f32x4 s = v[0];
#pragma unroll
  for (int sp = 1; sp < kMaxSplit; ++sp)
    if (sp < a.ksplit) s += v[sp];
  // The K tail (at most 16 rows), after the split sums, in ascending k. All
  // its loads are issued before the first add (rows past k_end read row
  // k_end - 1 and are not added), so their latencies overlap.
  if (a.k_end > a.K) {
    float xt[kMaxTail];
    f32x4 wt[kMaxTail];
#pragma unroll
    for (int t = 0; t < kMaxTail; ++t) {
      const int k = min(a.K + t, a.k_end - 1);
      xt[t] = a.x_tail[(int64_t)row * a.ldx_tail + k];
      const float* wr = a.W + (int64_t)k * a.ldw + col;
      if constexpr (WV) {
        wt[t] = *reinterpret_cast<const f32x4*>(wr);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) wt[t][c] = col + c < a.N ? wr[c] : 0.0f;
      }
    }
#pragma unroll
    for (int t = 0; t < kMaxTail; ++t)
      if (a.K + t < a.k_end) s += xt[t] * wt[t];
  }
  f32x4 y;
#pragma unroll
  for (int c = 0; c < 4; ++c) y[c] = epilogue_rt(s[c], bv[c], a.alpha, epi);
  float* dst = a.Y + (int64_t)row * a.ldy + col;
  if constexpr (WV) {
    *reinterpret_cast<f32x4*>(dst) = y;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (col + c < a.N) dst[c] = y[c];
  }
}

template <int MB, bool XV, int WM>
hipError_t launch_mb_x(int cols, int epi, const GemvF32Args& a, hipStream_t stream) {
  const dim3 grid(((a.N + cols - 1) / cols) * a.ksplit);
  auto block = [](int wn) { return dim3(waves_per_wg(MB, wn) * 64); };
  // Two columns per lane take 4-byte W loads where four would be realigned.
  constexpr int WM2 = WM == kWRealign ? kWScalar : WM;
  switch (cols) {
    case 32: hipLaunchKernelGGL((gemv_f32_kernel<MB, 2, 1, XV, WM2>), grid, block(1), 0, stream, a, epi); break;
    case 64: hipLaunchKernelGGL((gemv_f32_kernel<MB, 4, 1, XV, WM>), grid, block(1), 0, stream, a, epi); break;
    case 128: hipLaunchKernelGGL((gemv_f32_kernel<MB, 4, 2, XV, WM>), grid, block(2), 0, stream, a, epi); break;
    case 256: hipLaunchKernelGGL((gemv_f32_kernel<MB, 4, 4, XV, WM>), grid, block(4), 0, stream, a, epi); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}


template <int MB, int WM>
hipError_t launch_mb_w(int cols, int epi, const GemvF32Args& a, hipStream_t stream) {
  const bool xv = reinterpret_cast<uintptr_t>(a.X) % 16 == 0 && a.ldx % 4 == 0;
  return xv ? launch_mb_x<MB, true, WM>(cols, epi, a, stream) : launch_mb_x<MB, false, WM>(cols, epi, a, stream);
}

template <int MB>
hipError_t launch_mb(int cols, int epi, const GemvF32Args& a, hipStream_t stream) {
  switch (a.w_mode) {
    case kWVector: return launch_mb_w<MB, kWVector>(cols, epi, a, stream);
    case kWScalar: return launch_mb_w<MB, kWScalar>(cols, epi, a, stream);
    case kWRealign: return launch_mb_w<MB, kWRealign>(cols, epi, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

int gemv_f32_waves_k(int cols, int M) {
  const int wn = cols <= 64 ? 1 : cols / 64;
  return waves_per_wg((M + 15) / 16, wn) / wn;
}

int gemv_f32_w_mode(const GemvF32Args& a) {
  if (gemv_f32_vector_rows(a)) return kWVector;
  return a.N >= 4 ? kWRealign : kWScalar;
}

bool gemv_f32_vector_rows(const GemvF32Args& a) {
  auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  return al16(a.W) && al16(a.Y) && (a.bias == nullptr || al16(a.bias)) && a.ldw % 4 == 0 && a.ldy % 4 == 0 &&
         a.N % 4 == 0;
}
int gemv_f32_max_ksplit() { return kMaxSplit; }

hipError_t launch_gemv_f32(int epi, int cols, GemvF32Args a, hipStream_t stream) {
  const int mb = (a.M + 15) / 16;
  if (a.k_end < a.K || a.k_end - a.K > kMaxTail || (a.k_end > a.K && a.ksplit < 2)) return hipErrorInvalidValue;
  hipError_t e;
  switch (mb) {
    case 1: e = launch_mb<1>(cols, epi, a, stream); break;
    case 2: e = launch_mb<2>(cols, epi, a, stream); break;
    case 3: e = launch_mb<3>(cols, epi, a, stream); break;
    case 4: e = launch_mb<4>(cols, epi, a, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess || a.ksplit == 1) return e;
  const int64_t items = (int64_t)a.M * ((a.N + 3) / 4);
  const dim3 g((unsigned)((items + 63) / 64));
  if (a.w_mode == kWVector)
    hipLaunchKernelGGL(gemv_reduce_kernel<true>, g, dim3(64), 0, stream, a, epi, 16 * mb);
  else
    hipLaunchKernelGGL(gemv_reduce_kernel<false>, g, dim3(64), 0, stream, a, epi, 16 * mb);
  return hipGetLastError();
}

}  // namespace edsl
