// fp32 dense layer for small M (M <= 64): a weight-streaming kernel.
//
// Y[M,N] = epilogue(X[M,K] x W[K,N] (+ bias[N])) -- the same op as the tiled
// kernel (reference cpp/src/builders/LinalgBuilder.cpp:106-139, 180-239,
// 301-339), shaped for the HBM-bound case where W dominates the traffic
// (M=16, K=N=8192: W is 256 MiB, X and Y 512 KiB each).
//
// Every W element is read from HBM exactly once, with 16-byte coalesced loads,
// and used for all M rows at once on the matrix cores:
//  * v_mfma_f32_16x16x4_f32: lane l supplies X[row l%16][k-slot l/16] and
//    W[k-slot l/16][col l%16]. Lane group g = l/16 owns the k rows
//    k0+4g .. k0+4g+3 of each 16-row step: it loads those 4 k of its X row with
//    one 16-byte load and, for each k, 4 consecutive W columns with one 16-byte
//    load. MFMA (step s, column phase c) then pairs X[.][k0+4g+s] with
//    W[k0+4g+s][n0 + 4*(l%16) + c], so lane l%16 accumulates columns
//    n0 + 4*(l%16) + c: a wave covers 64 columns and stores float4 per row.
//  * A workgroup is 4 waves on one 64-column group; the waves split the
//    workgroup's K range and are summed in LDS in a fixed order.
//  * K is additionally split over `ksplit` workgroups so that the grid fills
//    the chip. Each writes its partial tile; the last one to arrive (device
//    atomic counter) sums the partials in split order, applies bias and
//    activation, stores Y, and re-arms the counter. The result is therefore
//    independent of which workgroup finishes last.
#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace edsl {
namespace {

constexpr int kWaves = 4;
constexpr int kCols = 64;  // columns per workgroup

template <int MB, int EPI>
__global__ void __launch_bounds__(kWaves * 64)
gemv_f32_kernel(GemvF32Args a) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int groups = a.N / kCols;
  const int g = blockIdx.x % groups;
  const int split = blockIdx.x / groups;
  const int n0 = g * kCols;
  const int kspan = a.K / a.ksplit;
  const int kwave = kspan / kWaves;  // multiple of 16
  const int kbeg = split * kspan + wave * kwave;
  const int li = lane & 15;
  const int lg = lane >> 4;

  f32x4 acc[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[mb][c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const float* wp = a.W + (int64_t)(kbeg + 4 * lg) * a.ldw + n0 + 4 * li;
  const float* xp[MB];
  bool xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int row = 16 * mb + li;
    xrow[mb] = row < a.M;
    xp[mb] = a.X + (int64_t)(xrow[mb] ? row : 0) * a.ldx + kbeg + 4 * lg;
  }
  const int64_t ldw = a.ldw;

  // U steps of 16 rows per iteration: all U*4 W loads are issued before the
  // first MFMA that needs them, keeping U KiB per wave in flight.
  auto steps = [&](auto u_tag, int k) {
    constexpr int U = decltype(u_tag)::value;
    f32x4 w[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        w[u][s] = __builtin_nontemporal_load(
            reinterpret_cast<const f32x4*>(wp + (int64_t)(16 * u + s) * ldw));
    f32x4 x[U][MB];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        x[u][mb] = *reinterpret_cast<const f32x4*>(xp[mb] + k + 16 * u);
        if (!xrow[mb]) x[u][mb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int c = 0; c < 4; ++c)
            acc[mb][c] =
                __builtin_amdgcn_mfma_f32_16x16x4f32(x[u][mb][s], w[u][s][c], acc[mb][c], 0, 0, 0);
    wp += (int64_t)16 * U * ldw;
  };

  int k = 0;
  for (; k + 64 <= kwave; k += 64) steps(std::integral_constant<int, 4>{}, k);
  for (; k < kwave; k += 16) steps(std::integral_constant<int, 1>{}, k);

  // Sum the 4 waves' K slices in wave order.
  __shared__ f32x4 red[kWaves - 1][MB * 4][64];
  if (wave > 0) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int c = 0; c < 4; ++c) red[wave - 1][mb * 4 + c][lane] = acc[mb][c];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kWaves - 1; ++w)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[mb][c] += red[w][mb * 4 + c][lane];

  // Lane holds rows 16*mb + 4*lg + r and columns n0 + 4*li + c.
  const int col = n0 + 4 * li;
  f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (epi_has_bias(EPI)) bv = *reinterpret_cast<const f32x4*>(a.bias + col);

  if (a.ksplit == 1) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mb + 4 * lg + r;
        if (row < a.M) {
          f32x4 y;
#pragma unroll
          for (int c = 0; c < 4; ++c) y[c] = apply_epilogue_f32<EPI>(acc[mb][c][r], bv[c], a.alpha);
          *reinterpret_cast<f32x4*>(a.Y + (int64_t)row * a.ldy + col) = y;
        }
      }
    return;
  }

  // Split-K: publish this slice, then let the last arriving workgroup reduce.
  const int prow = 16 * MB;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * mb + 4 * lg + r;
      f32x4 p = {acc[mb][0][r], acc[mb][1][r], acc[mb][2][r], acc[mb][3][r]};
      *reinterpret_cast<f32x4*>(a.partials + ((int64_t)split * prow + row) * a.N + col) = p;
    }
  __threadfence();
  unsigned prev = 0;
  if (lane == 0) prev = atomicAdd(&a.counters[g], 1u);
  prev = __shfl(prev, 0);
  if (prev != (unsigned)(a.ksplit - 1)) return;
  __threadfence();

#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * mb + 4 * lg + r;
      f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int sp = 0; sp < a.ksplit; ++sp)
        s += __builtin_nontemporal_load(
            reinterpret_cast<const f32x4*>(a.partials + ((int64_t)sp * prow + row) * a.N + col));
      if (row < a.M) {
        f32x4 y;
#pragma unroll
        for (int c = 0; c < 4; ++c) y[c] = apply_epilogue_f32<EPI>(s[c], bv[c], a.alpha);
        *reinterpret_cast<f32x4*>(a.Y + (int64_t)row * a.ldy + col) = y;
      }
    }
  if (lane == 0) atomicExch(&a.counters[g], 0u);
}

template <int MB>
hipError_t launch_mb(int epi, const GemvF32Args& a, hipStream_t stream) {
  const dim3 grid((a.N / kCols) * a.ksplit);
  const dim3 block(kWaves * 64);
#define EDSL_GEMV_CASE(E)                                                                \
  case E:                                                                                \
    hipLaunchKernelGGL((gemv_f32_kernel<MB, E>), grid, block, 0, stream, a);            \
    break;
  switch (epi) {
    EDSL_GEMV_CASE(epi_code(false, ACT_NONE))
    EDSL_GEMV_CASE(epi_code(true, ACT_NONE))
    EDSL_GEMV_CASE(epi_code(false, ACT_RELU))
    EDSL_GEMV_CASE(epi_code(true, ACT_RELU))
    EDSL_GEMV_CASE(epi_code(false, ACT_LEAKY))
    EDSL_GEMV_CASE(epi_code(true, ACT_LEAKY))
    default:
      return hipErrorInvalidValue;
  }
#undef EDSL_GEMV_CASE
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_f32(int epi, GemvF32Args a, hipStream_t stream) {
  const int mb = (a.M + 15) / 16;
  switch (mb) {
    case 1: return launch_mb<1>(epi, a, stream);
    case 2: return launch_mb<2>(epi, a, stream);
    case 3: return launch_mb<3>(epi, a, stream);
    case 4: return launch_mb<4>(epi, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace edsl
