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
// order. A pre-pass narrows X and W to int8 and writes them fragment-packed
// (each 32x32 block stored as the 64 lanes x 16 bytes the MFMA consumes, W
// transposed on the way), and flags any out-of-range value. The packed copies
// are padded with zeros to multiples of the 128-wide tile in M, N and K, so
// any shape runs on the matrix cores; the GEMM stores only the real M x N.
// The pre-pass writes one range flag per 64x64 tile of X and of W on every
// call (1: some value outside int8, else 0). Each GEMM workgroup reads the
// flags of the X row panels and W column panels its tile uses; if any is set,
// that tile alone takes the exact wrapping-i32 vector-ALU path on the
// original i32 tensors instead. Every flag is rewritten by every call, so a
// replayed graph never sees a previous call's state.
#include "common.hpp"
#include "kernels.hpp"

#include <type_traits>

namespace edsl {
namespace {

// ------------------------------------------------------------------ pre-pass
// Only used on the int8 path. The i32 sources may have any alignment / row
// stride: `vec_ok` selects 16-byte source loads.
constexpr int kNarrowTile = 64;

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

// Byte offset of element (r, k) inside a 64x64 tile held as its four packed
// fragments (2 row blocks x 2 k steps, 1 KB each, in [rb][kt] order).
__device__ __forceinline__ int tile_packed_offset(int r, int k) {
  return ((((r >> 5) * 2 + (k >> 5)) * 64 + (r & 31) + 32 * ((k >> 4) & 1)) << 4) + (k & 15);
}

// Grid: 64x64 tiles of the padded X (Mp x Kp), then of the padded W (Kp x Np).
// Thread t owns a 4x4 block of the tile (4 row loads of 16 bytes), narrows it,
// and writes it into LDS in packed order: for X each 16-byte row piece is
// already 4 consecutive k of one row (one packed word); for W the 4x4 block is
// transposed in registers so each word holds 4 consecutive k of one column.
// The packed tile then leaves with one 16-byte store per thread (four 1 KB
// fragments). Tiles that reach past the real M, N or K load element by element
// and write zeros there.
__global__ void __launch_bounds__(256) narrow_i8_kernel(NarrowI8Args a, int vec_ok_x, int vec_ok_w) {
  __shared__ uint32_t pk[kNarrowTile * kNarrowTile / 4];
  const int tid = threadIdx.x;
  const int bi = tid >> 4;        // 4-row block along the source's rows
  const int bj = 4 * (tid & 15);  // 4-column block along the source's columns
  const int x_tiles_k = a.Kp / kNarrowTile;
  const int x_tiles = (a.Mp / kNarrowTile) * x_tiles_k;
  bool bad = false;
  int r0, k0;  // tile origin in the packed matrix's (row, k) coordinates
  int8_t* dst;
  // 4 consecutive elements of row `row` from column `col` of a source with
  // `rows` x `cols` elements; zeros past either edge.
  auto load_edge = [](const int32_t* src, int64_t ld, int rows, int cols, int row, int col) {
    i32x4 v = {0, 0, 0, 0};
    if (row < rows) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col + e < cols) v[e] = src[(int64_t)row * ld + col + e];
    }
    return v;
  };
  if ((int)blockIdx.x < x_tiles) {
    r0 = (blockIdx.x / x_tiles_k) * kNarrowTile;
    k0 = (blockIdx.x % x_tiles_k) * kNarrowTile;
    dst = a.X8p;
    i32x4 v[4];
    if (r0 + kNarrowTile <= a.M && k0 + kNarrowTile <= a.K) {  // uniform per workgroup
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = load4(a.X + (int64_t)(r0 + 4 * bi + i) * a.ldx + k0 + bj, vec_ok_x);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = load_edge(a.X, a.ldx, a.M, a.K, r0 + 4 * bi + i, k0 + bj);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) pk[tile_packed_offset(4 * bi + i, bj) >> 2] = pack_i8x4(v[i], bad);
  } else {
    const int b = blockIdx.x - x_tiles;
    const int w_tiles_n = a.Np / kNarrowTile;
    k0 = (b / w_tiles_n) * kNarrowTile;
    r0 = (b % w_tiles_n) * kNarrowTile;  // packed rows are W's columns
    dst = a.W8p;
    i32x4 v[4];
    if (k0 + kNarrowTile <= a.K && r0 + kNarrowTile <= a.N) {  // uniform per workgroup
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = load4(a.W + (int64_t)(k0 + 4 * bi + i) * a.ldw + r0 + bj, vec_ok_w);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = load_edge(a.W, a.ldw, a.K, a.N, k0 + 4 * bi + i, r0 + bj);
    }
    uint32_t q[4];  // q[i] = W row k0 + 4bi + i, columns r0 + bj .. + 3 (byte e = column e)
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = pack_i8x4(v[i], bad);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // column r0 + bj + e, rows k0 + 4bi .. + 3 as one word (byte i = row i)
      uint32_t w = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) w |= ((q[i] >> (8 * e)) & 0xffu) << (8 * i);
      pk[tile_packed_offset(bj + e, 4 * bi) >> 2] = w;
    }
  }
  const int tile_bad = __syncthreads_or(bad ? 1 : 0);
  const int frag = tid >> 6, lane = tid & 63;
  const int rb = (r0 >> 5) + (frag >> 1), kt = (k0 >> 5) + (frag & 1);
  const i32x4 out = reinterpret_cast<const i32x4*>(pk)[tid];
  *reinterpret_cast<i32x4*>(dst + ((((int64_t)rb * (a.Kp >> 5) + kt) * 64 + lane) << 4)) = out;
  if (tid == 0) {
    // Written on every call: X flags [Mp/64][Kp/64], W flags [Np/64][Kp/64].
    uint8_t* f = dst == a.X8p ? a.flags_x : a.flags_w;
    f[(int64_t)(r0 / kNarrowTile) * (a.Kp / kNarrowTile) + k0 / kNarrowTile] = tile_bad ? 1 : 0;
  }
}

// Whether the tile at (m0, n0) must take the exact i32 path: any range flag
// of its two 64-row X panels or its two 64-column W panels is set. Uniform
// over the workgroup (NT threads). Flag rows of one panel are Kp/64 bytes,
// an even count, and the two panels of a 128-wide tile are adjacent, so the
// 2*Kp/64 flags are read as 4-byte words.
template <int NT>
__device__ __forceinline__ bool tile_out_of_range(const GemmI32Args& a, int m0, int n0) {
  const int kt = a.Kp / kNarrowTile;
  const uint32_t* fx = reinterpret_cast<const uint32_t*>(a.flags_x + (int64_t)(m0 / kNarrowTile) * kt);
  const uint32_t* fw = reinterpret_cast<const uint32_t*>(a.flags_w + (int64_t)(n0 / kNarrowTile) * kt);
  int bad = 0;
  for (int i = threadIdx.x; i < kt / 2; i += NT) bad |= (fx[i] | fw[i]) != 0;
  return __syncthreads_or(bad) != 0;
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
// 128x128 output tile per workgroup of 4 waves, each wave a 64x64 quadrant
// (2x2 blocks of 32x32). Operands come straight from the fragment-packed
// copies: each fragment is one fully coalesced 16-byte load per lane in the
// exact MFMA operand layout, so nothing is staged through LDS and no lane
// shuffles are needed. Fragments of step s + D are loaded while the MFMAs of
// step s run (D steps in flight; past the last step the last step is loaded
// again, which keeps the loop free of branches so the wait counts stay exact).
// v_mfma_i32_32x32x32_i8: lane l supplies 16 int8 of A row l%32 and of B^T row
// (= output column) l%32 from k-chunk l/32 of the step, so A and B always
// pair the same k.
template <int EPI, int D>
__global__ void __launch_bounds__(256) gemm_i8_kernel(GemmI32Args a) {
  __shared__ ValuSmem valu;
  int tm, tn;
  tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int m0 = tm * kI8Tile, n0 = tn * kI8Tile;

  if (tile_out_of_range<256>(a, m0, n0)) {  // some value outside int8: exact i32 path
    valu_tile_i32<EPI, 256>(a, m0, n0, valu);
    return;
  }

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int KT = a.Kp >> 5;  // 32-k steps of the padded K; a multiple of D
  const i32x4* ap[2];
  const i32x4* bp[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    ap[i] = reinterpret_cast<const i32x4*>(a.A8p) + (int64_t)((m0 >> 5) + 2 * wm + i) * KT * 64 + lane;
    bp[i] = reinterpret_cast<const i32x4*>(a.B8p) + (int64_t)((n0 >> 5) + 2 * wn + i) * KT * 64 + lane;
  }

  i32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // Prologue loads in the loop's order (slot by slot): the wait counts at the
  // loop head are exact only if the two orders agree.
  i32x4 fa[D][2], fb[D][2];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int s = min(d, KT - 1);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      fa[d][i] = ap[i][(int64_t)s * 64];
      fb[d][i] = bp[i][(int64_t)s * 64];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll 1
  for (int s0 = 0; s0 < KT; s0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[d][i], fb[d][j], acc[i][j], 0, 0, 0);
      // Keep the refill of this slot after its MFMAs and before the next
      // slot's, so each slot's loads stay D steps ahead of their use.
      __builtin_amdgcn_sched_barrier(0);
      const int sn = min(s0 + d + D, KT - 1);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        fa[d][i] = ap[i][(int64_t)sn * 64];
        fb[d][i] = bp[i][(int64_t)sn * 64];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Epilogue: lane holds rows 8*(r/4) + 4*half + r%4 and column l32 of each
  // block; each store instruction writes two full 128-byte row segments.
  // Non-temporal: the result is not re-read by this kernel.
  // Rows and columns past the real M and N (padding) are not stored; tiles
  // that lie inside take the unchecked copy of the loop.
  const int half = lane >> 5, l32 = lane & 31;
  auto store_tile = [&](auto checked) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 64 * wn + 32 * j + l32;
      const int32_t b = epi_has_bias(EPI) && (!checked || n < a.N) ? a.bias[n] : 0;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * half + (r & 3);
          if (!checked || (m < a.M && n < a.N))
            __builtin_nontemporal_store(apply_epilogue_i32<EPI>(acc[i][j][r], b), a.C + (int64_t)m * a.ldc + n);
        }
    }
  };
  if (m0 + kI8Tile <= a.M && n0 + kI8Tile <= a.N)
    store_tile(std::false_type{});
  else
    store_tile(std::true_type{});
}

// K-split waves: every wave computes the whole 128x128 tile (4x4 blocks of
// 32x32, 256 accumulator registers) over every fourth 32-k step (wave w takes
// steps w, w + 4, ...). Each A and B fragment is then fetched by exactly one
// wave -- half the vector-cache requests of the quadrant layout above, where
// every fragment is fetched by the two waves sharing its row or column block
// -- and each wave runs 16 MFMAs per 8 fragment loads instead of 4 per 4.
// Afterwards the four partial tiles are summed through LDS in two rounds of
// two row blocks; integer addition wraps associatively, so the order of the
// sum does not change the result. One workgroup per CU (all 512 registers per
// lane are available to its waves).
constexpr int kI8KsRedBytes = 4 * 2 * 4 * 16 * 64 * 4;  // [wave][ii][j][reg][lane] i32, 128 KB

template <int EPI, int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_i8_ksplit_kernel(GemmI32Args a) {
  __shared__ i32x4 red[kI8KsRedBytes / 16];
  static_assert(sizeof(ValuSmem) <= sizeof(red), "exact-path staging must fit the reduce buffer");
  int tm, tn;
  tile_coords(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int m0 = tm * kI8Tile, n0 = tn * kI8Tile;

  if (tile_out_of_range<256>(a, m0, n0)) {  // some value outside int8: exact i32 path
    valu_tile_i32<EPI, 256>(a, m0, n0, *reinterpret_cast<ValuSmem*>(red));
    return;
  }

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int KT = a.Kp >> 5;  // 32-k steps of the padded K, a multiple of 4
  const int NS = KT >> 2;   // steps per wave, a multiple of D
  // The tile's four 32-row blocks of packed X and four 32-column blocks of
  // packed W, read through buffer descriptors: the lane's 16 bytes at a
  // per-lane offset, the block and step at a scalar one (no 64-bit address
  // arithmetic in the loop).
  const int block_bytes = KT * 64 * 16;  // one 32-row (or 32-column) block: KT fragments
  const i32x4 rsrc_a = buffer_rsrc(a.A8p + (int64_t)(m0 >> 5) * block_bytes, 4 * (int64_t)block_bytes);
  const i32x4 rsrc_b = buffer_rsrc(a.B8p + (int64_t)(n0 >> 5) * block_bytes, 4 * (int64_t)block_bytes);
  const int vlane = lane * 16;

  i32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  // Loads of this wave's t-th step; past the last one the last is loaded again
  // (never used), which keeps the loop free of branches. (A loop that stops
  // loading D steps early and finishes with a tail of MFMAs issues 1/9 fewer
  // L2 requests at K = 2048 but measured 2% slower: the compiler moves the
  // accumulators between registers before the tail.)
  i32x4 fa[D][4], fb[D][4];
  auto load = [&](i32x4(&xa)[4], i32x4(&xb)[4], int t) {
    const int s = (min(t, NS - 1) * 4 + wave) * 64 * 16;  // the step's fragment, in bytes
#pragma unroll
    for (int i = 0; i < 4; ++i) xa[i] = raw_buffer_load_i32x4(rsrc_a, vlane, i * block_bytes + s, 0);
#pragma unroll
    for (int j = 0; j < 4; ++j) xb[j] = raw_buffer_load_i32x4(rsrc_b, vlane, j * block_bytes + s, 0);
  };
#pragma unroll
  for (int d = 0; d < D; ++d) {
    load(fa[d], fb[d], d);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll 1
  for (int t0 = 0; t0 < NS; t0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[d][i], fb[d][j], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      load(fa[d], fb[d], t0 + d + D);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Round h: every wave writes its partial blocks (2h + ii, j) for ii < 2,
  // j < 4; then wave w sums row block 2h + w/2, column blocks 2(w%2) + jj over
  // the four waves and stores them with the epilogue. A lane holds rows
  // 8*(r/4) + 4*half + r%4 and column l32 of each block, so each store
  // instruction writes two full 128-byte row segments.
  const int half = lane >> 5, l32 = lane & 31;
  auto slot = [&](int p, int ii, int j, int q) { return (((p * 2 + ii) * 4 + j) * 4 + q) * 64 + lane; };
  // Rows and columns past the real M and N (padding) are not stored; tiles
  // that lie inside take the unchecked copy of the epilogue.
  auto epilogue = [&](auto checked) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (h == 1) __syncthreads();  // round 0's reads are done before round 1 overwrites
#pragma unroll
      for (int ii = 0; ii < 2; ++ii)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const i32x16& v = acc[2 * h + ii][j];
            red[slot(wave, ii, j, q)] = i32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
          }
      __syncthreads();
      const int ii = wave >> 1;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * (wave & 1) + jj;
        const int n = n0 + 32 * j + l32;
        const int32_t b = epi_has_bias(EPI) && (!checked || n < a.N) ? a.bias[n] : 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          i32x4 sum = red[slot(0, ii, j, q)];
#pragma unroll
          for (int p = 1; p < 4; ++p) sum += red[slot(p, ii, j, q)];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = m0 + 32 * (2 * h + ii) + 8 * q + 4 * half + e;
            if (!checked || (m < a.M && n < a.N))
              __builtin_nontemporal_store(apply_epilogue_i32<EPI>(sum[e], b), a.C + (int64_t)m * a.ldc + n);
          }
        }
      }
    }
  };
  if (m0 + kI8Tile <= a.M && n0 + kI8Tile <= a.N)
    epilogue(std::false_type{});
  else
    epilogue(std::true_type{});
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

template <bool KSPLIT, int D>
hipError_t launch_i8_depth(int epi, const GemmI32Args& a, hipStream_t stream) {
  const dim3 grid(a.tiles_m * a.tiles_n), block(256);
#define EDSL_I8_CASE(E)                                                                      \
  case E:                                                                                    \
    if constexpr (KSPLIT)                                                                    \
      hipLaunchKernelGGL((gemm_i8_ksplit_kernel<E, D>), grid, block, 0, stream, a);          \
    else                                                                                     \
      hipLaunchKernelGGL((gemm_i8_kernel<E, D>), grid, block, 0, stream, a);                 \
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

// Variant table: wave layout and prefetch depth (32-k steps in flight per
// wave). The quadrant layout needs K/32 % depth == 0, the K-split one
// K/128 % depth == 0; a depth that does not divide falls to the next entry of
// its fallback list.
struct I8Variant {
  bool ksplit;
  int depth[3];  // preferred first; the last is always 1 or a divisor of 4
};
constexpr I8Variant kI8Table[kI8Variants] = {
    {false, {4, 4, 4}}, {false, {2, 2, 2}}, {false, {8, 4, 4}}, {true, {2, 1, 1}},
};

}  // namespace

hipError_t launch_narrow_i8(NarrowI8Args a, hipStream_t stream) {
  if (a.Mp % kI8Tile || a.Np % kI8Tile || a.Kp % kI8Tile || a.M > a.Mp || a.N > a.Np || a.K > a.Kp)
    return hipErrorInvalidValue;
  const int x_tiles = (a.Mp / kNarrowTile) * (a.Kp / kNarrowTile);
  const int w_tiles = (a.Kp / kNarrowTile) * (a.Np / kNarrowTile);
  const int vec_x = ((reinterpret_cast<uintptr_t>(a.X) & 15) == 0) && (a.ldx % 4 == 0);
  const int vec_w = ((reinterpret_cast<uintptr_t>(a.W) & 15) == 0) && (a.ldw % 4 == 0);
  hipLaunchKernelGGL(narrow_i8_kernel, dim3(x_tiles + w_tiles), dim3(256), 0, stream, a, vec_x, vec_w);
  return hipGetLastError();
}

int gemm_i8_depth(int variant, int K) {
  if (variant < 0 || variant >= kI8Variants) variant = kI8DefaultVariant;
  const I8Variant& v = kI8Table[variant];
  const int steps = v.ksplit ? K / 128 : K / 32;  // K: the padded K, a multiple of 128
  for (int d : v.depth)
    if (steps % d == 0) return d;
  return 1;
}

const char* gemm_i8_layout(int variant) {
  if (variant < 0 || variant >= kI8Variants) variant = kI8DefaultVariant;
  return kI8Table[variant].ksplit ? "ksplit" : "quadrant";
}

hipError_t launch_gemm_i8(int epi, GemmI32Args a, hipStream_t stream, int variant) {
  if (a.M <= 0 || a.N <= 0 || a.K <= 0 || a.Kp % kI8Tile || a.Kp < a.K) return hipErrorInvalidValue;
  a.tiles_m = (a.M + kI8Tile - 1) / kI8Tile;
  a.tiles_n = (a.N + kI8Tile - 1) / kI8Tile;
  if (variant < 0 || variant >= kI8Variants) variant = kI8DefaultVariant;
  const int d = gemm_i8_depth(variant, a.Kp);
  if (kI8Table[variant].ksplit) {
    switch (d) {
      case 1: return launch_i8_depth<true, 1>(epi, a, stream);
      case 2: return launch_i8_depth<true, 2>(epi, a, stream);
      default: return hipErrorInvalidValue;
    }
  }
  switch (d) {
    case 2: return launch_i8_depth<false, 2>(epi, a, stream);
    case 4: return launch_i8_depth<false, 4>(epi, a, stream);
    case 8: return launch_i8_depth<false, 8>(epi, a, stream);
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
