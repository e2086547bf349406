// Host-visible launch interface of the gfx950 dense-path kernels.
// All pointers are device pointers; leading dimensions are in elements.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "plan_f32.hpp"

namespace edsl {

// ---------------------------------------------------------------- fp32 tiled
struct GemmF32Args {
  const float* A;     // [M][K], row stride lda
  const float* B;     // [K][N], row stride ldb
  const float* bias;  // [N] or nullptr
  float* C;           // [M][N], row stride ldc
  int64_t lda, ldb, ldc;
  int M, N, K;
  int tiles_m, tiles_n;
  float alpha;        // leaky-ReLU slope
};

hipError_t launch_gemm_f32(int cfg, int epi, GemmF32Args args, hipStream_t stream);
// The tiles on 16x16 MFMA blocks (gemm_f32_m16.hip), 16-byte aligned operands
// and row strides: layout 0, a 128x128 tile with 32-deep K steps; 1, a 64x64
// tile with 64-deep K steps; 2, a 128x256 tile with 32-deep K steps; 3, the
// 128x128 tile with eight waves. guard
// kGuardNone: M and N multiples of the tile, K of the step; kGuardEdge: any
// M, N >= 4 and K >= 4 that are multiples of 4; kGuardScalar (layout 0 only):
// any shape, alignment and row strides. tiles_m and tiles_n are M and N over
// the tile, rounded up.
hipError_t launch_gemm_f32_m16(int layout, int guard, int epi, GemmF32Args args, hipStream_t stream);
// The one-wave 128x128 tile without LDS (gemm_f32_direct.hip), 16-byte aligned
// operands and row strides, N and K multiples of 4, A and B within 32-bit
// buffer offsets (gemm_f32_direct_offsets_fit). guard kGuardNone: M and N
// multiples of 128, K of 16; kGuardEdge: any such M, N, K.
hipError_t launch_gemm_f32_direct(int guard, int epi, GemmF32Args args, hipStream_t stream);
// Its 64x64 tile with K split over `ksplit` waves (1 or 4) of one
// workgroup, partial tiles summed through LDS, the same operand conditions.
// guard kGuardNone: M and N multiples of 64, K of 16 * ksplit; kGuardEdge
// (ksplit 4): any such M, N, K.
hipError_t launch_gemm_f32_direct64(int ksplit, int guard, int epi, GemmF32Args args, hipStream_t stream);
// The 16x16 tile for small layers: K split over four waves, every fragment
// loaded up front; M and N multiples of 16, K a multiple of 64 up to 512.
hipError_t launch_gemm_f32_direct16(int epi, GemmF32Args args, hipStream_t stream);
// The (16r x 16c) tile, r x c MFMA blocks per wave, K split over four waves,
// the same operand conditions. guard kGuardNone (r x c one of 2x2, 3x3, 4x4,
// 5x5, 6x6, 3x6, 6x3): M a multiple of 16r, N of 16c, K of 16 and at least
// 64; kGuardEdge (2x2 to 6x6): any such M, N, K.
hipError_t launch_gemm_f32_direct_rc(int r, int c, int guard, int epi, GemmF32Args args, hipStream_t stream);

// ------------------------------------------------------------ fp32 small-M
struct GemvF32Args {
  const float* X;     // [M][K], row stride ldx
  const float* W;     // [K][N], row stride ldw
  const float* bias;  // [N] or nullptr
  float* Y;           // [M][N], row stride ldy
  int64_t ldx, ldw, ldy;
  int M, N, K;
  int ksplit;         // K slices reduced by a second kernel (1 = none)
  float alpha;
  float* partials;    // [ksplit][16*ceil(M/16)][ldp] when ksplit > 1
  int64_t ldp;        // partials row pitch: N rounded up to a multiple of 4
  // K tail: rows K .. k_end-1 of W (k_end - K <= 16), with X read from x_tail
  // (row stride ldx_tail), are added by the reduce kernel; k_end == K: none.
  const float* x_tail;
  int64_t ldx_tail;
  int k_end;
  int w_mode;         // kWVector, kWScalar or kWRealign (gemv_f32_w_mode)
};

// How the small-M kernel reads W: one vector per lane and row (W, Y and the
// bias 16-byte aligned, row strides and N multiples of 4), a 4-byte load per
// column, or two aligned 16-byte chunks realigned in registers (N >= 4; the
// caller must leave the last row of W to the K tail).
enum : int { kWVector = 0, kWScalar = 1, kWRealign = 2 };

// A workgroup is 4 waves (one row block) or 8 over `cols` adjacent columns
// (32, 64, 128 or 256), the last block possibly partial; the waves not side
// by side split K, which is walked in 16-row chunks. Requirements (checked by the caller):
// 1 <= M <= 64, K % 16 == 0, ksplit > 1 when there is a K tail, w_mode set
// (kWRealign: K < the rows of W). Operands may have any alignment, row
// strides and N: X rows that are not 16-byte aligned are read with 4-byte
// loads; W, the bias and Y as w_mode says.
hipError_t launch_gemv_f32(int epi, int cols, GemvF32Args args, hipStream_t stream);
// Waves of a workgroup that split K, for this column block width and M.
int gemv_f32_waves_k(int cols, int M);
// W, Y and the bias 16-byte aligned with row strides and N multiples of 4.
bool gemv_f32_vector_rows(const GemvF32Args& a);
// The W mode for these operands: kWVector when gemv_f32_vector_rows holds,
// else kWRealign when N >= 4, else kWScalar.
int gemv_f32_w_mode(const GemvF32Args& a);

int gemv_f32_max_ksplit();
constexpr int kGemvMaxM = 64;

// ------------------------------------------------------------- integer path
// Fragment-packed int8 operand. A row-major int8 [R][K] matrix (R = the M rows
// of X, or the N columns of W) is stored as 32x32 fragments, ordered
// [R/32][K/32]; fragment (rb, kt) holds rows 32rb.. and k 32kt.. as 64 lanes x
// 16 bytes with lane = r % 32 + 32 * ((k % 32) / 16) and byte = k % 16 -- the
// v_mfma_i32_32x32x32_i8 operand of that block, one 16-byte load per lane.
// The packed copies cover M, N, K rounded up to multiples of kI8Tile (Mp, Np,
// Kp); elements past the real M, N or K are zero, so they add nothing.
struct NarrowI8Args {
  const int32_t* X;   // [M][K], ldx
  const int32_t* W;   // [K][N], ldw
  int8_t* X8p;        // X narrowed, fragment-packed over (Mp, Kp)
  int8_t* W8p;        // W narrowed, fragment-packed over (Np, Kp) (W transposed)
  int64_t ldx, ldw;
  int M, N, K;        // real sizes
  int Mp, Np, Kp;     // padded sizes (multiples of kI8Tile)
  // Range flags, one byte per 64x64 tile, all written on every call: 1 when the
  // tile holds a value outside [-128, 127], else 0. X: [Mp/64][Kp/64]; W:
  // [Np/64][Kp/64] (indexed by W's column tile, then its k tile).
  uint8_t* flags_x;
  uint8_t* flags_w;
};

struct GemmI32Args {
  const int8_t* A8p;  // fragment-packed X (int8 fast path)
  const int8_t* B8p;  // fragment-packed W^T (int8 fast path)
  const int32_t* X;   // [M][K], ldx   (exact i32 fallback)
  const int32_t* W;   // [K][N], ldw   (exact i32 fallback)
  const int32_t* bias;
  int32_t* C;         // [M][N], ldc
  int64_t ldx, ldw, ldc;
  int M, N, K;
  int Kp;             // K of the packed copies (int8 path; a multiple of kI8Tile)
  int tiles_m, tiles_n;
  // Range flags of the narrowing pass (int8 path): a tile takes the exact i32
  // path when a flag of its X row panels or W column panels is set.
  const uint8_t* flags_x;
  const uint8_t* flags_w;
};

constexpr int kI8Tile = 128;   // tile of the int8 MFMA path; packed copies are padded to it
hipError_t launch_narrow_i8(NarrowI8Args args, hipStream_t stream);
// variant = wave layout + fragment prefetch depth in 32-k steps:
//   0..2: 2x2 waves of 64x64 quadrants, depth 4, 2, 8 (8 needs K % 256 == 0,
//         else 4);
//   3:    K-split waves (each wave the whole tile on every fourth k step),
//         depth 2 (1 when K/128 is odd);
// -1 = default.
constexpr int kI8Variants = 4;
constexpr int kI8DefaultVariant = 3;
int gemm_i8_depth(int variant, int K);
const char* gemm_i8_layout(int variant);
hipError_t launch_gemm_i8(int epi, GemmI32Args args, hipStream_t stream, int variant = -1);
// Exact wrapping i32 GEMM on the vector ALUs: any shape, any alignment.
hipError_t launch_gemm_i32_valu(int epi, GemmI32Args args, hipStream_t stream);

// ------------------------------------- the reference's unfused GPU sequence
// Y = 0 (linalg.fill), and Y = epilogue(Y (+ bias)) in place (the bias /
// activation generic), for comparison with the fused kernels.
hipError_t launch_fill_zero_f32(float* Y, int64_t ldy, int M, int N, hipStream_t stream);
hipError_t launch_bias_act_f32(float* Y, int64_t ldy, const float* bias, int M, int N, int epi, float alpha,
                               hipStream_t stream);

}  // namespace edsl
