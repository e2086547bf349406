// Shared device-side definitions for the gfx950 dense-path kernels.
//
// Epilogue semantics follow the reference's linalg lowering of the dense layer:
//   bias:  linalg.generic body `arith.addf` / `arith.addi`
//          (reference cpp/src/builders/LinalgBuilder.cpp:301-339)
//   relu:  `arith.maximumf(x, 0)` for f32 (LinalgBuilder.cpp:213-215) -- NaN
//          propagates and max(-0, +0) = +0; for i32 the reference spells ReLU as
//          tensor_map(v -> If(v > 0, v, 0)) (LinalgBuilder.cpp:141-178).
//   leaky: max(x,0) + alpha*min(x,0) with arith.maximumf / arith.minimumf,
//          mulf, addf (LinalgBuilder.cpp:216-225).
//   if-relu: the f32 ReLU written tensor_map(v -> If(v > 0.0, v, 0.0))
//          (LinalgBuilder.cpp:141-178, comparison predicate
//          ArithBuilder.cpp:122-126): cmpf ogt is false for NaN and -0, so
//          both give the constant +0.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace edsl {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

// Epilogue code: bit 0 = bias present; bits 1-2 = activation.
enum : int {
  EPI_BIAS_BIT = 1,
  ACT_NONE = 0,
  ACT_RELU = 1,
  ACT_LEAKY = 2,
  ACT_IF_RELU = 3,
};
constexpr int epi_code(bool bias, int act) { return (bias ? 1 : 0) | (act << 1); }
constexpr bool epi_has_bias(int epi) { return (epi & 1) != 0; }
constexpr int epi_act(int epi) { return (epi >> 1) & 3; }

// arith.maximumf(x, +0.0): NaN in -> NaN out; -0 -> +0.
__device__ __forceinline__ float maximumf_zero(float x) {
  return (x > 0.0f || x != x) ? x : 0.0f;
}
// arith.minimumf(x, +0.0): NaN in -> NaN out; -0 -> -0; positive -> +0.
__device__ __forceinline__ float minimumf_zero(float x) {
  return (x < 0.0f || x != x || x == 0.0f) ? x : 0.0f;
}

template <int EPI>
__device__ __forceinline__ float apply_epilogue_f32(float acc, float b, float alpha) {
  float y = acc;
  if constexpr (epi_has_bias(EPI)) y = __fadd_rn(y, b);
  if constexpr (epi_act(EPI) == ACT_RELU) {
    y = maximumf_zero(y);
  } else if constexpr (epi_act(EPI) == ACT_IF_RELU) {
    y = y > 0.0f ? y : 0.0f;
  } else if constexpr (epi_act(EPI) == ACT_LEAKY) {
    // mulf then addf, each rounded (no contraction), as the reference emits them.
    y = __fadd_rn(maximumf_zero(y), __fmul_rn(minimumf_zero(y), alpha));
  }
  return y;
}

template <int EPI>
__device__ __forceinline__ int32_t apply_epilogue_i32(int32_t acc, int32_t b) {
  // arith.addi wraps modulo 2^32.
  int32_t y = acc;
  if constexpr (epi_has_bias(EPI)) y = (int32_t)((uint32_t)y + (uint32_t)b);
  if constexpr (epi_act(EPI) == ACT_RELU) y = y > 0 ? y : 0;
  return y;
}

// Raw buffer loads: the <4 x i32> descriptor form of the intrinsics, so that a
// descriptor built from uniform values stays in scalar registers. A load whose
// per-lane offset lies at or past the descriptor's byte count reads zero.
// (These names bind to the intrinsics; they have no definitions.)
__device__ f32x4 raw_buffer_load_f32x4(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4f32");
__device__ f32x2 raw_buffer_load_f32x2(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v2f32");
__device__ float raw_buffer_load_f32(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.f32");
__device__ i32x4 raw_buffer_load_i32x4(i32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");

// Descriptor of `bytes` bytes from `base` (raw addressing: stride 0, the
// 32-bit data format word of the gfx9 family), clamped to [0, 2^31 - 1].
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

// Workgroup -> output tile mapping.
//
// The hardware hands workgroup w to XCD (w % 8). Each XCD has its own L2, so
// consecutive *logical* tiles are given to the same XCD: logical id
// L = (w % 8) * (T / 8) + w / 8 when the tile count T divides by 8. Logical ids
// are then walked in groups of kGroupM tile-rows, column-major inside a group,
// so one XCD's tiles share a few A row-panels and B column-panels. With eight
// rows, the 32 tiles one XCD runs at once at 4096^3 (128x256 tiles) cover
// 8 rows x 4 columns: 16 + 16 MiB of panels per round, against 8 + 32 MiB
// for four rows (same time; 537 against 671 MB of L2-miss reads).
__device__ __forceinline__ void tile_coords(int wg, int tiles_m, int tiles_n, int& tm,
                                            int& tn) {
  constexpr int kXcds = 8;
  constexpr int kGroupM = 8;
  const int total = tiles_m * tiles_n;
  int L = wg;
  if (total % kXcds == 0) L = (wg % kXcds) * (total / kXcds) + wg / kXcds;
  const int span = kGroupM * tiles_n;
  const int group = L / span;
  const int first_m = group * kGroupM;
  const int rows = min(tiles_m - first_m, kGroupM);
  const int in_group = L - group * span;
  tm = first_m + in_group % rows;
  tn = in_group / rows;
}

}  // namespace edsl
