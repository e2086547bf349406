// The fp32 tile configurations and the planner that picks one for a layer.
// Host-only (no HIP): the kernels are in gemm_f32.hip, gemm_f32_m16.hip and
// gemm_f32_direct.hip, the planner's callers in runtime.cpp, and tests build
// this file alone to check plans without a device.
#pragma once

#include <stdint.h>

namespace edsl {

// Bounds handling of a tile configuration.
enum : int {
  kGuardNone = 0,  // M, N, K multiples of the tile; 16-byte aligned operands and row strides
  kGuardEdge = 1,  // partial edge tiles; 16-byte aligned operands, strides, N and K multiples of 4
  kGuardAll = 2,   // any shape and alignment (element-wise checks)
  kGuardScalar = 3,  // partial edge tiles, any alignment, K and N: 4-byte accesses at clamped addresses
};

struct GemmF32Config {
  int bm, bn, bk;
  int waves_m, waves_n;
  int guard;          // kGuard*
  const char* name;
};

// The shipped tile configurations (plan_f32.cpp says what each is for).
// A family is a tile with its bounds variants -- exact (kGuardNone), edge
// tiles (kGuardEdge), any shape (kGuardScalar) -- where built.
enum F32Tile : int {
  kF32Guard64 = 0,      // 64x64x16, element-checked (kGuardAll)
  kF32T32,              // 32x32x64, four K waves, 32x32 MFMA blocks
  kF32T32Edge,
  kF32T32Any,
  kF32T64Any,           // 64x64x32, two K waves, loads four steps ahead
  kF32T64K2Any,         // 64x64x64, two K waves, loads two steps ahead
  kF32T256Any,          // 256x256x16, 4x4 waves
  kF32M16_128,          // 128x128x32 on 16x16 MFMA blocks (gemm_f32_m16.hip layout 0)
  kF32M16_128Edge,
  kF32M16_128Any,
  kF32M16_64,           // 64x64x64 on 16x16 blocks (layout 1)
  kF32M16_64Edge,
  kF32M16_128x256,      // 128x256x32 on 16x16 blocks, eight waves (layout 2)
  kF32M16_128x256Edge,
  kF32M16_128W8,        // 128x128x32 on 16x16 blocks, eight waves (layout 3)
  kF32M16_128W8Edge,
  kF32Direct128,        // 128x128x16, one wave per tile, no LDS (gemm_f32_direct.hip)
  kF32Direct128Edge,
  kF32Direct64,         // 64x64x16, one wave per tile, no LDS
  kF32Direct64K4,       // 64x64x64, four waves splitting K, partials summed through LDS
  kF32Direct64K4Edge,
  kF32Direct16K4,       // 16x16x64, four waves splitting K, every load up front (small layers)
  kF32DirectRC2x2,      // 16R x 16C, four waves splitting K (K % 16 == 0, K >= 64; R x C blocks per wave)
  kF32DirectRC3x3,
  kF32DirectRC5x5,
  kF32DirectRC6x6,
  kF32DirectRC3x6,
  kF32DirectRC6x3,
  kF32DirectRC4x4,      // 64x64x64 on the R x C kernel: one round of K-split 64x64 tiles
  kF32DirectRC2x2Edge,  // edge twins of the square R x C tiles
  kF32DirectRC3x3Edge,
  kF32DirectRC4x4Edge,
  kF32DirectRC5x5Edge,
  kF32DirectRC6x6Edge,
  kF32Tiles
};
int gemm_f32_num_configs();
const GemmF32Config& gemm_f32_config(int cfg);

// Rows up to which a layer is one the small-M kernel could take; such layers
// go to the 32x32 tiles when it does not.
constexpr int kF32SmallM = 64;

struct F32TileQuery {
  int64_t M, N, K;
  int64_t lda, ldb;  // row strides of A and B, in elements
  // Every operand 16-byte aligned, row strides multiples of 4 elements.
  bool aligned;
  int cus;      // compute units of the device
  int forced;   // a configuration to take when it fits these operands, or -1
};
// The configuration for a tiled fp32 layer (M, N, K >= 0).
int plan_f32_tile(const F32TileQuery& q);

// The one-wave tiles read A and B through buffer descriptors with 32-bit
// byte offsets: 128 rows of A from a tile's first row, and all K rows of B
// (plus a partial group's overrun) from a tile's first column, must be
// addressable that way.
bool gemm_f32_direct_offsets_fit(int64_t K, int64_t lda, int64_t ldb);

}  // namespace edsl
