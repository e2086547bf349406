// The fp32 tile configurations and their planner (plan_f32.hpp).
#include "plan_f32.hpp"

#include <initializer_list>

namespace edsl {
namespace {

// The shipped tile configurations, indexed by F32Tile (plan_f32.hpp). Each
// name spells the tile (BM x BN x BK), its waves and, for the tiles on 32x32
// MFMA blocks, the waves splitting K (_kN) and the K steps of global loads
// issued ahead (_pfN); a suffix gives the bounds variant (_edge: kGuardEdge,
// _anyshape: kGuardScalar, _guard: kGuardAll).
//  kF32Guard64: 64x64x16, 2x2 waves, element-checked loads and stores: any
//      shape and alignment; the plan for K = 0.
//  kF32T32*: 32x32x64 on one output block with four waves splitting each K
//      step, all four 64-deep K steps of a 256-deep K loaded up front (256^3:
//      7.54 TFLOP/s against 7.31 one step ahead); layers of at most 64 rows
//      and many-tile shapes of small outputs.
//  kF32T64Any: 64x64x32, two waves per output block splitting K, loads four
//      steps ahead, LDS stores of the next step issued ahead of the MFMAs
//      (SCHED 1): any-shape layers of at most one tile per CU.
//  kF32T64K2Any: 64x64x64, two K waves, loads two steps ahead: any-shape
//      layers of more 64x64 tiles than CUs (1025^3: 49.0 us against 54.8 us
//      for the 64x64 layout on 16x16 blocks).
//  kF32T256Any: 256x256x16, 4x4 waves (wave tile 64x64): 4001^3 and
//      misaligned 4096^3 1116 and 1059 us against 1153 and 1151 us for
//      kF32M16_128Any.
//  kF32M16_*: the tiles on 16x16 MFMA blocks (gemm_f32_m16.hip): 128x128x32
//      with one wave per SIMD and two workgroups per CU (4096^3 965 us
//      against 986 us for 256x256x16 with 16 waves on 32x32 blocks; 2048^3
//      141 against 165 us for 128x128x16), its 64x64x64 twin (1024^3 21.6
//      against 23.3 us), 128x256x32 with 2x4 waves of 64x64 and one
//      workgroup per CU (4096^3 938-941 against 959-962 us for 128x128,
//      8192^3 7411 against 7519 us), and 128x128x32 with eight waves for
//      exactly one tile per CU (2048^3 137 against 139-141 us). A 64x64x64
//      layout with eight waves, two per wave tile splitting K, measured 2 %
//      slower than the four-wave one at 1024^3 (22.3-22.5 against 21.8-22.1
//      us) once the latter's fragment reads were placed early, and is not
//      built.
//  kF32Direct128*: 128x128x16 with one wave per tile and no LDS
//      (gemm_f32_direct.hip): fragments loaded straight into the MFMA operand
//      registers, four tiles per CU; for layers whose tiles fill whole rounds
//      of 4 x CUs (4096^3 900-906 us against 926-934 us for 128x256x32,
//      8192^3 7148 against 7342 us, 4096x256x4096 70.5 against 72.9 us).
//  kF32Direct64*: its 64x64 twin, one wave per tile (bk 16) or four waves of
//      one workgroup splitting K (bk 64), partials summed through LDS, and
//      the split tile's edge twin (the unsplit one's tied the eight-wave
//      128x128 edge tile at 2000^3, 122.3 against 123.1 us, and is not
//      built). K
//      split two or eight ways measured no better than four (1024^3 19.5-19.6
//      against 18.2-19.6 us, 4096x4096x512 121.3 against 121.7 us) and is
//      not built.
//  kF32Direct16K4: the one-wave 16x16 tile for small layers, K split over
//      four waves of a workgroup with every fragment loaded up front.
//  kF32DirectRC*: one-wave tiles of R x C 16x16 blocks (32x32, 48x48, 80x80,
//      96x96, 48x96, 96x48), K split over four waves of a workgroup, for
//      layers whose 64x64 tiles leave a round of workgroups partly empty
//      (768^3: 144 tiles of 64x64 or 256 of 48x48, 15.3 against 10.5 us),
//      the 4x4 instance (64x64) for one round of 64x64 K-split tiles, and
//      edge twins of the square ones (1500^3 on 96x96: 62.7 against 84.6 us).
const GemmF32Config kConfigs[] = {
    {64, 64, 16, 2, 2, kGuardAll, "f32_64x64x16_w2x2_guard"},
    {32, 32, 64, 1, 1, kGuardNone, "f32_32x32x64_w1x1_k4_pf4"},
    {32, 32, 64, 1, 1, kGuardEdge, "f32_32x32x64_w1x1_k4_pf4_edge"},
    {32, 32, 64, 1, 1, kGuardScalar, "f32_32x32x64_w1x1_k4_pf4_anyshape"},
    {64, 64, 32, 2, 2, kGuardScalar, "f32_64x64x32_w2x2_k2_pf4_anyshape"},
    {64, 64, 64, 2, 2, kGuardScalar, "f32_64x64x64_w2x2_k2_pf2_anyshape"},
    {256, 256, 16, 4, 4, kGuardScalar, "f32_256x256x16_w4x4_anyshape"},
    {128, 128, 32, 2, 2, kGuardNone, "f32_128x128x32_mfma16"},
    {128, 128, 32, 2, 2, kGuardEdge, "f32_128x128x32_mfma16_edge"},
    {128, 128, 32, 2, 2, kGuardScalar, "f32_128x128x32_mfma16_anyshape"},
    {64, 64, 64, 2, 2, kGuardNone, "f32_64x64x64_mfma16"},
    {64, 64, 64, 2, 2, kGuardEdge, "f32_64x64x64_mfma16_edge"},
    {128, 256, 32, 2, 4, kGuardNone, "f32_128x256x32_mfma16"},
    {128, 256, 32, 2, 4, kGuardEdge, "f32_128x256x32_mfma16_edge"},
    {128, 128, 32, 2, 4, kGuardNone, "f32_128x128x32_mfma16_w8"},
    {128, 128, 32, 2, 4, kGuardEdge, "f32_128x128x32_mfma16_w8_edge"},
    {128, 128, 16, 1, 1, kGuardNone, "f32_128x128x16_direct"},
    {128, 128, 16, 1, 1, kGuardEdge, "f32_128x128x16_direct_edge"},
    {64, 64, 16, 1, 1, kGuardNone, "f32_64x64x16_direct"},
    {64, 64, 64, 1, 1, kGuardNone, "f32_64x64x64_direct_k4"},
    {64, 64, 64, 1, 1, kGuardEdge, "f32_64x64x64_direct_k4_edge"},
    {16, 16, 64, 1, 1, kGuardNone, "f32_16x16x64_direct_k4"},
    {32, 32, 64, 1, 1, kGuardNone, "f32_32x32x64_direct_rc"},
    {48, 48, 64, 1, 1, kGuardNone, "f32_48x48x64_direct_rc"},
    {80, 80, 64, 1, 1, kGuardNone, "f32_80x80x64_direct_rc"},
    {96, 96, 64, 1, 1, kGuardNone, "f32_96x96x64_direct_rc"},
    {48, 96, 64, 1, 1, kGuardNone, "f32_48x96x64_direct_rc"},
    {96, 48, 64, 1, 1, kGuardNone, "f32_96x48x64_direct_rc"},
    {64, 64, 64, 1, 1, kGuardNone, "f32_64x64x64_direct_rc"},
    {32, 32, 64, 1, 1, kGuardEdge, "f32_32x32x64_direct_rc_edge"},
    {48, 48, 64, 1, 1, kGuardEdge, "f32_48x48x64_direct_rc_edge"},
    {64, 64, 64, 1, 1, kGuardEdge, "f32_64x64x64_direct_rc_edge"},
    {80, 80, 64, 1, 1, kGuardEdge, "f32_80x80x64_direct_rc_edge"},
    {96, 96, 64, 1, 1, kGuardEdge, "f32_96x96x64_direct_rc_edge"},
};
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);
static_assert(kNumConfigs == kF32Tiles, "one table entry per F32Tile");

}  // namespace

int gemm_f32_num_configs() { return kNumConfigs; }

bool gemm_f32_direct_offsets_fit(int64_t K, int64_t lda, int64_t ldb) {
  constexpr int64_t kMax = 0x7fffffff;
  return K >= 0 && lda >= 0 && ldb >= 0 && 128 * lda * 4 + 64 <= kMax && (K + 16) * ldb * 4 + 1024 <= kMax;
}
const GemmF32Config& gemm_f32_config(int cfg) { return kConfigs[cfg]; }

int plan_f32_tile(const F32TileQuery& q) {
  const int64_t M = q.M, N = q.N, K = q.K;
  const bool aligned = q.aligned;
  int cfg = -1;
  // Partial edge tiles need 16-byte vectors that are all in or all out of
  // range: K and N multiples of 4 (true for every contiguous aligned operand).
  const bool edge_ok = aligned && K >= 4 && N >= 4 && M >= 1 && K % 4 == 0 && N % 4 == 0;
  const bool direct_ok = gemm_f32_direct_offsets_fit(K, q.lda, q.ldb);
  auto fits = [&](int c) {
    const GemmF32Config& g = gemm_f32_config(c);
    if (c >= kF32Direct128 && !direct_ok) return false;  // the one-wave tiles
    if (c == kF32Direct16K4 && K > 512)
      return false;
    if (c >= kF32DirectRC2x2) {  // the R x C tiles split K / 16 groups over four waves
      if (g.guard == kGuardEdge) return edge_ok;
      return aligned && M % g.bm == 0 && N % g.bn == 0 && K % 16 == 0 && K >= 64;
    }
    if (g.guard == kGuardNone) return aligned && K > 0 && M % g.bm == 0 && N % g.bn == 0 && K % g.bk == 0;
    if (g.guard == kGuardEdge) return edge_ok;
    return K > 0;  // kGuardScalar, kGuardAll: any shape, stride and alignment
  };
  // The first of a tile's bounds variants that fits these operands, or -1.
  auto pick = [&](std::initializer_list<int> variants) {
    for (int c : variants)
      if (fits(c)) return c;
    return -1;
  };
  auto tiles_of = [&](int c) {
    const GemmF32Config& g = gemm_f32_config(c);
    return (int64_t)((M + g.bm - 1) / g.bm) * ((N + g.bn - 1) / g.bn);
  };
  if (q.forced >= 0 && q.forced < gemm_f32_num_configs() && fits(q.forced)) {
    cfg = q.forced;
  } else if (K > 0 && M <= kF32SmallM) {
    // Layers of at most 64 rows that the small-M kernel does not take (W or Y
    // rows unaligned, N not a multiple of 4, short K) run on the 32x32 tiles:
    // larger tiles spend most of their MFMAs on rows past M (16x4096x50257:
    // 287 us on 32x32 against 364-1139 us on 64x64 to 256x256 tiles and 406
    // us on the element-checked 64x64 tile; the same order at 16, 48 and 64
    // rows).
    cfg = pick({kF32T32, kF32T32Edge, kF32T32Any});
  } else if (K > 0) {
    // Candidates are tried in order of preference. The first whose tiles give
    // every CU a workgroup is taken, unless it is larger than 64x64 and needs
    // more than one round of workgroups with the last round keeping fewer
    // than three quarters of the CUs busy (4097x4096: 272 tiles of 256x256
    // would take two rounds of 4096^3-sized work). When none fills the chip,
    // the candidate with the most tiles.
    int best = -1, first_rejected = -1;
    int64_t best_tiles = 0;
    auto consider = [&](int c) {  // true when c is taken
      if (c < 0) return false;
      const GemmF32Config& g = gemm_f32_config(c);
      const int64_t tiles = tiles_of(c);
      if (tiles >= q.cus) {
        const int64_t rounds = (tiles + q.cus - 1) / q.cus;
        if (g.bm * g.bn > 64 * 64 && 4 * tiles < 3 * rounds * q.cus) {
          if (first_rejected < 0) first_rejected = c;
          return false;
        }
        cfg = c;
        return true;
      }
      if (tiles > best_tiles) {
        best_tiles = tiles;
        best = c;
      }
      return false;
    };
    if (edge_ok) {
      // 16-byte vector tiles (exact where the tile divides the layer, else
      // their edge-tile twins): the 128x128 tile on 16x16 MFMA blocks, then
      // its 64x64 twin, then 32x32 tiles.
      const int c128 = pick({kF32M16_128, kF32M16_128Edge});
      const int c64 = pick({kF32M16_64, kF32M16_64Edge});
      bool skip128 = false;
      if (tiles_of(c128) >= q.cus) {
        // The 128x128 tile against its 64x64 and 128x256 twins, by how the
        // tiles fall on the CUs. Two 128x128 (or 64x64) workgroups share a
        // CU, so a CU with n tiles runs n/2 pairs (each pair ~0.94x the time
        // of two tiles alone) and one tile alone when n is odd; a 64x64 tile
        // takes ~0.27x a 128x128 one, and a 128x256 workgroup (eight waves,
        // one per CU) ~0.98x a pair. 3000^3: 576 tiles of 128x128 leave 64
        // CUs a third tile, 533 us against 470 us on 2209 tiles of 64x64.
        // 4096^3: 939-940 us on 512 tiles of 128x256 against 952-960 us on
        // 1024 of 128x128 (8192^3 7411 against 7519 us); 6000^3 stays on
        // 128x128 (3157 us against 3437 us for 1128 tiles of 128x256, five
        // rounds of one per CU), and so does 2048^3 (one tile per CU, 141 us
        // against 153 us on 64x64). The constants were fitted on those
        // shapes on MI355X.
        auto cu_time = [&](int64_t n_tiles) {
          const int64_t n = (n_tiles + q.cus - 1) / q.cus;
          return (double)(n / 2) * 2.0 * 0.94 + (double)(n % 2);
        };
        const double t128 = cu_time(tiles_of(c128));
        const double t64 = 0.27 * cu_time(tiles_of(c64));
        const int cwide = pick({kF32M16_128x256, kF32M16_128x256Edge});
        const int64_t tw = tiles_of(cwide);
        const double twide =
            tw >= q.cus ? (double)((tw + q.cus - 1) / q.cus) * 2.0 * 0.94 * 0.98 : 1e30;
        // The one-wave 128x128 tile (gemm_f32_direct.hip) runs one tile per
        // SIMD, four per CU at a time; a round of them takes ~3.6 of the
        // units above (4096^3: 914-927 us against 937 us for two rounds of
        // 128x256; 8192^3: 7167 against 7373-7385 us). It wins where its
        // tiles fill whole rounds of 4 x cus.
        const int cdirect = pick({kF32Direct128, kF32Direct128Edge});
        const double tdirect =
            cdirect >= 0 ? (double)((tiles_of(cdirect) + 4 * q.cus - 1) / (4 * q.cus)) * 3.6 : 1e30;
        if (tdirect < twide && tdirect < t128 && tdirect < t64) {
          cfg = cdirect;
        } else if (twide <= t128 && twide <= t64) {
          cfg = cwide;
        } else if (t64 < t128) {
          skip128 = true;
        } else if (tiles_of(c128) == q.cus) {
          // Exactly one 128x128 tile per CU: its eight-wave layout (two waves
          // per SIMD to cover each other's waits; 2048^3 137 against 139-141
          // us, 2000^3 137 against 141 us).
          cfg = pick({kF32M16_128W8, kF32M16_128W8Edge});
        }
      }
      // The one-wave 64x64 tiles (gemm_f32_direct.hip) take every layer of
      // whole 64x64 tiles that the one-wave 128x128 tile does not fill, from
      // about half a tile per CU on: with K split over four waves of a workgroup, or
      // unsplit where the tiles fill one or two waves per SIMD exactly. Same
      // box against the tiles the model above picks: 1024^3 18.2 against 18.9
      // us, 4096x4096x512 121.7 against 134.3 us, 2048^3 (unsplit) 117.3
      // against 122.7 us, 3072^3 394 against 428 us, 5120^3 1779 against 1929
      // us, 6144^3 3071 against 3229 us, 2048x4096x4096 (unsplit) 455 against
      // 466 us on 128x256; 4096^3 stays on the 128x128 one (902 against 915
      // us), and so do more than two unsplit waves per SIMD (4096^3 unsplit:
      // 1120 us). Short K (below 256) is left to the tiles above.
      // Partial 64x64 tiles take the K-split edge twin from one tile per CU
      // to two (1000^3 21.8 against 23.6 us, 1000x4000x1000 64.0 against
      // 68.7 us on the LDS-staged 64x64 edge tile); at four per CU it loses
      // to the eight-wave 128x128 edge tile (2000^3 133.4 against 121.8 us),
      // with more it ties (3000^3 428 against 440 us, 4097x4096x4096 1056
      // against 1052 us), and short K is slower (4097x256x4096 114 against
      // 88 us).
      if (cfg != kF32Direct128 && cfg != kF32Direct128Edge && K >= 256) {
        const int64_t t64n = ((M + 63) / 64) * ((N + 63) / 64);
        int cd = -1;
        if (M % 64 == 0 && N % 64 == 0) {
          // From 9/16 of a tile per CU (768^3: 144 tiles, 15.1 against 18.3 us
          // on the 32x32 tiles; 768x256x1024, 192 tiles: 7.9 against 9.0 us;
          // 768x1024x1024 18.8 against 23.0 us); fewer tiles lose
          // (320x448x1536, 120 tiles: 10.3 against 9.3 us).
          if (16 * t64n >= 9 * q.cus) {
            if (t64n % (4 * q.cus) == 0 && t64n <= 8 * q.cus) cd = pick({kF32Direct64});
            if (cd < 0) cd = pick({kF32Direct64K4});
          }
        } else if (K >= 512 && t64n >= q.cus && t64n <= 2 * q.cus) {
          cd = pick({kF32Direct64K4Edge});
        }
        if (cd >= 0) cfg = cd;
      }
      // The R x C one-wave tiles (K split over four waves, one workgroup per
      // CU) where their tiles fill the CUs more evenly than 64x64 ones. Cost:
      // the MFMAs of each SIMD, R x C blocks over a quarter of K per round of
      // workgroups; the 64x64 K-split tile is R = C = 4, the unsplit one 16
      // blocks over all of K per round of four tiles per CU. In one round
      // (768^3: 256 tiles of 48x48, 10.5 against 15.3 us; 1536x3072x1536 on
      // 96x96 114.9 against 141.6 us; 720x768x720 10.5 against 19.0 us on the
      // 32x32 edge tile); over several rounds tiles of 64 and more that read
      // no more per output than 64x64 ones (2560x1024x2560 on 80x80 113.3
      // against 124.8 us; 48x48 tiles over nine rounds took 234.2 us at
      // 2304^3 against 211.7 us for 64x64).
      if (cfg != kF32Direct128 && cfg != kF32Direct128Edge && K >= 256 && edge_ok && direct_ok) {
        const int64_t t64n = ((M + 63) / 64) * ((N + 63) / 64);
        const int64_t cus = q.cus;
        int64_t inc = -1;  // the incumbent's cost where comparable
        if (cfg == kF32Direct64K4 || cfg == kF32Direct64K4Edge) inc = 16 * ((t64n + cus - 1) / cus);
        if (cfg == kF32Direct64) inc = 64 * ((t64n + 4 * cus - 1) / (4 * cus));
        // Candidates by cost; a tile that reads more per output than a 64x64
        // one, or is narrower than 64, over several rounds only where it costs
        // at most 2/3 of every other candidate (128x4096x4096: 512 tiles of
        // 32x32 in two rounds, 51.0 us, against one half-full round of 64x64,
        // 62.9-63.2 us).
        struct Cand {
          int c;
          int64_t cost, rounds;
          bool light;  // one round, or no more reads per output than 64x64
        };
        Cand cands[7];
        int n_cands = 0;
        for (int c0 : {kF32DirectRC2x2, kF32DirectRC3x3, kF32DirectRC4x4, kF32DirectRC5x5, kF32DirectRC6x6,
                       kF32DirectRC3x6, kF32DirectRC6x3}) {
          const int edge_twin = c0 == kF32DirectRC2x2 ? kF32DirectRC2x2Edge
                                : c0 == kF32DirectRC3x3 ? kF32DirectRC3x3Edge
                                : c0 == kF32DirectRC4x4 ? kF32DirectRC4x4Edge
                                : c0 == kF32DirectRC5x5 ? kF32DirectRC5x5Edge
                                : c0 == kF32DirectRC6x6 ? kF32DirectRC6x6Edge : -1;
          // Edge twins from K = 384 (at 256 the LDS-staged edge tiles were
          // 1-9 % faster: 96x256x4096 6.0 against 6.6 us; 500^3 5.8 against
          // 8.6 us).
          const int c = fits(c0) ? c0 : edge_twin >= 0 && K >= 384 && fits(edge_twin) ? edge_twin : -1;
          if (c < 0) continue;
          const GemmF32Config& g = gemm_f32_config(c);
          const int64_t rounds = (tiles_of(c) + cus - 1) / cus;
          const int64_t cost = (int64_t)(g.bm / 16) * (g.bn / 16) * rounds;
          // Over several rounds only square-ish tiles of 64 and more (48x96
          // over three rounds: 1536x1024x2304 79.6 against 72.2 us for 64x64).
          const bool light = rounds == 1 || (g.bm >= 64 && g.bn >= 64 && 32 * (g.bm + g.bn) <= g.bm * g.bn);
          cands[n_cands++] = {c, cost, rounds, light};
        }
        int64_t light_min = -1;
        for (int i = 0; i < n_cands; ++i)
          if (cands[i].light && (light_min < 0 || cands[i].cost < light_min)) light_min = cands[i].cost;
        int best_rc = -1;
        int64_t best_cost = 0, best_rounds = 0;
        for (int i = 0; i < n_cands; ++i) {
          const Cand& k = cands[i];
          if (!k.light && !(light_min < 0 || 3 * k.cost <= 2 * light_min)) continue;
          if (best_rc < 0 || k.cost < best_cost || (k.cost == best_cost && k.rounds < best_rounds)) {
            best_rc = k.c;
            best_cost = k.cost;
            best_rounds = k.rounds;
          }
        }
        // With no comparable incumbent: one round at least half full, or
        // several rounds at 2/3 of the cost of such a round at most.
        bool take = best_rc >= 0 && (inc >= 0 ? best_cost < inc : best_rounds == 1 && 2 * tiles_of(best_rc) >= cus);
        if (best_rc >= 0 && inc < 0 && best_rounds > 1)
          for (int i = 0; i < n_cands; ++i)
            if (cands[i].rounds == 1 && 2 * tiles_of(cands[i].c) >= cus && 3 * best_cost <= 2 * cands[i].cost)
              take = true;
        if (take)
          cfg = best_rc;
        else if (cfg == kF32Direct64K4 && t64n <= cus && fits(kF32DirectRC4x4))
          // One round of K-split 64x64 tiles: the R x C kernel's 4 x 4 instance
          // (1024^3 20.1-20.3 against 20.6-20.8 us, alternating on one box;
          // over several rounds neither is ahead: 3072^3 425-447 against
          // 415-445 us). Its edge twin measured no better than the 64x64
          // K-split edge twin at 1000^3 (21.5-22.6 against 22.0 us).
          cfg = kF32DirectRC4x4;
      }
      // Small layers of at most one 16x16 tile per CU, K up to 512: the 16x16
      // one-wave tile with K split over four waves and every load up front
      // (256^3 2.9 against 4.4 us on the 32x32 tile; 256x512x256 3.6 against
      // 6.0 us). With more tiles it ties or loses (512x256x512 4.8 against
      // 4.8 us, 512^3 7.5 against 6.6 us).
      if (cfg < 0 && tiles_of(kF32Direct16K4) <= q.cus) {
        const int c16 = pick({kF32Direct16K4});
        if (c16 >= 0) cfg = c16;
      }
      if (cfg < 0 && !skip128) consider(c128);
      if (cfg < 0) consider(c64);
      if (cfg < 0) consider(pick({kF32T32, kF32T32Edge}));
    } else {
      // Rows not 16-byte aligned, or K or N not a multiple of 4: the
      // any-shape tiles (4-byte accesses at clamped addresses) keep such
      // layers on large MFMA tiles (2001^3: 57.8 TFLOP/s on the small
      // element-checked tile alone). Measured order: 256x256 first (4001^3
      // and misaligned 4096^3: 1116 and 1059 us against 1153 and 1151 us for
      // 128x128 on 16x16 blocks), then 128x128 on 16x16 blocks (2001^3 175 us
      // against 233 us for 128x128 on 32x32 blocks, which is therefore not
      // built, and 194 us for 64x64;
      // 2048^3 with every row misaligned 174 against 179 us), then the 64x64
      // tiles: with loads four K steps ahead while there is one workgroup per
      // CU at most (at two per CU the other workgroup hides the loads and the
      // two-step twin wins), then 32x32.
      for (int c : {kF32T256Any, kF32M16_128Any})
        if (consider(c)) break;
      if (cfg < 0 && tiles_of(kF32T64Any) <= q.cus) consider(kF32T64Any);
      if (cfg < 0) consider(kF32T64K2Any);
      if (cfg < 0) consider(kF32T32Any);
    }
    if (cfg < 0) cfg = best >= 0 ? best : first_rejected;
  }
  if (cfg < 0) cfg = kF32Guard64;  // K = 0: any shape and alignment
  return cfg;
}

}  // namespace edsl
