// Prints the fp32 tile plan for each query line "M N K aligned cus" on
// stdin, and the configuration table for the line "table". Built with g++
// against ml-edsl_amd/csrc/plan_f32.cpp alone (no HIP). Test infrastructure.
#include <cstdio>
#include <cstring>

#include "../../ml-edsl_amd/csrc/plan_f32.hpp"

int main() {
  char line[256];
  while (fgets(line, sizeof(line), stdin)) {
    if (strncmp(line, "table", 5) == 0) {
      for (int c = 0; c < edsl::gemm_f32_num_configs(); ++c) {
        const edsl::GemmF32Config& g = edsl::gemm_f32_config(c);
        printf("%d %s %d %d %d %d\n", c, g.name, g.bm, g.bn, g.bk, g.guard);
      }
      continue;
    }
    long long M, N, K;
    int aligned, cus;
    if (sscanf(line, "%lld %lld %lld %d %d", &M, &N, &K, &aligned, &cus) != 5) return 2;
    // Contiguous operands: row strides K and N.
    const int c = edsl::plan_f32_tile(edsl::F32TileQuery{M, N, K, K, N, aligned != 0, cus, -1});
    printf("%s\n", edsl::gemm_f32_config(c).name);
  }
  return 0;
}
