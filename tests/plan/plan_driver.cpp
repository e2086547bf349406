// Prints the fp32 tile plan for each query line "M N K aligned cus [lda ldb]" on
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
    long long M, N, K, lda = -1, ldb = -1;
    int aligned, cus;
    const int got = sscanf(line, "%lld %lld %lld %d %d %lld %lld", &M, &N, &K, &aligned, &cus, &lda, &ldb);
    if (got != 5 && got != 7) return 2;
    // Row strides K and N (contiguous operands) unless given.
    if (got == 5) {
      lda = K;
      ldb = N;
    }
    const int c = edsl::plan_f32_tile(edsl::F32TileQuery{M, N, K, lda, ldb, aligned != 0, cus, -1});
    printf("%s\n", edsl::gemm_f32_config(c).name);
  }
  return 0;
}
