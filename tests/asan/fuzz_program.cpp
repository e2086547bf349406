// Sanitizer fuzz driver for the FunctionDef decoder (program.cpp): every
// fixture is compiled, described and bound to a function pointer; then
// truncated at every length and corrupted (1-4 random bytes, fixed seed)
// many times. Any out-of-bounds access or undefined behaviour aborts the run
// under -fsanitize=address,undefined. Test infrastructure only.
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iterator>
#include <random>
#include <string>
#include <vector>

#include "../../include/edsl_hip_program.h"

int main(int argc, char** argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: fuzz_program ITERATIONS FIXTURE...\n");
    return 2;
  }
  const long iters = atol(argv[1]);
  std::vector<std::string> cases;
  for (int i = 2; i < argc; ++i) {
    std::ifstream f(argv[i], std::ios::binary);
    cases.emplace_back(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
  }
  edsl_hip_module* m = edsl_hip_module_create();
  int compiled = 0;
  char buf[4096];
  for (const std::string& c : cases) {
    if (edsl_hip_module_compile_function(m, c.data(), c.size()) == 0) ++compiled;
    edsl_hip_module_list_functions(m, buf, sizeof buf);
    edsl_hip_module_describe(m, buf, sizeof buf);
  }
  // every listed function yields a pointer (or a clean error)
  const int n = edsl_hip_module_list_functions(m, nullptr, 0);
  std::string names(n + 1, '\0');
  edsl_hip_module_list_functions(m, &names[0], names.size());
  size_t pos = 0;
  while (pos < (size_t)n) {
    size_t end = names.find('\n', pos);
    if (end == std::string::npos || end > (size_t)n) end = n;
    const std::string fn = names.substr(pos, end - pos);
    (void)edsl_hip_module_get_function_pointer(m, fn.c_str());
    // binding: the index of a named parameter, a bind with the wrong shape
    // (an error), a bind of the right shape when it is 1x1 .. 64x64, unbind
    int idx = -1;
    (void)edsl_hip_module_param_index(m, fn.c_str(), "X", &idx);
    static float host[64 * 64 + 64];
    for (int64_t d = 1; d <= 64; d *= 4) {
      const int64_t shape[2] = {d, d};
      (void)edsl_hip_module_bind_parameter(m, fn.c_str(), idx < 0 ? 0 : idx, host, shape, 2);
      (void)edsl_hip_module_bind_parameter(m, fn.c_str(), 1, host, shape, 1);
    }
    edsl_hip_module_describe(m, buf, sizeof buf);
    (void)edsl_hip_module_unbind_parameter(m, fn.c_str(), -1);
    pos = end + 1;
  }
  edsl_hip_module_clear(m);
  for (const std::string& c : cases)
    for (size_t len = 0; len < c.size(); ++len) {
      edsl_hip_module_compile_function(m, c.data(), len);
      edsl_hip_module_clear(m);
    }
  std::mt19937_64 rng(12345);
  for (long it = 0; it < iters; ++it) {
    std::string c = cases[it % cases.size()];
    const int flips = 1 + (int)(rng() % 4);
    for (int f = 0; f < flips; ++f) c[rng() % c.size()] = (char)(rng() & 0xff);
    edsl_hip_module_compile_function(m, c.data(), c.size());
    edsl_hip_module_get_function_pointer(m, "x");
    edsl_hip_module_clear(m);
  }
  edsl_hip_module_destroy(m);
  printf("fuzz ok: %d of %zu fixtures compiled, %ld corruptions\n", compiled, cases.size(), iters);
  return 0;
}
