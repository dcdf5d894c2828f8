// expf_check.cpp - test helper: compares llmrs::exact_expf (the device
// kernels' exponential, compiled here for the host) with the host libm's
// expf over every float bit pattern from `first` to `last` in steps of
// `stride`, and prints "checked <n> mismatches <m> first <hex>".
// Build: g++ -O2 -std=c++17 -ffp-contract=off -fopenmp.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "kernels/exact_math.h"

int main(int argc, char** argv) {
  const uint64_t first = argc > 1 ? std::strtoull(argv[1], nullptr, 0) : 0;
  const uint64_t last = argc > 2 ? std::strtoull(argv[2], nullptr, 0) : 0xffffffffull;
  const uint64_t stride = argc > 3 ? std::strtoull(argv[3], nullptr, 0) : 1;
  long long checked = 0, bad = 0;
  uint64_t first_bad = ~0ull;
#pragma omp parallel for reduction(+ : checked, bad) reduction(min : first_bad) schedule(static)
  for (long long i = (long long)first; i <= (long long)last; i += (long long)stride) {
    const uint32_t u = (uint32_t)i;
    float x;
    std::memcpy(&x, &u, 4);
    if (std::isnan(x)) continue;
    const float a = expf(x), b = llmrs::exact_expf(x);
    uint32_t ua, ub;
    std::memcpy(&ua, &a, 4);
    std::memcpy(&ub, &b, 4);
    ++checked;
    if (ua != ub) {
      ++bad;
      if ((uint64_t)u < first_bad) first_bad = u;
    }
  }
  std::printf("checked %lld mismatches %lld first 0x%llx\n", checked, bad,
              (unsigned long long)(bad ? first_bad : 0));
  return 0;
}
