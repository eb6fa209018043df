// Test driver (not product): checks gkv::expf_cpu_exact, the fp32 exp of the
// exact attention path, against the host C library's expf on every fp32 input
// (all 2^32 bit patterns; NaNs compared by NaN-ness). Prints the number of
// mismatches and the first few; exit status 0 when there are none.
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "exact_math.hpp"

int main(int argc, char **argv) {
  const int n_threads = argc > 1 ? atoi(argv[1]) : 8;
  std::atomic<uint64_t> bad{0};
  std::vector<std::thread> th;
  std::vector<uint32_t> first(n_threads, 0);
  std::vector<int> have(n_threads, 0);
  const uint64_t total = 1ull << 32;
  for (int k = 0; k < n_threads; k++)
    th.emplace_back([&, k] {
      uint64_t nb = 0;
      for (uint64_t u = k; u < total; u += n_threads) {
        float x;
        const uint32_t b = (uint32_t)u;
        memcpy(&x, &b, 4);
        const float a = expf(x), e = gkv::expf_cpu_exact(x);
        uint32_t ua, ue;
        memcpy(&ua, &a, 4);
        memcpy(&ue, &e, 4);
        if (ua != ue && !(std::isnan(a) && std::isnan(e))) {
          if (!have[k]) {
            have[k] = 1;
            first[k] = b;
          }
          nb++;
        }
      }
      bad += nb;
    });
  for (auto &t : th)
    t.join();
  printf("inputs %llu mismatches %llu\n", (unsigned long long)total,
         (unsigned long long)bad.load());
  for (int k = 0; k < n_threads; k++)
    if (have[k]) {
      float x;
      memcpy(&x, &first[k], 4);
      printf("  x = %a (0x%08x): libm %a, exact %a\n", x, first[k], expf(x),
             gkv::expf_cpu_exact(x));
    }
  return bad.load() == 0 ? 0 : 1;
}
