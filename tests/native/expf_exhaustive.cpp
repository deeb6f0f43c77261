// Exhaustive check of csrc/libm_ref.h's expf_ref against the host's expf:
// every one of the 2^32 float bit patterns, compared bit for bit (NaNs by
// class). Prints "inputs N mismatches M first 0x........" and exits 0 when
// M == 0. Built and run by tests/test_libm_ref.py.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#define MI_LIBM_HD
#include "libm_ref.h"

int main(int argc, char** argv) {
  const int nth = argc > 1 ? atoi(argv[1]) : 8;
  static const uint64_t tab[32] = MI_EXPF_TABLE;
  std::vector<unsigned long long> bad(nth, 0);
  std::vector<uint32_t> first(nth, 0);
  std::vector<std::thread> th;
  for (int w = 0; w < nth; ++w)
    th.emplace_back([&, w] {
      for (uint64_t u = (uint64_t)w; u < (1ULL << 32); u += (uint64_t)nth) {
        const uint32_t ui = (uint32_t)u;
        float x;
        std::memcpy(&x, &ui, 4);
        const float want = expf(x), got = mi::expf_ref(x, tab);
        uint32_t a, b;
        std::memcpy(&a, &want, 4);
        std::memcpy(&b, &got, 4);
        const bool same = a == b || (std::isnan(want) && std::isnan(got));
        if (!same && bad[w]++ == 0) first[w] = ui;
      }
    });
  for (auto& t : th) t.join();
  unsigned long long total = 0;
  uint32_t f = 0;
  for (int w = 0; w < nth; ++w) {
    if (bad[w] && !total) f = first[w];
    total += bad[w];
  }
  std::printf("inputs 4294967296 mismatches %llu first 0x%08x\n", total, f);
  return total == 0 ? 0 : 1;
}
