// Writes tests/golden/shuffle_libstdcxx.json: permutations produced by this
// image's libstdc++ std::shuffle over std::mt19937(seed), the draws stock
// XGBoost's x86-64 build makes when it samples features (upstream
// ColumnSampler; the reference's src/tree.cpp:28-45 makes the same call).
//
//   g++ -O2 -std=c++17 -o make_shuffle_fixture make_shuffle_fixture.cpp
//   ./make_shuffle_fixture > shuffle_libstdcxx.json
//
// n <= 128 keep the whole permutation; larger n a position-weighted checksum
// (sum of perm[i] * (2i + 1) mod 2^64) and the first 64 entries.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <numeric>
#include <random>
#include <vector>

int main() {
  const unsigned long seeds[] = {0ul, 1ul, 7ul, 42ul, 2147483647ul, 3737844653ul};
  const unsigned ns[] = {1, 2, 3, 4, 5, 8, 13, 32, 64, 100, 101, 127, 128, 1000, 2000, 65535, 65536, 100000};
  std::printf("{\"generator\": \"g++ %s, libstdc++ %d\",\n \"cases\": [\n", __VERSION__, __GLIBCXX__);
  bool first = true;
  for (unsigned long seed : seeds) {
    for (unsigned n : ns) {
      std::vector<uint32_t> v(n);
      std::iota(v.begin(), v.end(), 0u);
      std::mt19937 rng(seed);
      std::shuffle(v.begin(), v.end(), rng);
      uint64_t sum = 0;
      for (size_t i = 0; i < v.size(); ++i) sum += (uint64_t)v[i] * (2 * (uint64_t)i + 1);
      const size_t shown = n <= 128 ? n : 64;
      std::printf("%s  {\"seed\": %lu, \"n\": %u, \"checksum\": %llu, \"next_draw\": %lu, \"head\": [", first ? "" : ",\n",
                  seed, n, (unsigned long long)sum, (unsigned long)rng());
      for (size_t i = 0; i < shown; ++i) std::printf("%s%u", i ? ", " : "", v[i]);
      std::printf("]}");
      first = false;
    }
  }
  std::printf("\n ]}\n");
  return 0;
}
