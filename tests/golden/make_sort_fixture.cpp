// Writes tests/golden/sort_ties_libstdcxx.json: the order in which this
// image's libstdc++ std::sort leaves elements whose keys compare equal.
// Stock XGBoost's weighted quantile sketch sorts each batch of (value,
// weight) entries with std::sort on the value alone (upstream
// WQSummary::Queue::MakeSummary) and then merges equal values in the sorted
// order, so the tie order decides which of +0/-0 represents a zero and the
// order in which the weights of equal values are added.  The reference's
// kernels/sketch_sort.metal.h restates libc++'s tie order for the same
// reason; this fixture pins the libstdc++ one (x86-64 builds).
//
//   g++ -O2 -std=c++17 -o make_sort_fixture make_sort_fixture.cpp
//   ./make_sort_fixture > sort_ties_libstdcxx.json
//
// Inputs: key classes from a 64-bit LCG (x = x * 6364136223846793005 +
// 1442695040888963407, class = (x >> 33) % k), or a fixed pattern; the sort
// compares classes only.  Output per case: the input element ids in sorted
// order -- all of them up to 257 elements, else the first 64 and a
// position-weighted checksum (sum of id[i] * (2i + 1) mod 2^64).
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <vector>

struct Entry {
  uint32_t key, id;
  bool operator<(const Entry& o) const { return key < o.key; }  // the value alone, as the sketch's entries
};

static std::vector<uint32_t> make_keys(const char* pattern, uint32_t n, uint32_t k, uint64_t seed) {
  std::vector<uint32_t> v(n);
  uint64_t x = seed;
  for (uint32_t i = 0; i < n; ++i) {
    x = x * 6364136223846793005ull + 1442695040888963407ull;
    const uint32_t r = (uint32_t)((x >> 33) % k);
    const char p = pattern[0];
    v[i] = p == 'r' ? r                                   // random classes
         : p == 'a' ? (uint32_t)((uint64_t)i * k / n)     // ascending runs of equal classes
         : p == 'd' ? (uint32_t)((uint64_t)(n - 1 - i) * k / n)  // descending
         : p == 'o' ? (uint32_t)(i < n / 2 ? i : n - 1 - i) % k  // organ pipe
         : (uint32_t)((i * 7919u) % k);                   // 's': strided classes
  }
  return v;
}

int main() {
  const char* patterns[] = {"r", "a", "d", "o", "s"};
  const uint32_t ns[] = {0, 1, 2, 3, 5, 15, 16, 17, 18, 31, 32, 33, 64, 100, 257, 1000, 4096, 7170, 20000};
  const uint32_t ks[] = {1, 2, 3, 7, 50, 1000, 1u << 30};
  const uint64_t seeds[] = {1, 12345};
  std::printf("{\"generator\": \"g++ %s, libstdc++ %d\",\n \"cases\": [\n", __VERSION__, __GLIBCXX__);
  bool first = true;
  for (const char* pattern : patterns) {
    for (uint32_t n : ns) {
      for (uint32_t k : ks) {
        for (uint64_t seed : seeds) {
          if (pattern[0] != 'r' && seed != seeds[0]) continue;  // patterns do not depend on the seed
          const std::vector<uint32_t> keys = make_keys(pattern, n, k, seed);
          std::vector<Entry> v(n);
          for (uint32_t i = 0; i < n; ++i) v[i] = Entry{keys[i], i};
          std::sort(v.begin(), v.end());
          uint64_t sum = 0;
          for (size_t i = 0; i < v.size(); ++i) sum += (uint64_t)v[i].id * (2 * (uint64_t)i + 1);
          const size_t shown = n <= 257 ? n : 64;
          std::printf("%s  {\"pattern\": \"%s\", \"n\": %u, \"k\": %u, \"seed\": %llu, \"checksum\": %llu, \"order\": [",
                      first ? "" : ",\n", pattern, n, k, (unsigned long long)seed, (unsigned long long)sum);
          for (size_t i = 0; i < shown; ++i) std::printf("%s%u", i ? "," : "", v[i].id);
          std::printf("]}");
          first = false;
        }
      }
    }
  }
  std::printf("\n ]}\n");
  return 0;
}
