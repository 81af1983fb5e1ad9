// TEST INFRASTRUCTURE ONLY (parity oracle).
//
// The real libstdc++ std::sort on (value, index) pairs with the comparator that
// torch.sort(descending=True) uses on CPU, so tests can pin the C emulation in
// oracle/coverage_ref.c (and the GPU kernel) against the genuine algorithm.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <utility>
#include <vector>

extern "C" void oracle_libstdcxx_sort_desc(float* v, int64_t* id, int64_t n) {
  std::vector<std::pair<float, int64_t>> a((size_t)n);
  for (int64_t i = 0; i < n; ++i) a[(size_t)i] = {v[i], id[i]};
  std::sort(a.begin(), a.end(), [](const std::pair<float, int64_t>& x, const std::pair<float, int64_t>& y) {
    return (std::isnan(x.first) && !std::isnan(y.first)) || (x.first > y.first);
  });
  for (int64_t i = 0; i < n; ++i) {
    v[i] = a[(size_t)i].first;
    id[i] = a[(size_t)i].second;
  }
}
