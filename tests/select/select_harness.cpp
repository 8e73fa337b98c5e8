// Host check of dartkv_amd/csrc/dkv_select.h against libstdc++ (test infrastructure).
//
// For random scores with many ties (and some NaNs), the k channels chosen and
// their order must equal what torch.topk(sorted=True) on CPU produces, i.e.
// libstdc++'s partial_sort (k * 64 <= n) or nth_element + sort (otherwise)
// over (score, index) pairs compared by score only, NaN first.  Both item
// forms are checked: (score, index) pairs in memory, and packed
// (rank << 7 | index) words (the form the GPU selection keeps in lanes).
// Prints "trials T mismatches M"; exit status 1 on any mismatch.
// With the argument "stdin": reads cases "n k s_0 .. s_{n-1}" and prints, per
// case, the selected indices from both item forms on one line each.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <random>
#include <string>
#include <utility>
#include <vector>

#include "dkv_select.h"

using namespace dkv;

static int run_stdin() {
  int n, k;
  while (std::scanf("%d %d", &n, &k) == 2) {
    std::vector<float> s(n);
    for (auto& x : s) {
      char buf[64];
      if (std::scanf("%63s", buf) != 1) return 2;
      x = std::strtof(buf, nullptr);
    }
    std::vector<SelItem> work(n);
    std::vector<int32_t> idx(k);
    select_topk(s.data(), n, k, work.data(), idx.data());
    for (int j = 0; j < k; ++j) std::printf("%d ", idx[j]);
    std::printf("\n");
    std::vector<PackedItem> packed(n);
    for (int j = 0; j < n; ++j) packed[j].k = (sel_rank(s[j], s.data(), n) << 7) | (uint32_t)j;
    int stack[3 * 16];
    sel_topk(n, k, PtrArray<PackedItem>{packed.data()}, PtrArray<int>{stack}, 16);
    for (int j = 0; j < k; ++j) std::printf("%d ", (int)(packed[j].k & 127u));
    std::printf("\n");
  }
  return 0;
}

int main(int argc, char** argv) {
  if (argc > 1 && std::string(argv[1]) == "stdin") return run_stdin();
  const int trials = argc > 1 ? std::atoi(argv[1]) : 20000;
  std::mt19937 rng(20260823u);
  long mismatches = 0;
  auto before = [](const std::pair<float, int>& x, const std::pair<float, int>& y) {
    const bool xn = std::isnan(x.first), yn = std::isnan(y.first);
    return (xn && !yn) || x.first > y.first;
  };
  for (int t = 0; t < trials; ++t) {
    const int n = 1 + (int)(rng() % (t % 2 ? 128 : 300));
    const int k = 1 + (int)(rng() % n);
    const int levels = 1 + (int)(rng() % 12);
    std::vector<float> s(n);
    for (auto& x : s) x = (float)(rng() % levels) * 0.25f;
    if (rng() % 8 == 0) s[rng() % n] = NAN;
    std::vector<std::pair<float, int>> ref(n);
    for (int j = 0; j < n; ++j) ref[j] = {s[j], j};
    if ((long)k * 64 <= n) {
      std::partial_sort(ref.begin(), ref.begin() + k, ref.end(), before);
    } else {
      std::nth_element(ref.begin(), ref.begin() + k - 1, ref.end(), before);
      std::sort(ref.begin(), ref.begin() + k - 1, before);
    }
    // (score, index) pairs
    std::vector<SelItem> work(n);
    std::vector<int32_t> idx(k);
    select_topk(s.data(), n, k, work.data(), idx.data());
    bool bad = false;
    for (int j = 0; j < k; ++j) bad |= idx[j] != ref[j].second;
    // packed (rank, index) words, n <= 128
    if (n <= 128) {
      std::vector<PackedItem> packed(n);
      for (int j = 0; j < n; ++j) packed[j].k = (sel_rank(s[j], s.data(), n) << 7) | (uint32_t)j;
      int stack[3 * 16];
      sel_topk(n, k, PtrArray<PackedItem>{packed.data()}, PtrArray<int>{stack}, 16);
      for (int j = 0; j < k; ++j) bad |= (int)(packed[j].k & 127u) != ref[j].second;
    }
    // a full sort (the introsort alone)
    std::vector<std::pair<float, int>> ref2(n);
    for (int j = 0; j < n; ++j) ref2[j] = {s[j], j};
    std::sort(ref2.begin(), ref2.end(), before);
    for (int j = 0; j < n; ++j) work[j] = SelItem{s[j], j};
    int stack2[3 * kSelStack];
    sel_sort(PtrArray<SelItem>{work.data()}, 0, n, PtrArray<int>{stack2}, kSelStack);
    for (int j = 0; j < n; ++j) bad |= work[j].i != ref2[j].second;
    mismatches += bad ? 1 : 0;
  }
  std::printf("trials %d mismatches %ld\n", trials, mismatches);
  return mismatches == 0 ? 0 : 1;
}
