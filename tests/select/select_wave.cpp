// Host check of the wave-parallel selection (dartkv_amd/csrc/dkv_select_wave.h) against
// libstdc++ and against the serial restatement (dkv_select.h).  Test infrastructure.
//
// The wave's 64 lanes run in a loop (HostWave); each step of the header reads before it writes
// across a sync(), so the loop gives what the lanes compute in parallel.  For random (rank, index)
// items with many ties the first k items must equal std::nth_element(k - 1) + std::sort(k - 1)
// (torch.topk(sorted=True) order on CPU).  Cases where the header hands back to the serial code
// (heap select, partial_sort) are counted, not compared.
// Prints "trials T mismatches M fallbacks F"; exit status 1 on any mismatch.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <utility>
#include <vector>

#include "dkv_select_wave.h"

using namespace dkv;

struct HostWave {
  template <class T>
  struct PerPos {
    T v[128];
    T& at(int x, int) { return v[x]; }
  };
  template <class F>
  void each(F fn) {
    for (int h = 0; h < 2; ++h)
      for (int lane = 0; lane < 64; ++lane) fn(lane + 64 * h, h);
  }
  template <class F>
  uint64_t ballot(F pred, int h) {
    uint64_t m = 0;
    for (int lane = 0; lane < 64; ++lane)
      if (pred(lane + 64 * h)) m |= 1ull << lane;
    return m;
  }
  bool first_lane() const { return true; }
  void sync() {}
};

int main(int argc, char** argv) {
  const int trials = argc > 1 ? std::atoi(argv[1]) : 50000;
  std::mt19937 rng(7u);
  long mismatches = 0, fallbacks = 0;
  auto before = [](const std::pair<float, int>& x, const std::pair<float, int>& y) {
    const bool xn = std::isnan(x.first), yn = std::isnan(y.first);
    return (xn && !yn) || x.first > y.first;
  };
  for (int t = 0; t < trials; ++t) {
    const int n = t % 3 == 0 ? 128 : 1 + (int)(rng() % 128);
    const int k = t % 5 == 0 ? std::min(n, 32) : 1 + (int)(rng() % n);
    const int mode = (int)(rng() % 4);
    std::vector<float> s(n);
    const int levels = 1 + (int)(rng() % (mode == 0 ? 3 : mode == 1 ? 12 : 60));
    for (auto& x : s) x = (float)(rng() % levels) * 0.25f;
    if (mode == 3) {  // presorted runs (ascending or descending), the adversarial inputs of quicksort
      if (rng() & 1) std::sort(s.begin(), s.end());
      else std::sort(s.begin(), s.end(), [](float a, float b) { return a > b; });
    }
    if (rng() % 10 == 0) s[rng() % n] = NAN;
    std::vector<std::pair<float, int>> ref(n);
    for (int j = 0; j < n; ++j) ref[j] = {s[j], j};
    if ((long)k * 64 <= n) {
      std::partial_sort(ref.begin(), ref.begin() + k, ref.end(), before);
    } else {
      std::nth_element(ref.begin(), ref.begin() + k - 1, ref.end(), before);
      std::sort(ref.begin(), ref.begin() + k - 1, before);
    }
    uint32_t a[128];
    uint8_t lpos[128], rpos[128];
    int stack[3 * kWaveSelStack];
    for (int j = 0; j < n; ++j) a[j] = (sel_rank(s[j], s.data(), n) << 7) | (uint32_t)j;
    HostWave w;
    const WaveSelBuffers buf{a, lpos, rpos, stack};
    if (!wsel_topk(buf, w, n, k)) {
      ++fallbacks;
      continue;
    }
    bool bad = false;
    for (int j = 0; j < k; ++j) bad |= (int)(a[j] & 127u) != ref[j].second;
    // the serial restatement on the same items
    std::vector<PackedItem> packed(n);
    for (int j = 0; j < n; ++j) packed[j].k = (sel_rank(s[j], s.data(), n) << 7) | (uint32_t)j;
    int st[3 * 16];
    sel_topk(n, k, PtrArray<PackedItem>{packed.data()}, PtrArray<int>{st}, 16);
    for (int j = 0; j < k; ++j) bad |= packed[j].k != a[j];
    if (bad && mismatches < 5) std::printf("mismatch: n %d k %d mode %d levels %d\n", n, k, mode, levels);
    mismatches += bad ? 1 : 0;
  }
  std::printf("trials %d mismatches %ld fallbacks %ld\n", trials, mismatches, fallbacks);
  return mismatches == 0 ? 0 : 1;
}
