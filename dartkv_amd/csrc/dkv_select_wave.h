// Wave-parallel form of the promoted-channel selection in dkv_select.h: the same
// result as sel_topk (torch.topk(largest=True, sorted=True) order on CPU, ties
// included) for up to 128 packed (rank, index) items, computed by one wave64.
//
// sel_topk runs libstdc++'s nth_element(k - 1) and then sort(first k - 1) on the
// items.  Both are made of two kinds of steps, and each kind has a closed form
// that a wave evaluates with a few ballots, prefix counts and LDS scatters
// instead of one item access per step on one lane:
//
// * Hoare partition of [f, l) around pivot p (sel_partition_unguarded).  Let
//   l_1 < l_2 < ... be the positions in [f, l) whose item does not rank before
//   p, and r_1 > r_2 > ... those whose item does not rank after p.  The left
//   scan stops exactly at the l_i and the right scan at the r_i (a position
//   already swapped holds an item that stops the other scan, and it lies beyond
//   the next original stopper), so the partition swaps item l_i with item r_i
//   for i = 1..m, where m counts the i with l_i < r_i (true for a prefix of i),
//   and returns min(l_{m+1}, r_m) (a missing term is +infinity).  The
//   median-of-three pivot move before it is a few uniform compares.
// * Insertion sort of a range (the end of nth_element and of sort): it only
//   moves an item past items it strictly ranks before, so its result is the
//   stable sort of the range's current arrangement: the item at x lands at
//   (items of the range ranking before it) + (equal items earlier than x).
//
// The loops that choose the ranges (introselect, introsort with its stack of
// right-hand ranges) are the scalar control of dkv_select.h.  When libstdc++
// would switch to heap select (a depth limit) or use partial_sort (small k),
// wsel_topk returns false and the caller runs sel_topk on fresh items.
//
// The steps are written against a lane model: `each(fn)` runs fn(x, h) for the
// positions x = lane + 64 h (h = 0, 1) a lane owns, `ballot(pred, h)` gathers
// pred(lane + 64 h) over the lanes, `sync()` orders the LDS traffic of the
// wave, and PerPos<T> is a lane's private value per position.  The device
// model is one real wave (dkv::DeviceWave in quantize.hip); the host model
// (tests/select/select_wave.cpp) runs the 64 lanes in a loop and is checked
// against libstdc++ by tests/test_select_order.py.
#pragma once
#include <stdint.h>

#include "dkv_select.h"

namespace dkv {

constexpr int kWaveSelStack = 16;

// Selection arrays (LDS on the device).
struct WaveSelBuffers {
  uint32_t* a;    // [128] packed items (rank << 7 | index)
  uint8_t* lpos;  // [128] left stoppers in scan order
  uint8_t* rpos;  // [128] right stoppers in scan order
  int* stack;     // [3 * kWaveSelStack] sort ranges (first, last, depth)
};

DKV_SEL uint32_t wsel_rank(uint32_t w) { return w >> 7; }
DKV_SEL int wsel_popc(uint64_t x) { return __builtin_popcountll(x); }

template <class W>
DKV_SEL void wsel_median_to(const WaveSelBuffers& s, W& w, int result, int x, int y, int z) {
  // every lane reads the same items and takes the same branch (sel_median_to)
  const PtrArray<PackedItem> a{(PackedItem*)s.a};
  int pick;
  if (sel_before(a.get(x), a.get(y))) {
    if (sel_before(a.get(y), a.get(z))) pick = y;
    else if (sel_before(a.get(x), a.get(z))) pick = z;
    else pick = x;
  } else if (sel_before(a.get(x), a.get(z))) {
    pick = x;
  } else if (sel_before(a.get(y), a.get(z))) {
    pick = z;
  } else {
    pick = y;
  }
  const uint32_t at_result = s.a[result], at_pick = s.a[pick];
  w.sync();
  if (w.first_lane()) {
    s.a[result] = at_pick;
    s.a[pick] = at_result;
  }
  w.sync();
}

// sel_partition_unguarded(a, f, l, piv) in closed form; returns the cut.
template <class W>
DKV_SEL int wsel_partition(const WaveSelBuffers& s, W& w, int f, int l, int piv) {
  const uint32_t pr = wsel_rank(s.a[piv]);
  uint64_t mL[2], mR[2];
  for (int h = 0; h < 2; ++h) {
    mL[h] = w.ballot([&](int x) { return x >= f && x < l && wsel_rank(s.a[x]) <= pr; }, h);
    mR[h] = w.ballot([&](int x) { return x >= f && x < l && wsel_rank(s.a[x]) >= pr; }, h);
  }
  const int nL = wsel_popc(mL[0]) + wsel_popc(mL[1]);
  const int nR = wsel_popc(mR[0]) + wsel_popc(mR[1]);
  w.each([&](int x, int h) {
    const int lane = x & 63;
    if ((mL[h] >> lane) & 1ull)  // its order among the left stoppers, from the left
      s.lpos[(h ? wsel_popc(mL[0]) : 0) + wsel_popc(mL[h] & ((2ull << lane) - 1ull)) - 1] = (uint8_t)x;
    if ((mR[h] >> lane) & 1ull)  // among the right stoppers, from the right
      s.rpos[(h ? 0 : wsel_popc(mR[1])) + wsel_popc(mR[h] & ~((1ull << lane) - 1ull)) - 1] = (uint8_t)x;
  });
  w.sync();
  const int pairs = nL < nR ? nL : nR;
  uint64_t crossed[2];
  for (int h = 0; h < 2; ++h) crossed[h] = w.ballot([&](int j) { return j < pairs && s.lpos[j] < s.rpos[j]; }, h);
  const int m = wsel_popc(crossed[0]) + wsel_popc(crossed[1]);
  // swap item l_j with item r_j for j < m: every read before any write
  typename W::template PerPos<uint32_t> u, v;
  w.each([&](int j, int h) {
    if (j < m) {
      u.at(j, h) = s.a[s.lpos[j]];
      v.at(j, h) = s.a[s.rpos[j]];
    }
  });
  w.sync();
  w.each([&](int j, int h) {
    if (j < m) {
      s.a[s.lpos[j]] = v.at(j, h);
      s.a[s.rpos[j]] = u.at(j, h);
    }
  });
  const int left = m < nL ? (int)s.lpos[m] : 1 << 20;
  const int right = m >= 1 ? (int)s.rpos[m - 1] : 1 << 20;
  w.sync();
  return left < right ? left : right;
}

template <class W>
DKV_SEL int wsel_partition_pivot(const WaveSelBuffers& s, W& w, int f, int l) {
  const int mid = f + (l - f) / 2;
  wsel_median_to(s, w, f, f + 1, mid, l - 1);
  return wsel_partition(s, w, f + 1, l, f);
}

// Insertion sort of [f, l), i.e. the stable sort of its current arrangement.
template <class W>
DKV_SEL void wsel_stable_sort(const WaveSelBuffers& s, W& w, int f, int l) {
  if (l - f < 2) return;
  typename W::template PerPos<int> dest;
  typename W::template PerPos<uint32_t> item;
  w.each([&](int x, int h) {
    dest.at(x, h) = -1;
    if (x >= f && x < l) {
      const uint32_t r = wsel_rank(s.a[x]);
      int d = f;
      for (int y = f; y < l; ++y) {
        const uint32_t ry = wsel_rank(s.a[y]);
        d += (ry > r) || (ry == r && y < x);
      }
      dest.at(x, h) = d;
      item.at(x, h) = s.a[x];
    }
  });
  w.sync();
  w.each([&](int x, int h) {
    if (dest.at(x, h) >= 0) s.a[dest.at(x, h)] = item.at(x, h);
  });
  w.sync();
}

// sel_topk(n, k) on the n <= 128 items of s.a.  Returns false, with the items
// partly permuted, where libstdc++ would take heap select or partial_sort.
template <class W>
DKV_SEL bool wsel_topk(const WaveSelBuffers& s, W& w, int n, int k) {
  if (n > 128 || k < 1 || k > n || (int64_t)k * 64 <= (int64_t)n) return false;
  // nth_element(0, k - 1, n)
  if (k - 1 != n) {
    int f = 0, l = n, depth = 2 * sel_floor_log2(n);
    while (l - f > 3) {
      if (depth == 0) return false;
      --depth;
      const int cut = wsel_partition_pivot(s, w, f, l);
      if (cut <= k - 1) f = cut;
      else l = cut;
    }
    wsel_stable_sort(s, w, f, l);
  }
  // sort(0, k - 1): partition ranges longer than 16, then one insertion sort
  const int last = k - 1;
  if (last > 0) {
    constexpr int kThreshold = 16;
    if (w.first_lane()) {
      s.stack[0] = 0;
      s.stack[kWaveSelStack] = last;
      s.stack[2 * kWaveSelStack] = 2 * sel_floor_log2(last);
    }
    w.sync();
    int top = 1;
    while (top > 0) {
      --top;
      const int f = s.stack[top];
      int l = s.stack[kWaveSelStack + top], depth = s.stack[2 * kWaveSelStack + top];
      w.sync();
      while (l - f > kThreshold) {
        if (depth == 0 || top >= kWaveSelStack) return false;
        --depth;
        const int cut = wsel_partition_pivot(s, w, f, l);
        if (w.first_lane()) {
          s.stack[top] = cut;
          s.stack[kWaveSelStack + top] = l;
          s.stack[2 * kWaveSelStack + top] = depth;
        }
        w.sync();
        ++top;
        l = cut;
      }
    }
    wsel_stable_sort(s, w, 0, last);
  }
  return true;
}

}  // namespace dkv
