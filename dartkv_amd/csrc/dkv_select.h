// Promoted-channel selection that reproduces torch.topk(largest=True, sorted=True)
// on CPU bit-for-bit, including the order of tied scores.
//
// The reference selects channels with `score.topk(count, dim=-1, sorted=True)`
// (reference src/dart/mixed.py:155-156 and :160-161).  ATen's CPU top-k builds
// (value, index) pairs in index order and, when k*64 > n, runs libstdc++
// nth_element(first, first+k-1, last) followed by sort(first, first+k-1);
// otherwise partial_sort(first, first+k, last).  The comparator is
// "x.value > y.value" (NaN first) and never looks at the index, so tied values
// end up in whatever order the selection algorithm's swaps leave them.  Tied
// bf16 scores are common, so the stored channel order depends on those exact
// steps.
//
// This file restates the published introselect / introsort / heap-select
// algorithms (median-of-three pivot moved to the front, unguarded Hoare
// partition, insertion-sort threshold 16, depth limit 2*floor(log2 n), heap
// fallback) as iterative code over an abstract array: `a.get(i)`, `a.set(i, x)`
// and `a.shifted(d)` (the array starting at element d).  The steps only ever
// compare items with sel_before, so the same code runs on (score, index) pairs
// and on packed (rank, index) words: the rank of a score among the page's
// scores orders and ties exactly like the score itself.  The GPU kernels use
// the pairs in LDS.  tests/test_select_order.py checks both item forms against
// libstdc++'s std::nth_element / std::sort / std::partial_sort and against
// torch.topk on the host.
#pragma once
#include <stdint.h>

#ifndef DKV_HD
#if defined(__HIPCC__)
#define DKV_HD __host__ __device__
#else
#define DKV_HD
#endif
#endif
// Every step is inlined into its caller (the GPU kernels run it on LDS arrays).
#define DKV_SEL DKV_HD inline __attribute__((always_inline))

namespace dkv {

struct SelItem {
  float v;
  int32_t i;
};

// A score's rank among the page's scores (bits 14..7) and its index (bits 6..0).
struct PackedItem {
  uint32_t k;
};

// "a ranks before b": larger value first; NaN ranks before any non-NaN value.
DKV_SEL bool sel_before(const SelItem& a, const SelItem& b) {
  const bool an = a.v != a.v, bn = b.v != b.v;
  return (an && !bn) || (a.v > b.v);
}
DKV_SEL bool sel_before(const PackedItem& a, const PackedItem& b) { return (a.k >> 7) > (b.k >> 7); }

// Order-preserving rank of score v among scores s[0..n): the number of scores
// below v, and 255 for NaN (NaN ranks first).  Equal scores get equal ranks.
DKV_SEL uint32_t sel_rank(float v, const float* s, int n) {
  if (v != v) return 255u;
  uint32_t r = 0;
  for (int j = 0; j < n; ++j) r += s[j] < v ? 1u : 0u;
  return r;
}

// Plain memory (host arrays, LDS, private arrays).
template <class T>
struct PtrArray {
  T* p;
  DKV_HD T get(int i) const { return p[i]; }
  DKV_HD void set(int i, const T& x) const { p[i] = x; }
  DKV_HD PtrArray shifted(int d) const { return PtrArray{p + d}; }
};

template <class A>
DKV_SEL void sel_swap(A a, int x, int y) {
  const auto t = a.get(x);
  a.set(x, a.get(y));
  a.set(y, t);
}

DKV_SEL int sel_floor_log2(int n) {
  int r = 0;
  while (n > 1) {
    n >>= 1;
    ++r;
  }
  return r;
}

// ---- binary heap on [0, len) whose root is the element that ranks last ----

// Move `value` up from `hole` while its parent ranks before it.
template <class A, class T>
DKV_SEL void sel_heap_sift_up(A a, int hole, int top, T value) {
  int parent = (hole - 1) / 2;
  while (hole > top && sel_before(a.get(parent), value)) {
    a.set(hole, a.get(parent));
    hole = parent;
    parent = (hole - 1) / 2;
  }
  a.set(hole, value);
}

// Fill the hole at `hole` by walking down along the child that ranks later,
// then sift `value` up from the leaf that was reached.
template <class A, class T>
DKV_SEL void sel_heap_adjust(A a, int hole, int len, T value) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (sel_before(a.get(child), a.get(child - 1))) --child;
    a.set(hole, a.get(child));
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    a.set(hole, a.get(child - 1));
    hole = child - 1;
  }
  sel_heap_sift_up(a, hole, top, value);
}

template <class A>
DKV_SEL void sel_make_heap(A a, int len) {
  if (len < 2) return;
  for (int parent = (len - 2) / 2;; --parent) {
    sel_heap_adjust(a, parent, len, a.get(parent));
    if (parent == 0) return;
  }
}

// Move the root of heap [0, len) to element `out` and re-heap with the old
// value of `out`.
template <class A>
DKV_SEL void sel_heap_pop_into(A a, int len, int out) {
  const auto value = a.get(out);
  a.set(out, a.get(0));
  sel_heap_adjust(a, 0, len, value);
}

// Keep the `middle` best-ranked of [0, last) in a heap on [0, middle).
template <class A>
DKV_SEL void sel_heap_select(A a, int middle, int last) {
  sel_make_heap(a, middle);
  for (int i = middle; i < last; ++i) {
    if (sel_before(a.get(i), a.get(0))) sel_heap_pop_into(a, middle, i);
  }
}

template <class A>
DKV_SEL void sel_sort_heap(A a, int len) {
  while (len > 1) {
    --len;
    sel_heap_pop_into(a, len, len);
  }
}

// ---- insertion sorts ----

template <class A>
DKV_SEL void sel_linear_insert_unguarded(A a, int pos) {
  const auto value = a.get(pos);
  int prev = pos - 1;
  while (sel_before(value, a.get(prev))) {
    a.set(pos, a.get(prev));
    pos = prev;
    --prev;
  }
  a.set(pos, value);
}

template <class A>
DKV_SEL void sel_insertion_sort(A a, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i < last; ++i) {
    if (sel_before(a.get(i), a.get(first))) {
      const auto value = a.get(i);
      for (int j = i; j > first; --j) a.set(j, a.get(j - 1));
      a.set(first, value);
    } else {
      sel_linear_insert_unguarded(a, i);
    }
  }
}

// ---- partitioning ----

// Put the median (under sel_before) of a[x], a[y], a[z] into a[result].
template <class A>
DKV_SEL void sel_median_to(A a, int result, int x, int y, int z) {
  if (sel_before(a.get(x), a.get(y))) {
    if (sel_before(a.get(y), a.get(z)))
      sel_swap(a, result, y);
    else if (sel_before(a.get(x), a.get(z)))
      sel_swap(a, result, z);
    else
      sel_swap(a, result, x);
  } else if (sel_before(a.get(x), a.get(z))) {
    sel_swap(a, result, x);
  } else if (sel_before(a.get(y), a.get(z))) {
    sel_swap(a, result, z);
  } else {
    sel_swap(a, result, y);
  }
}

// Hoare partition of [first, last) around a[pivot] (pivot lies outside the range).
template <class A>
DKV_SEL int sel_partition_unguarded(A a, int first, int last, int pivot) {
  for (;;) {
    while (sel_before(a.get(first), a.get(pivot))) ++first;
    --last;
    while (sel_before(a.get(pivot), a.get(last))) --last;
    if (!(first < last)) return first;
    sel_swap(a, first, last);
    ++first;
  }
}

template <class A>
DKV_SEL int sel_partition_pivot(A a, int first, int last) {
  const int mid = first + (last - first) / 2;
  sel_median_to(a, first, first + 1, mid, last - 1);
  return sel_partition_unguarded(a, first + 1, last, first);
}

// ---- nth_element / sort / partial_sort ----

template <class A>
DKV_SEL void sel_nth_element(A a, int first, int nth, int last) {
  if (first == last || nth == last) return;
  int depth = 2 * sel_floor_log2(last - first);
  while (last - first > 3) {
    if (depth == 0) {
      sel_heap_select(a.shifted(first), nth + 1 - first, last - first);
      sel_swap(a, first, nth);
      return;
    }
    --depth;
    const int cut = sel_partition_pivot(a, first, last);
    if (cut <= nth)
      first = cut;
    else
      last = cut;
  }
  sel_insertion_sort(a, first, last);
}

// Explicit stack for sel_sort's right-hand ranges: it never holds more than
// 2 floor(log2(n)) + 1 entries (one per depth level).
constexpr int kSelStack = 64;

// `stack` is an int array of 3 * cap elements (first, last, depth);
// cap >= 2 floor(log2(last - first)) + 1.
template <class A, class S>
DKV_SEL void sel_sort(A a, int first, int last, S stack, int cap) {
  if (first == last) return;
  constexpr int kThreshold = 16;
  // Explicit stack replaces the right-hand recursion; the ranges it holds are
  // disjoint, so the processing order does not change the result.
  stack.set(0, first);
  stack.set(cap, last);
  stack.set(2 * cap, 2 * sel_floor_log2(last - first));
  int top = 1;
  while (top > 0) {
    --top;
    int f = stack.get(top), l = stack.get(cap + top), depth = stack.get(2 * cap + top);
    while (l - f > kThreshold) {
      if (depth == 0) {
        sel_heap_select(a.shifted(f), l - f, l - f);
        sel_sort_heap(a.shifted(f), l - f);
        break;
      }
      --depth;
      const int cut = sel_partition_pivot(a, f, l);
      stack.set(top, cut);
      stack.set(cap + top, l);
      stack.set(2 * cap + top, depth);
      ++top;
      l = cut;
    }
  }
  if (last - first > kThreshold) {
    sel_insertion_sort(a, first, first + kThreshold);
    for (int i = first + kThreshold; i < last; ++i) sel_linear_insert_unguarded(a, i);
  } else {
    sel_insertion_sort(a, first, last);
  }
}

template <class A>
DKV_SEL void sel_partial_sort(A a, int middle, int last) {
  sel_heap_select(a, middle, last);
  sel_sort_heap(a, middle);
}

// Leave the k best-ranked of the n items of `work` in its first k elements,
// in torch.topk(sorted=True) order.  Requires 0 < k <= n.
template <class A, class S>
DKV_SEL void sel_topk(int n, int k, A work, S stack, int cap) {
  if ((int64_t)k * 64 <= (int64_t)n) {
    sel_partial_sort(work, k, n);
  } else {
    sel_nth_element(work, 0, k - 1, n);
    sel_sort(work, 0, k - 1, stack, cap);
  }
}

// Indices of the `k` best-ranked scores, in torch.topk(sorted=True) order.
// `work` holds n (score[j], j) items already filled in; `stack` 3 * cap ints.
// (A caller on the GPU passes LDS, so the kernel needs no private memory.)
template <class It, class St>
DKV_SEL void select_topk_filled(int n, int k, It work, int32_t* out_idx, St stack, int cap = kSelStack) {
  const PtrArray<SelItem> w{&work[0]};
  sel_topk(n, k, w, PtrArray<int>{&stack[0]}, cap);
  for (int j = 0; j < k; ++j) out_idx[j] = w.get(j).i;
}

template <class It, class St>
DKV_SEL void select_topk(const float* score, int n, int k, It work, int32_t* out_idx, St stack,
                         int cap = kSelStack) {
  for (int j = 0; j < n; ++j) {
    work[j].v = score[j];
    work[j].i = j;
  }
  select_topk_filled(n, k, work, out_idx, stack, cap);
}

DKV_SEL void select_topk(const float* score, int n, int k, SelItem* work, int32_t* out_idx) {
  int stack[3 * kSelStack];
  select_topk(score, n, k, work, out_idx, (int*)stack);
}

}  // namespace dkv
