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
// fallback) as iterative code that runs on one GPU lane or on the host.  The CPU
// test suite checks it against std::nth_element / std::sort /
// std::partial_sort and against torch.topk.
#pragma once
#include <stdint.h>

#ifndef DKV_HD
#if defined(__HIPCC__)
#define DKV_HD __host__ __device__
#else
#define DKV_HD
#endif
#endif

namespace dkv {

struct SelItem {
  float v;
  int32_t i;
};

// "a ranks before b": larger value first; NaN ranks before any non-NaN value.
DKV_HD inline bool sel_before(const SelItem& a, const SelItem& b) {
  const bool an = a.v != a.v, bn = b.v != b.v;
  return (an && !bn) || (a.v > b.v);
}

template <class It>
DKV_HD inline void sel_swap(It a, SelItem* b) {
  SelItem t = *a;
  *a = *b;
  *b = t;
}

DKV_HD inline int sel_floor_log2(int n) {
  int r = 0;
  while (n > 1) {
    n >>= 1;
    ++r;
  }
  return r;
}

// ---- binary heap on [0, len) whose root is the element that ranks last ----

// Move `value` up from `hole` while its parent ranks before it.
template <class It>
DKV_HD inline void sel_heap_sift_up(It a, int hole, int top, SelItem value) {
  int parent = (hole - 1) / 2;
  while (hole > top && sel_before(a[parent], value)) {
    a[hole] = a[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  a[hole] = value;
}

// Fill the hole at `hole` by walking down along the child that ranks later,
// then sift `value` up from the leaf that was reached.
template <class It>
DKV_HD inline void sel_heap_adjust(It a, int hole, int len, SelItem value) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (sel_before(a[child], a[child - 1])) --child;
    a[hole] = a[child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    a[hole] = a[child - 1];
    hole = child - 1;
  }
  sel_heap_sift_up(a, hole, top, value);
}

template <class It>
DKV_HD inline void sel_make_heap(It a, int len) {
  if (len < 2) return;
  for (int parent = (len - 2) / 2;; --parent) {
    SelItem value = a[parent];
    sel_heap_adjust(a, parent, len, value);
    if (parent == 0) return;
  }
}

// Move the root of heap [0, len) to `*out` and re-heap with the old `*out`.
template <class It>
DKV_HD inline void sel_heap_pop_into(It a, int len, SelItem* out) {
  SelItem value = *out;
  *out = a[0];
  sel_heap_adjust(a, 0, len, value);
}

// Keep the `middle` best-ranked of [0, last) in a heap on [0, middle).
template <class It>
DKV_HD inline void sel_heap_select(It a, int middle, int last) {
  sel_make_heap(a, middle);
  for (int i = middle; i < last; ++i) {
    if (sel_before(a[i], a[0])) sel_heap_pop_into(a, middle, &a[i]);
  }
}

template <class It>
DKV_HD inline void sel_sort_heap(It a, int len) {
  while (len > 1) {
    --len;
    sel_heap_pop_into(a, len, &a[len]);
  }
}

// ---- insertion sorts ----

template <class It>
DKV_HD inline void sel_linear_insert_unguarded(It a, int pos) {
  SelItem value = a[pos];
  int prev = pos - 1;
  while (sel_before(value, a[prev])) {
    a[pos] = a[prev];
    pos = prev;
    --prev;
  }
  a[pos] = value;
}

template <class It>
DKV_HD inline void sel_insertion_sort(It a, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i < last; ++i) {
    if (sel_before(a[i], a[first])) {
      SelItem value = a[i];
      for (int j = i; j > first; --j) a[j] = a[j - 1];
      a[first] = value;
    } else {
      sel_linear_insert_unguarded(a, i);
    }
  }
}

// ---- partitioning ----

// Put the median (under sel_before) of a[x], a[y], a[z] into a[result].
template <class It>
DKV_HD inline void sel_median_to(It a, int result, int x, int y, int z) {
  if (sel_before(a[x], a[y])) {
    if (sel_before(a[y], a[z]))
      sel_swap(&a[result], &a[y]);
    else if (sel_before(a[x], a[z]))
      sel_swap(&a[result], &a[z]);
    else
      sel_swap(&a[result], &a[x]);
  } else if (sel_before(a[x], a[z])) {
    sel_swap(&a[result], &a[x]);
  } else if (sel_before(a[y], a[z])) {
    sel_swap(&a[result], &a[z]);
  } else {
    sel_swap(&a[result], &a[y]);
  }
}

// Hoare partition of [first, last) around a[pivot] (pivot lies outside the range).
template <class It>
DKV_HD inline int sel_partition_unguarded(It a, int first, int last, int pivot) {
  for (;;) {
    while (sel_before(a[first], a[pivot])) ++first;
    --last;
    while (sel_before(a[pivot], a[last])) --last;
    if (!(first < last)) return first;
    sel_swap(&a[first], &a[last]);
    ++first;
  }
}

template <class It>
DKV_HD inline int sel_partition_pivot(It a, int first, int last) {
  const int mid = first + (last - first) / 2;
  sel_median_to(a, first, first + 1, mid, last - 1);
  return sel_partition_unguarded(a, first + 1, last, first);
}

// ---- nth_element / sort / partial_sort ----

template <class It>
DKV_HD inline void sel_nth_element(It a, int first, int nth, int last) {
  if (first == last || nth == last) return;
  int depth = 2 * sel_floor_log2(last - first);
  while (last - first > 3) {
    if (depth == 0) {
      sel_heap_select(a + first, nth + 1 - first, last - first);
      sel_swap(&a[first], &a[nth]);
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

// `stack` holds 3 * cap ints (first, last, depth; an int pointer or any type
// with `stack[j]` -> int& and `stack + j`); cap >= 2 floor(log2(last - first)) + 1.
template <class It, class St>
DKV_HD inline void sel_sort(It a, int first, int last, St stack, int cap) {
  if (first == last) return;
  constexpr int kThreshold = 16;
  // Explicit stack replaces the right-hand recursion; the ranges it holds are
  // disjoint, so the processing order does not change the result.
  St st_first = stack;
  St st_last = stack + cap;
  St st_depth = stack + 2 * cap;
  int top = 0;
  st_first[0] = first;
  st_last[0] = last;
  st_depth[0] = 2 * sel_floor_log2(last - first);
  top = 1;
  while (top > 0) {
    --top;
    int f = st_first[top], l = st_last[top], depth = st_depth[top];
    while (l - f > kThreshold) {
      if (depth == 0) {
        sel_heap_select(a + f, l - f, l - f);
        sel_sort_heap(a + f, l - f);
        break;
      }
      --depth;
      const int cut = sel_partition_pivot(a, f, l);
      st_first[top] = cut;
      st_last[top] = l;
      st_depth[top] = depth;
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

template <class It>
DKV_HD inline void sel_partial_sort(It a, int middle, int last) {
  sel_heap_select(a, middle, last);
  sel_sort_heap(a, middle);
}

// Indices of the `k` best-ranked scores, in torch.topk(sorted=True) order.
// `work` holds n items of scratch (a SelItem pointer, or any type with
// `work[j]` -> SelItem& and `work + j`) and `stack` 3 * kSelStack ints (a
// caller on the GPU passes LDS, so the kernel needs no private memory).
// Requires 0 < k <= n.
// select_topk on a work array the caller has already filled with
// (score[j], j) for j < n.
template <class It, class St>
DKV_HD inline __attribute__((always_inline)) void select_topk_filled(int n, int k, It work, int32_t* out_idx,
                                                                     St stack, int cap = kSelStack) {
  if ((int64_t)k * 64 <= (int64_t)n) {
    sel_partial_sort(work, k, n);
  } else {
    sel_nth_element(work, 0, k - 1, n);
    sel_sort(work, 0, k - 1, stack, cap);
  }
  for (int j = 0; j < k; ++j) out_idx[j] = work[j].i;
}

template <class It, class St>
DKV_HD inline __attribute__((always_inline)) void select_topk(const float* score, int n, int k, It work,
                                                              int32_t* out_idx, St stack, int cap = kSelStack) {
  for (int j = 0; j < n; ++j) {
    work[j].v = score[j];
    work[j].i = j;
  }
  select_topk_filled(n, k, work, out_idx, stack, cap);
}

DKV_HD inline void select_topk(const float* score, int n, int k, SelItem* work, int32_t* out_idx) {
  int stack[3 * kSelStack];
  select_topk(score, n, k, work, out_idx, (int*)stack);
}

}  // namespace dkv
