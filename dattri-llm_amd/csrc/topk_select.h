// Top-k selection in the order torch.topk returns on the CPU.
//
// The router of transformers' MixtralTopKRouter.forward (installed
// transformers 5.15.0) is torch.topk(softmax(logits.float()), k).  On the CPU,
// ATen's topk_impl_loop (torch/include/ATen/native/TopKImpl.h) orders
// (probability, expert) pairs with "NaN first, then larger first" and
//   - for k * 64 <= n: std::partial_sort of the first k,
//   - otherwise:       std::nth_element at k - 1, then std::sort of the first
//                      k - 1 (k <= 16, so the insertion sort libstdc++ uses for
//                      ranges of at most 16 elements).
// Equal probabilities (tied logits, all-NaN rows) come out in whatever order
// those libstdc++ algorithms leave them, which is neither index order nor
// stable.  The routines below follow libstdc++'s published algorithms
// (introselect with a median-of-three pivot, binary-heap select and heap
// sort, insertion sort) step for step, so the indices agree with torch.topk
// bit for bit, ties included.
//
// Usable from device code (the router kernel) and from host code (the CPU
// check of this file).  A queue Q exposes get(i) / set(i, entry) / swap(i, j).
#pragma once

#if defined(__HIPCC__)
#define DA_TOPK_HD __host__ __device__ __forceinline__
#else
#define DA_TOPK_HD inline
#endif

namespace da {
namespace topk {

struct Entry {
  float p;  // probability
  int e;    // expert index
};

// Strict weak order "x is returned before y": NaN before any number, then
// larger first (ATen's comparator for largest = true).
DA_TOPK_HD bool before(const Entry& x, const Entry& y) {
  const bool xn = x.p != x.p, yn = y.p != y.p;
  return (xn && !yn) || x.p > y.p;
}

DA_TOPK_HD int floor_log2(int n) {
  int r = 0;
  while (n > 1) {
    n >>= 1;
    ++r;
  }
  return r;
}

// libstdc++ __insertion_sort on [lo, hi).
template <class Q>
DA_TOPK_HD void insertion_sort(Q& q, int lo, int hi) {
  if (lo == hi) return;
  for (int i = lo + 1; i < hi; ++i) {
    const Entry v = q.get(i);
    if (before(v, q.get(lo))) {
      for (int j = i; j > lo; --j) q.set(j, q.get(j - 1));
      q.set(lo, v);
    } else {  // q[lo] is not after v, so the walk stops at lo + 1 at the latest
      int j = i;
      while (j > lo + 1 && before(v, q.get(j - 1))) {
        q.set(j, q.get(j - 1));
        --j;
      }
      q.set(j, v);
    }
  }
}

// libstdc++ __move_median_to_first: the median of a, b, c swapped into r.
template <class Q>
DA_TOPK_HD void median_to_first(Q& q, int r, int a, int b, int c) {
  const Entry ea = q.get(a), eb = q.get(b), ec = q.get(c);
  int m;
  if (before(ea, eb)) {
    if (before(eb, ec)) m = b;
    else if (before(ea, ec)) m = c;
    else m = a;
  } else if (before(ea, ec)) {
    m = a;
  } else if (before(eb, ec)) {
    m = c;
  } else {
    m = b;
  }
  q.swap(r, m);
}

// libstdc++ __unguarded_partition of [first, last) around the entry at pivot
// (outside the range, so its value does not move).  The median-of-three
// pivot guarantees both scans stop inside the range; the bounds below only
// make that explicit.
template <class Q>
DA_TOPK_HD int unguarded_partition(Q& q, int first, int last, int pivot) {
  const Entry p = q.get(pivot);
  const int lo = first, hi = last;
  for (;;) {
    while (first < hi - 1 && before(q.get(first), p)) ++first;
    --last;
    while (last > lo && before(p, q.get(last))) --last;
    if (!(first < last)) return first;
    q.swap(first, last);
    ++first;
  }
}

// libstdc++ __adjust_heap + __push_heap (a max-heap under `before`, i.e. the
// root is the entry returned last).  Positions are relative to `first`.
template <class Q>
DA_TOPK_HD void adjust_heap(Q& q, int first, int hole, int len, Entry v) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (before(q.get(first + child), q.get(first + child - 1))) --child;
    q.set(first + hole, q.get(first + child));
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    q.set(first + hole, q.get(first + child - 1));
    hole = child - 1;
  }
  while (hole > top) {
    const int parent = (hole - 1) / 2;
    if (!before(q.get(first + parent), v)) break;
    q.set(first + hole, q.get(first + parent));
    hole = parent;
  }
  q.set(first + hole, v);
}

template <class Q>
DA_TOPK_HD void make_heap(Q& q, int first, int last) {
  const int len = last - first;
  if (len < 2) return;
  for (int parent = (len - 2) / 2;; --parent) {
    adjust_heap(q, first, parent, len, q.get(first + parent));
    if (parent == 0) return;
  }
}

template <class Q>
DA_TOPK_HD void pop_heap(Q& q, int first, int last, int result) {
  const Entry v = q.get(result);
  q.set(result, q.get(first));
  adjust_heap(q, first, 0, last - first, v);
}

// libstdc++ __heap_select: [first, middle) ends up holding the entries that
// come first, as a heap.
template <class Q>
DA_TOPK_HD void heap_select(Q& q, int first, int middle, int last) {
  make_heap(q, first, middle);
  for (int i = middle; i < last; ++i)
    if (before(q.get(i), q.get(first))) pop_heap(q, first, middle, i);
}

template <class Q>
DA_TOPK_HD void sort_heap(Q& q, int first, int last) {
  while (last - first > 1) {
    --last;
    pop_heap(q, first, last, last);
  }
}

// libstdc++ std::nth_element (__introselect, depth limit 2 * floor(log2 n)).
template <class Q>
DA_TOPK_HD void nth_element(Q& q, int nth, int n) {
  if (n == 0 || nth == n) return;
  int first = 0, last = n, depth = 2 * floor_log2(n);
  while (last - first > 3) {
    if (depth == 0) {
      heap_select(q, first, nth + 1, last);
      q.swap(first, nth);
      return;
    }
    --depth;
    median_to_first(q, first, first + 1, first + (last - first) / 2, last - 1);
    const int cut = unguarded_partition(q, first + 1, last, first);
    if (cut <= nth) first = cut;
    else last = cut;
  }
  insertion_sort(q, first, last);
}

// The first k entries of q (n of them, entry i = (p_i, i) on entry) in
// torch.topk's CPU order, 1 <= k <= min(n, 16).
template <class Q>
DA_TOPK_HD void select_topk(Q& q, int n, int k) {
  if (k * 64 <= n) {
    heap_select(q, 0, k, n);  // std::partial_sort
    sort_heap(q, 0, k);
  } else {
    nth_element(q, k - 1, n);
    insertion_sort(q, 0, k - 1);  // std::sort of <= 15 entries
  }
}

}  // namespace topk
}  // namespace da
