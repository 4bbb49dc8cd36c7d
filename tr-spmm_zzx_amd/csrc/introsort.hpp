// std::sort as libstdc++ implements it, restated for device code.
//
// The format builder orders a window's 2:4 units with std::sort under a comparator that is not a
// total order (TR-source/Block/block_online.cpp:358-363: degree desc, then nnz desc, over unit
// indices), so which of two tied units comes first is decided by the steps of the library's
// introsort, and the 2:4 group order of every output array follows from it.  A device builder
// must therefore take exactly those steps.  This header restates them from libstdc++'s
// <bits/stl_algo.h> / <bits/stl_heap.h> (the algorithm GCC has shipped unchanged since GCC 4.x):
//
//   sort(first, last):       if non-empty, introsort_loop(first, last, 2 * floor(log2(n)))
//                            then final_insertion_sort(first, last)
//   introsort_loop:          while more than 16 elements: at depth 0 heap-sort the range and
//                            stop; else depth - 1, cut = partition around the median of
//                            (first + 1, middle, last - 1) moved to first, recurse on
//                            [cut, last), continue with [first, cut)
//   unguarded_partition:     Hoare scan from first + 1 and last - 1 against the pivot at
//                            first, swapping pairs that stop both scans, until they cross
//   final_insertion_sort:    guarded insertion sort of the first 16 elements, unguarded
//                            insertion of the rest
//   heap sort:               make_heap (adjust_heap from the last parent down) then sort_heap
//                            (pop_heap of the root to the back, repeatedly)
//
// Functions are templates over the element type and a comparator comp(a, b) = "a before b";
// every comparison and every move happens in the library's order, so equal elements end where
// the library puts them.  `TRS_HD` makes them callable from host and device code.
#pragma once
#include <cstdint>

#if defined(__HIPCC__)
#define TRS_HD __host__ __device__
#else
#define TRS_HD
#endif

namespace trs {
namespace isort {

constexpr int64_t kThreshold = 16;   // libstdc++ _S_threshold

TRS_HD inline int lg(int64_t n) {   // floor(log2(n)), n > 0 (std::__lg)
  int r = 0;
  while (n > 1) {
    n >>= 1;
    ++r;
  }
  return r;
}

template <class T>
TRS_HD inline void swap_at(T* a, T* b) {
  T t = *a;
  *a = *b;
  *b = t;
}

// std::__move_median_to_first
template <class T, class Cmp>
TRS_HD void move_median_to_first(T* result, T* a, T* b, T* c, Cmp& comp) {
  if (comp(*a, *b)) {
    if (comp(*b, *c)) swap_at(result, b);
    else if (comp(*a, *c)) swap_at(result, c);
    else swap_at(result, a);
  } else if (comp(*a, *c)) {
    swap_at(result, a);
  } else if (comp(*b, *c)) {
    swap_at(result, c);
  } else {
    swap_at(result, b);
  }
}

// std::__unguarded_partition: [first, last) against *pivot
template <class T, class Cmp>
TRS_HD T* unguarded_partition(T* first, T* last, T* pivot, Cmp& comp) {
  while (true) {
    while (comp(*first, *pivot)) ++first;
    --last;
    while (comp(*pivot, *last)) --last;
    if (!(first < last)) return first;
    swap_at(first, last);
    ++first;
  }
}

// std::__unguarded_partition_pivot
template <class T, class Cmp>
TRS_HD T* partition_pivot(T* first, T* last, Cmp& comp) {
  T* mid = first + (last - first) / 2;
  move_median_to_first(first, first + 1, mid, last - 1, comp);
  return unguarded_partition(first + 1, last, first, comp);
}

// std::__push_heap
template <class T, class Cmp>
TRS_HD void push_heap(T* first, int64_t hole, int64_t top, T value, Cmp& comp) {
  int64_t parent = (hole - 1) / 2;
  while (hole > top && comp(first[parent], value)) {
    first[hole] = first[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  first[hole] = value;
}

// std::__adjust_heap
template <class T, class Cmp>
TRS_HD void adjust_heap(T* first, int64_t hole, int64_t len, T value, Cmp& comp) {
  const int64_t top = hole;
  int64_t child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (comp(first[child], first[child - 1])) child--;
    first[hole] = first[child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    first[hole] = first[child - 1];
    hole = child - 1;
  }
  push_heap(first, hole, top, value, comp);
}

// std::__make_heap
template <class T, class Cmp>
TRS_HD void make_heap(T* first, T* last, Cmp& comp) {
  const int64_t len = last - first;
  if (len < 2) return;
  int64_t parent = (len - 2) / 2;
  while (true) {
    T value = first[parent];
    adjust_heap(first, parent, len, value, comp);
    if (parent == 0) return;
    parent--;
  }
}

// std::__sort_heap (each step is std::__pop_heap(first, last - 1, last - 1))
template <class T, class Cmp>
TRS_HD void sort_heap(T* first, T* last, Cmp& comp) {
  while (last - first > 1) {
    --last;
    T value = *last;
    *last = *first;
    adjust_heap(first, (int64_t)0, (int64_t)(last - first), value, comp);
  }
}

// std::__partial_sort(first, last, last): heap select over an empty tail, then sort_heap
template <class T, class Cmp>
TRS_HD void heap_sort(T* first, T* last, Cmp& comp) {
  make_heap(first, last, comp);
  sort_heap(first, last, comp);
}

// std::__unguarded_linear_insert
template <class T, class Cmp>
TRS_HD void unguarded_linear_insert(T* last, Cmp& comp) {
  T val = *last;
  T* next = last - 1;
  while (comp(val, *next)) {
    *last = *next;
    last = next;
    --next;
  }
  *last = val;
}

// std::__insertion_sort
template <class T, class Cmp>
TRS_HD void insertion_sort(T* first, T* last, Cmp& comp) {
  if (first == last) return;
  for (T* i = first + 1; i != last; ++i) {
    if (comp(*i, *first)) {
      T val = *i;
      for (T* j = i; j != first; --j) *j = *(j - 1);   // move_backward(first, i, i + 1)
      *first = val;
    } else {
      unguarded_linear_insert(i, comp);
    }
  }
}

// std::__final_insertion_sort
template <class T, class Cmp>
TRS_HD void final_insertion_sort(T* first, T* last, Cmp& comp) {
  if (last - first > kThreshold) {
    insertion_sort(first, first + kThreshold, comp);
    for (T* i = first + kThreshold; i != last; ++i) unguarded_linear_insert(i, comp);
  } else {
    insertion_sort(first, last, comp);
  }
}

// std::__introsort_loop with the recursion on [cut, last) kept on an explicit stack (the ranges it
// leaves are disjoint, so the order in which they are finished does not change the result).
template <class T, class Cmp>
TRS_HD void introsort_loop(T* first, T* last, int depth, Cmp& comp) {
  struct Range { T* first; T* last; int depth; };
  Range stack[128];
  int top = 0;
  stack[top++] = Range{first, last, depth};
  while (top > 0) {
    Range r = stack[--top];
    while (r.last - r.first > kThreshold) {
      if (r.depth == 0) {
        heap_sort(r.first, r.last, comp);
        break;
      }
      --r.depth;
      T* cut = partition_pivot(r.first, r.last, comp);
      stack[top++] = Range{cut, r.last, r.depth};
      r.last = cut;
    }
  }
}

// std::sort(first, last, comp)
template <class T, class Cmp>
TRS_HD void sort(T* first, T* last, Cmp comp) {
  if (first == last) return;
  introsort_loop(first, last, 2 * lg(last - first), comp);
  final_insertion_sort(first, last, comp);
}

// The partition step as lists instead of moving scans, the form the device builder runs with a
// wave per range.  With p the pivot's key after move_median_to_first, L = the positions of
// (first, last) whose element the left scan stops at (comp(x, pivot) false), ascending, and
// R = the positions the right scan stops at (comp(pivot, x) false), descending, followed by
// `first` itself (where the unguarded right scan always stops), all read before any swap:
//   k* = the first k with R[k] <= L[k];  the pairs (L[k], R[k]), k < k*, are swapped;
//   cut = L[0] if k* = 0, else min(L[k*], R[k*-1]).
// (The left scan of round k* stops at R[k*-1] when no original stop lies before it: that slot
// then holds the element swapped in from L[k*-1].)  Equal to partition_pivot's result for any
// input; the tests check it against the scans above.
template <class T, class Cmp>
TRS_HD int64_t partition_by_lists(T* a, int64_t first, int64_t last, Cmp& comp, int64_t* Lbuf, int64_t* Rbuf) {
  const int64_t mid = first + (last - first) / 2;
  move_median_to_first(a + first, a + first + 1, a + mid, a + last - 1, comp);
  const T pivot = a[first];
  int64_t nl = 0, nr = 0;
  for (int64_t i = first + 1; i < last; ++i)
    if (!comp(a[i], pivot)) Lbuf[nl++] = i;
  for (int64_t i = last - 1; i > first; --i)
    if (!comp(pivot, a[i])) Rbuf[nr++] = i;
  Rbuf[nr++] = first;
  int64_t k = 0;
  while (k < nl && k < nr && Rbuf[k] > Lbuf[k]) ++k;
  // k = k*; the left list never runs out before the crossing (libstdc++'s median guarantees a
  // stop); guard anyway
  int64_t cut = k < nl ? Lbuf[k] : last;
  if (k > 0 && Rbuf[k - 1] < cut) cut = Rbuf[k - 1];
  for (int64_t j = 0; j < k; ++j) swap_at(a + Lbuf[j], a + Rbuf[j]);
  return cut;
}

// A range of L elements that all compare equal, entered with depth limit d: introsort_loop's
// steps do not depend on the elements, so each one's final offset follows from its own.  Per
// step: move_median_to_first swaps offsets 0 and L / 2 (every comparison is false); the scans stop
// at every position, so the pairs (1 + k, L - 1 - k), k < (L - 1) / 2, swap; the cut is
// (L + 1) / 2; then the part holding the element continues, one depth lower, until at most 16
// remain (the final insertion sort moves no equal elements).  tied_depth_ok(L, d): the depth limit
// lasts (no part of more than 16 elements reaches depth 0, where the loop would heap-sort).
TRS_HD inline bool tied_depth_ok(int64_t L, int d) {
  while (L > kThreshold) {
    if (d == 0) return false;
    --d;
    L = (L + 1) / 2;   // the larger part
  }
  return true;
}

TRS_HD inline int64_t tied_final_offset(int64_t L, int64_t o) {
  int64_t base = 0;
  while (L > kThreshold) {
    const int64_t mid = L / 2;
    if (o == 0) o = mid;
    else if (o == mid) o = 0;
    const int64_t ks = (L - 1) / 2;
    if ((o >= 1 && o <= ks) || o >= L - ks) o = L - o;
    const int64_t c = (L + 1) / 2;
    if (o >= c) {
      base += c;
      o -= c;
      L -= c;
    } else {
      L = c;
    }
  }
  return base + o;
}

// The same step in batches of `lanes` pairs, as a wave runs it (one lane per pair), restated
// sequentially for the host tests.  The two lists are filled by scans of `lanes` positions at a
// time, which may read positions that an earlier batch has already swapped; such a read lies at
// or beyond the previous batch's last right stop (or at or below its last left stop), where the
// rule above stops the step with a cut that does not depend on it.  Buffers hold 2 * lanes
// entries each.  Returns the cut; the array is left as partition_pivot leaves it.
template <class T, class Cmp>
TRS_HD int64_t partition_batched(T* a, int64_t first, int64_t last, Cmp& comp, int lanes, int64_t* Lbuf,
                                 int64_t* Rbuf) {
  const int64_t mid = first + (last - first) / 2;
  move_median_to_first(a + first, a + first + 1, a + mid, a + last - 1, comp);
  const T pivot = a[first];
  int64_t aL = first + 1, aR = last - 1;   // next positions the scans read
  int64_t nL = 0, nR = 0;                  // buffered stops
  int64_t rprev = last;                    // right stop of the previous pair
  while (true) {
    while (nL < lanes && aL < last) {
      for (int j = 0; j < lanes; ++j)
        if (aL + j < last && !comp(a[aL + j], pivot)) Lbuf[nL++] = aL + j;
      aL += lanes;
    }
    while (nR < lanes && aR >= first) {
      for (int j = 0; j < lanes; ++j)
        if (aR - j >= first && !comp(pivot, a[aR - j])) Rbuf[nR++] = aR - j;
      aR -= lanes;
    }
    int kk = lanes;   // first lane whose pair has crossed
    for (int j = 0; j < lanes; ++j) {
      const int64_t L = j < nL ? Lbuf[j] : last, R = j < nR ? Rbuf[j] : -1;
      if (R <= L) { kk = j; break; }
    }
    for (int j = 0; j < kk; ++j) swap_at(a + Lbuf[j], a + Rbuf[j]);
    if (kk < lanes) {
      const int64_t L = kk < nL ? Lbuf[kk] : last;
      const int64_t rp = kk == 0 ? rprev : Rbuf[kk - 1];
      return rp < L ? rp : L;
    }
    rprev = Rbuf[lanes - 1];
    for (int64_t j = lanes; j < nL; ++j) Lbuf[j - lanes] = Lbuf[j];
    for (int64_t j = lanes; j < nR; ++j) Rbuf[j - lanes] = Rbuf[j];
    nL -= lanes;
    nR -= lanes;
  }
}

}  // namespace isort
}  // namespace trs
