// Test helper (compiled by tests/test_introsort.py with g++): checks the introsort restatement of
// tr-spmm_zzx_amd/csrc/introsort.hpp against this compiler's std::sort, and the list form of its
// partition against the scanning form.  Every check returns the number of trials that differ.
#include <algorithm>
#include <cstdint>
#include <numeric>
#include <random>
#include <vector>

#include "introsort.hpp"

namespace {

// The builder's use: unit indices sorted by a key, descending, ties left to the algorithm.
struct ByKeyDesc {
  const int32_t* key;
  bool operator()(int32_t a, int32_t b) const { return key[a] > key[b]; }
};

bool same_as_std(const std::vector<int32_t>& key) {
  const int64_t n = (int64_t)key.size();
  std::vector<int32_t> a(n), b(n);
  std::iota(a.begin(), a.end(), 0);
  std::iota(b.begin(), b.end(), 0);
  std::sort(a.begin(), a.end(), ByKeyDesc{key.data()});
  trs::isort::sort(b.data(), b.data() + n, ByKeyDesc{key.data()});
  return a == b;
}

// McIlroy's adversary ("A killer adversary for quicksort", 1999): values are fixed lazily as the
// sort compares them, so that the recorded input drives this very algorithm into its worst
// case -- for introsort, past the depth limit into the heap sort.
std::vector<int32_t> killer_input(int64_t n) {
  std::vector<int32_t> val(n);
  const int32_t gas = (int32_t)n;
  std::fill(val.begin(), val.end(), gas);
  int32_t nsolid = 0;
  int64_t candidate = 0;
  std::vector<int32_t> ptr(n);
  std::iota(ptr.begin(), ptr.end(), 0);
  auto cmp = [&](int32_t x, int32_t y) {
    if (val[x] == gas && val[y] == gas) {
      if (x == candidate) val[x] = nsolid++;
      else val[y] = nsolid++;
    }
    if (val[x] == gas) candidate = x;
    else if (val[y] == gas) candidate = y;
    return val[x] < val[y];
  };
  std::sort(ptr.begin(), ptr.end(), cmp);
  for (auto& v : val)
    if (v == gas) v = nsolid++;
  return val;
}

}  // namespace

extern "C" {

// Random keys over `alphabet` values (1 = all equal), `trials` of each size in sizes[].
int64_t check_random(const int64_t* sizes, int32_t nsizes, int32_t alphabet, int32_t trials, uint64_t seed) {
  std::mt19937_64 rng(seed);
  int64_t bad = 0;
  for (int32_t s = 0; s < nsizes; ++s)
    for (int32_t t = 0; t < trials; ++t) {
      std::vector<int32_t> key((size_t)sizes[s]);
      for (auto& k : key) k = (int32_t)(rng() % (uint64_t)alphabet);
      bad += !same_as_std(key);
    }
  return bad;
}

// The builder's case: keys non-increasing in the index (units in count order), runs of random
// lengths over `alphabet` values.
int64_t check_monotone(const int64_t* sizes, int32_t nsizes, int32_t alphabet, int32_t trials, uint64_t seed) {
  std::mt19937_64 rng(seed);
  int64_t bad = 0;
  for (int32_t s = 0; s < nsizes; ++s)
    for (int32_t t = 0; t < trials; ++t) {
      std::vector<int32_t> key((size_t)sizes[s]);
      for (auto& k : key) k = (int32_t)(rng() % (uint64_t)alphabet);
      std::sort(key.begin(), key.end(), [](int32_t a, int32_t b) { return a > b; });
      bad += !same_as_std(key);
    }
  return bad;
}

// Adversarial inputs that exhaust the depth limit (heap-sort path), also with ties (value / tie).
int64_t check_killer(const int64_t* sizes, int32_t nsizes, int32_t tie) {
  int64_t bad = 0;
  for (int32_t s = 0; s < nsizes; ++s) {
    std::vector<int32_t> key = killer_input(sizes[s]);
    for (auto& k : key) k = -k / tie;   // ByKeyDesc sorts descending: negate the ascending killer
    bad += !same_as_std(key);
  }
  return bad;
}

// 1 if the killer input of size n drives the restatement's loop to a range of more than 16
// elements at depth 0, where introsort_loop switches to the heap sort (the loop below walks the
// same ranges as introsort_loop, with the header's partition step).
int32_t killer_reaches_heap_sort(int64_t n) {
  std::vector<int32_t> key = killer_input(n);
  for (auto& k : key) k = -k;
  std::vector<int32_t> a((size_t)n);
  std::iota(a.begin(), a.end(), 0);
  ByKeyDesc cmp{key.data()};
  struct Range { int32_t* first; int32_t* last; int depth; };
  std::vector<Range> stack{{a.data(), a.data() + n, 2 * trs::isort::lg(n)}};
  while (!stack.empty()) {
    Range r = stack.back();
    stack.pop_back();
    while (r.last - r.first > trs::isort::kThreshold) {
      if (r.depth == 0) return 1;
      --r.depth;
      int32_t* cut = trs::isort::partition_pivot(r.first, r.last, cmp);
      stack.push_back({cut, r.last, r.depth});
      r.last = cut;
    }
  }
  return 0;
}

// partition_by_lists against partition_pivot on random arrays (values over `alphabet`), both the
// array after the step and the cut.
int64_t check_partition_lists(int64_t n_max, int32_t alphabet, int32_t trials, uint64_t seed, int32_t monotone) {
  std::mt19937_64 rng(seed);
  int64_t bad = 0;
  std::vector<int64_t> L, R;
  for (int32_t t = 0; t < trials; ++t) {
    const int64_t n = 17 + (int64_t)(rng() % (uint64_t)(n_max - 16));
    std::vector<int32_t> key((size_t)n);
    for (auto& k : key) k = (int32_t)(rng() % (uint64_t)alphabet);
    if (monotone) std::sort(key.begin(), key.end(), [](int32_t a, int32_t b) { return a > b; });
    std::vector<int32_t> a((size_t)n), b;
    std::iota(a.begin(), a.end(), 0);
    std::shuffle(a.begin(), a.end(), rng);
    if (monotone) std::iota(a.begin(), a.end(), 0);
    b = a;
    ByKeyDesc cmp{key.data()};
    int32_t* cut_a = trs::isort::partition_pivot(a.data(), a.data() + n, cmp);
    L.assign((size_t)n + 1, 0);
    R.assign((size_t)n + 1, 0);
    const int64_t cut_b = trs::isort::partition_by_lists(b.data(), (int64_t)0, n, cmp, L.data(), R.data());
    bad += (cut_a - a.data() != cut_b) || a != b;
  }
  return bad;
}

// partition_batched (the wave form, `lanes` pairs per batch) against partition_pivot, and whole
// sorts whose every partition step is the batched one against std::sort.
int64_t check_partition_batched(int64_t n_max, int32_t alphabet, int32_t trials, uint64_t seed, int32_t monotone,
                                int32_t lanes) {
  std::mt19937_64 rng(seed);
  int64_t bad = 0;
  std::vector<int64_t> L(2 * (size_t)lanes + 1), R(2 * (size_t)lanes + 1);
  for (int32_t t = 0; t < trials; ++t) {
    const int64_t n = 17 + (int64_t)(rng() % (uint64_t)(n_max - 16));
    std::vector<int32_t> key((size_t)n);
    for (auto& k : key) k = (int32_t)(rng() % (uint64_t)alphabet);
    if (monotone) std::sort(key.begin(), key.end(), [](int32_t a, int32_t b) { return a > b; });
    std::vector<int32_t> a((size_t)n), b;
    std::iota(a.begin(), a.end(), 0);
    if (!monotone) std::shuffle(a.begin(), a.end(), rng);
    b = a;
    ByKeyDesc cmp{key.data()};
    int32_t* cut_a = trs::isort::partition_pivot(a.data(), a.data() + n, cmp);
    const int64_t cut_b = trs::isort::partition_batched(b.data(), (int64_t)0, n, cmp, lanes, L.data(), R.data());
    bad += (cut_a - a.data() != cut_b) || a != b;
  }
  return bad;
}

// A full sort with partition_batched in place of the scanning partition, the leaves finished by
// a stable insertion sort each (what the final insertion sort amounts to after the loop), against
// std::sort: the device builder's whole order.
int64_t check_batched_sort(const int64_t* sizes, int32_t nsizes, int32_t alphabet, int32_t trials, uint64_t seed,
                           int32_t lanes) {
  std::mt19937_64 rng(seed);
  int64_t bad = 0;
  std::vector<int64_t> L(2 * (size_t)lanes + 1), R(2 * (size_t)lanes + 1);
  for (int32_t s = 0; s < nsizes; ++s)
    for (int32_t t = 0; t < trials; ++t) {
      const int64_t n = sizes[s];
      std::vector<int32_t> key((size_t)n);
      for (auto& k : key) k = (int32_t)(rng() % (uint64_t)alphabet);
      std::sort(key.begin(), key.end(), [](int32_t a, int32_t b) { return a > b; });
      std::vector<int32_t> a((size_t)n), b((size_t)n);
      std::iota(a.begin(), a.end(), 0);
      std::iota(b.begin(), b.end(), 0);
      ByKeyDesc cmp{key.data()};
      std::sort(a.begin(), a.end(), cmp);
      struct Range { int64_t f, l; int d; };
      std::vector<Range> stack;
      if (n > 1) stack.push_back({0, n, 2 * trs::isort::lg(n)});
      while (!stack.empty()) {
        Range r = stack.back();
        stack.pop_back();
        bool heap = false;
        while (r.l - r.f > trs::isort::kThreshold) {
          if (r.d == 0) {
            trs::isort::heap_sort(b.data() + r.f, b.data() + r.l, cmp);
            heap = true;
            break;
          }
          --r.d;
          const int64_t cut = trs::isort::partition_batched(b.data(), r.f, r.l, cmp, lanes, L.data(), R.data());
          stack.push_back({cut, r.l, r.d});
          r.l = cut;
        }
        if (!heap) std::stable_sort(b.begin() + r.f, b.begin() + r.l, cmp);
      }
      bad += a != b;
    }
  return bad;
}

// tied_final_offset against the restated loop on ranges of equal elements (every comparison
// false), for lengths 0..Lmax and depth limits from the least that lasts to 3 more; returns the
// number of (L, d) that differ, or -1 if tied_depth_ok disagrees with the loop reaching a heap sort.
int64_t check_tied(int64_t Lmax) {
  struct Never {
    bool operator()(int32_t, int32_t) const { return false; }
  };
  int64_t bad = 0;
  for (int64_t L = 0; L <= Lmax; L += (L < 3000 ? 1 : 997)) {
    int dmin = 0;
    while (!trs::isort::tied_depth_ok(L, dmin)) ++dmin;
    for (int d = (dmin > 0 ? dmin - 1 : 0); d <= dmin + 3; ++d) {
      std::vector<int32_t> a((size_t)L);
      std::iota(a.begin(), a.end(), 0);
      Never cmp;
      // does the loop heap-sort at depth d? walk its ranges as killer_reaches_heap_sort does
      bool heap = false;
      {
        struct Range { int64_t f, l; int d; };
        std::vector<Range> st{{0, L, d}};
        std::vector<int32_t> b = a;
        while (!st.empty() && !heap) {
          Range r = st.back();
          st.pop_back();
          while (r.l - r.f > trs::isort::kThreshold) {
            if (r.d == 0) { heap = true; break; }
            --r.d;
            int32_t* cut = trs::isort::partition_pivot(b.data() + r.f, b.data() + r.l, cmp);
            st.push_back({cut - b.data(), r.l, r.d});
            r.l = cut - b.data();
          }
        }
      }
      if (heap == trs::isort::tied_depth_ok(L, d)) return -1;
      if (heap) continue;
      if (L > 0) trs::isort::introsort_loop(a.data(), a.data() + L, d, cmp);
      if (L > 0) trs::isort::final_insertion_sort(a.data(), a.data() + L, cmp);
      for (int64_t o = 0; o < L; ++o)
        if (a[(size_t)trs::isort::tied_final_offset(L, o)] != o) { ++bad; break; }
    }
  }
  return bad;
}

}  // extern "C"
