// Statistics-only 2:4 matching (trs_match_2to4 in include/trspmm.h), the counterpart of the
// reference's matching_utils.match_2to4 (TR-source/Block/block_matching_window_para_dr.cpp).
//
// Per window of `window_size` rows (windows are independent; OpenMP over windows, counts summed):
//   columns   every distinct column of the window with a 16-bit row mask; row r of the window
//             contributes bit (1 << (r mod 32)) kept to 16 bits, which is what the reference's int
//             shift stored into uint16_t does on x86 (:296-300).  Columns ascend by id (:110-113).
//   1:2       column i pairs with the first later unmatched column within 32 positions whose
//             masks do not overlap, else with the first one of least overlap <= t_max; without a
//             partner it goes to the dense pool (:120-157)
//   2:4       pair i takes the first later unused pair within 1024 positions whose masks do not
//             conflict, Z = (G1a & G2b) | (G2a & G1b) == 0 with G1 = and, G2 = or of a pair's masks;
//             without one, both of its columns go to the pool (:166-210)
//   routing   the pool in order: whole blocks of dense_threshold columns are TC blocks, the rest
//             fill 2:4 groups two real columns at a time (:218-259); groups per window round up to
//             tiles of 4 (:264-270)
// The scans walk linked lists of the still-free candidates, so a candidate that is taken is never
// visited again; the position limits (32, 1024) are the reference's, counted over all candidates.
#include <algorithm>
#include <cstdint>
#include <new>
#include <vector>

#include <omp.h>

#include "format.hpp"

namespace {

constexpr int kSearchWindow = 32;
constexpr int kGroupSearchWindow = 1024;

struct Totals {
  int64_t groups = 0, tc_blocks = 0, tiles = 0, pad_groups = 0, fine = 0, coarse = 0, fake = 0;
  int64_t tc_nnz = 0, tc_count = 0, tc_max = 0, tc_min = 999999;

  void add(const Totals& o) {
    groups += o.groups;
    tc_blocks += o.tc_blocks;
    tiles += o.tiles;
    pad_groups += o.pad_groups;
    fine += o.fine;
    coarse += o.coarse;
    fake += o.fake;
    tc_nnz += o.tc_nnz;
    tc_count += o.tc_count;
    tc_max = std::max(tc_max, o.tc_max);
    tc_min = std::min(tc_min, o.tc_min);
  }
};

// Doubly linked list over positions 0..n-1 of the candidates still free (sentinel at n).
struct FreeList {
  std::vector<int32_t> next, prev;
  void reset(int32_t n) {
    next.resize(n + 1);
    prev.resize(n + 1);
    for (int32_t i = 0; i <= n; ++i) {
      next[i] = i + 1;
      prev[i] = i - 1;
    }
    next[n] = 0;        // sentinel: head = next[n]
    prev[0] = n;
    if (n == 0) next[0] = 0;
  }
  void take(int32_t i) {
    next[prev[i]] = next[i];
    prev[next[i]] = prev[i];
  }
};

struct Scratch {
  std::vector<uint64_t> keys;          // (column << 16) | row bit
  std::vector<uint16_t> mask;          // per window column
  std::vector<int32_t> pool;           // window column positions
  std::vector<uint16_t> g1, g2;        // per pair
  std::vector<int32_t> pnnz, pa, pb;   // per pair: nnz, column positions
  FreeList free_cols, free_pairs;
};

void match_window(int32_t win_rows, int32_t dense_threshold, int32_t t_max, Scratch& s, Totals& t) {
  const int32_t n = (int32_t)s.mask.size();
  const uint16_t* m = s.mask.data();
  s.pool.clear();
  s.g1.clear();
  s.g2.clear();
  s.pnnz.clear();
  s.pa.clear();
  s.pb.clear();

  // 1:2 pairs.  Column i is the head of the free list when it is reached, so "later unmatched
  // columns" are its successors in the list; the scan stops at position i + 32.
  FreeList& fc = s.free_cols;
  fc.reset(n);
  for (int32_t i = fc.next[n]; i != n; i = fc.next[n]) {
    fc.take(i);
    const uint16_t mi = m[i];
    const int32_t j_end = std::min(i + 1 + kSearchWindow, n);
    int32_t best = -1, min_cost = t_max + 1;
    for (int32_t j = fc.next[n]; j != n && j < j_end; j = fc.next[j]) {
      const int32_t cost = __builtin_popcount((uint32_t)(mi & m[j]));
      if (cost == 0) {
        best = j;
        break;
      }
      if (cost <= t_max && cost < min_cost) {
        min_cost = cost;
        best = j;
      }
    }
    if (best >= 0) {
      fc.take(best);
      s.g1.push_back((uint16_t)(mi & m[best]));
      s.g2.push_back((uint16_t)(mi | m[best]));
      s.pnnz.push_back(__builtin_popcount(mi) + __builtin_popcount(m[best]));
      s.pa.push_back(i);
      s.pb.push_back(best);
    } else {
      s.pool.push_back(i);
      ++t.fine;
    }
  }

  // 2:4 groups over the pairs, same scheme.
  const int32_t np = (int32_t)s.g1.size();
  int64_t groups = 0;
  FreeList& fp = s.free_pairs;
  fp.reset(np);
  for (int32_t i = fp.next[np]; i != np; i = fp.next[np]) {
    fp.take(i);
    const uint16_t a1 = s.g1[i], a2 = s.g2[i];
    const int32_t j_end = std::min(i + 1 + kGroupSearchWindow, np);
    int32_t hit = -1;
    for (int32_t j = fp.next[np]; j != np && j < j_end; j = fp.next[j])
      if (((a1 & s.g2[j]) | (a2 & s.g1[j])) == 0) {
        hit = j;
        break;
      }
    if (hit >= 0) {
      fp.take(hit);
      ++groups;
      t.fake += 2 * (int64_t)win_rows - (s.pnnz[i] + s.pnnz[hit]);
    } else {
      s.pool.push_back(s.pa[i]);
      s.pool.push_back(s.pb[i]);
      t.coarse += 2;
    }
  }

  // routing of the pool
  const int32_t nd = (int32_t)s.pool.size();
  int32_t done = 0;
  for (; nd - done >= dense_threshold; done += dense_threshold) {
    int64_t block = 0;
    for (int32_t k = 0; k < dense_threshold; ++k) block += __builtin_popcount(m[s.pool[done + k]]);
    t.tc_nnz += block;
    t.tc_count += 1;
    t.tc_max = std::max(t.tc_max, block);
    t.tc_min = std::min(t.tc_min, block);
    t.tc_blocks += 1;
  }
  for (int32_t k = done; k < nd; k += 2) {
    int64_t real = __builtin_popcount(m[s.pool[k]]);
    if (k + 1 < nd) real += __builtin_popcount(m[s.pool[k + 1]]);
    t.fake += 2 * (int64_t)win_rows - real;
    ++groups;
  }
  const int64_t tiles = (groups + 3) / 4;
  t.groups += groups;
  t.tiles += tiles;
  t.pad_groups += tiles * 4 - groups;
}

// Distinct columns of rows [r0, r1) with their masks, ascending by column.
void window_columns(const int32_t* rowptr, const int32_t* col, int32_t r0, int32_t r1, Scratch& s) {
  s.keys.clear();
  s.mask.clear();
  for (int32_t r = r0; r < r1; ++r) {
    const uint64_t bit = (uint16_t)(1u << ((r - r0) & 31));
    for (int32_t e = rowptr[r]; e < rowptr[r + 1]; ++e) s.keys.push_back(((uint64_t)(uint32_t)col[e] << 16) | bit);
  }
  std::sort(s.keys.begin(), s.keys.end());
  for (size_t k = 0; k < s.keys.size();) {
    const uint64_t c = s.keys[k] >> 16;
    uint16_t mk = 0;
    for (; k < s.keys.size() && (s.keys[k] >> 16) == c; ++k) mk |= (uint16_t)s.keys[k];
    s.mask.push_back(mk);
  }
}

}  // namespace

extern "C" {

int trs_match_2to4(const int32_t* rowptr, const int32_t* col, int32_t rows, int64_t nnz, int32_t window_size,
                   int32_t dense_threshold, int32_t t_max, int32_t num_threads, trs_match_stats* out) {
  if (!out || rows < 0 || nnz < 0 || (rows > 0 && !rowptr) || (nnz > 0 && !col) || num_threads < 0) {
    trs::set_error("trs_match_2to4: bad arguments");
    return TRS_EINVAL;
  }
  if (window_size < 1 || window_size > 64) {
    trs::set_error("trs_match_2to4: window_size must be in [1, 64]");
    return TRS_EINVAL;
  }
  if (dense_threshold < 1) {
    trs::set_error("trs_match_2to4: dense_threshold must be >= 1");
    return TRS_EINVAL;
  }
  int64_t cols = 0;
  for (int64_t j = 0; j < nnz; ++j) {
    if (col[j] < 0) {
      trs::set_error("trs_match_2to4: negative column index");
      return TRS_ERANGE;
    }
    cols = std::max(cols, (int64_t)col[j] + 1);
  }
  if (rows <= 0 || cols <= 0) {
    trs::set_error("trs_match_2to4: invalid matrix dimensions (no rows or no columns)");
    return TRS_EINVAL;
  }
  if (rowptr[0] < 0 || rowptr[rows] > nnz) {
    trs::set_error("trs_match_2to4: rowptr outside [0, nnz]");
    return TRS_EINVAL;
  }
  for (int32_t i = 0; i < rows; ++i)
    if (rowptr[i + 1] < rowptr[i]) {
      trs::set_error("trs_match_2to4: rowptr not monotone");
      return TRS_EINVAL;
    }

  const int32_t nwin = (int32_t)(((int64_t)rows + window_size - 1) / window_size);
  Totals total;
  int oom = 0;
  const int threads = num_threads > 0 ? num_threads : omp_get_max_threads();
#pragma omp parallel num_threads(threads)
  {
    Totals mine;
    Scratch s;
#pragma omp for schedule(dynamic, 16) nowait
    for (int32_t w = 0; w < nwin; ++w) {
      // an exception may not leave a worksharing loop: it is caught in its own iteration
      try {
        const int32_t r0 = w * window_size;
        const int32_t r1 = (int32_t)std::min<int64_t>((int64_t)r0 + window_size, rows);
        window_columns(rowptr, col, r0, r1, s);
        if (!s.mask.empty()) match_window(r1 - r0, dense_threshold, t_max, s, mine);
      } catch (const std::bad_alloc&) {
#pragma omp atomic write
        oom = 1;
      }
    }
#pragma omp critical(trs_match_totals)
    total.add(mine);
  }
  if (oom) {
    trs::set_error("trs_match_2to4: out of memory");
    return TRS_ENOMEM;
  }

  out->total_rows = rows;
  out->total_cols = cols;
  out->total_nnz = rowptr[rows];
  out->sparsity = 1.0 - (double)rowptr[rows] / ((double)rows * (double)cols);
  out->num_row_panels = nwin;
  out->num_sptc_groups = total.groups;
  out->num_tc_blocks = total.tc_blocks;
  out->num_16x16_blocks = total.tiles;
  out->block_padding_groups = total.pad_groups;
  out->fine_fallback = total.fine;
  out->coarse_fallback = total.coarse;
  out->fake_zeros = total.fake;
  out->tc_total_nnz = total.tc_nnz;
  out->tc_block_count = total.tc_count;
  out->tc_block_max_nnz = total.tc_max;
  out->tc_block_min_nnz = total.tc_min;
  return TRS_OK;
}

}  // extern "C"
