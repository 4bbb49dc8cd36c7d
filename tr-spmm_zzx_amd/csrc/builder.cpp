// Hybrid-format builder: CSR -> the reference's 29-array "online" tuple (bit-exact) + spill list.
//
// Reference: TR-source/Block/block_online.cpp:545-871 (`block_sptc_2to4_online`).  The array
// layout, the per-window routing rules and the tie rules are the reference's; the implementation
// is new:
//   * windows are independent (the reference serialises them in window order through std::map,
//     block_online.cpp:569-570, 736-776), so they are built in parallel with OpenMP into per-window
//     buffers and concatenated afterwards;
//   * per-window column statistics come from one sort of (column, local row, edge) keys instead of
//     unordered_map/unordered_set lookups (block_online.cpp:588-603);
//   * for column vectors holding only 0/1 per 2-bit row field (always the case for window <= 16,
//     because each (row, column) is counted once) the conflict test of block_online.cpp:83-88 can
//     never fire, so every unit pair is compatible.  Then: units are consecutive pairs of the
//     (count desc, column asc) candidate order; every unit has degree n-1; the max-degree order is
//     libstdc++ std::sort by nnz desc over 0..n-1 (same comparator outcomes as
//     block_online.cpp:360-363, hence the same tie order); and the greedy partner is the
//     lowest-index unmatched unit of maximal nnz (block_online.cpp:365-386), found with per-nnz
//     buckets in O(n) instead of an O(n^2) graph;
//   * other windows (window > 16, where the reference's 32-bit shift wraps) run the literal rules
//     with O(n) memory.
// It also emits the spill: entries that no output array carries (2:4 groups keep only the first
// two present values per row, block_online.cpp:690-694, and the rest is lost in the reference).
#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <immintrin.h>
#include <memory>
#include <memory_resource>
#include <omp.h>
#include <optional>
#include <string>
#include <vector>

#include "format.hpp"
#include "half.hpp"

namespace {

// A window's output arrays live until the serialisation copies them into the format, so they are
// allocated from a per-thread monotonic arena (released once, after the build) instead of the
// general heap: freeing and re-allocating them window after window returned memory to the system
// and faulted it back in, which doubled a first build in a fresh process (grid+hubs 0.76 s against
// 0.35 s for a second one, R-MAT 0.45 s against 0.26 s on the GPU box host).
template <class T>
using wvec = std::pmr::vector<T>;

struct Cuda {
  wvec<int32_t> cnt, row, atomic, col;
  wvec<float> val;
  explicit Cuda(std::pmr::memory_resource* r) : cnt(r), row(r), atomic(r), col(r), val(r) {}
};

struct Win {
  // TC
  wvec<int32_t> t_parts, t_subcnt, t_col, t_atomic;
  wvec<int64_t> t_bin;
  wvec<float> t_val;
  // CUDA residual, long and short parts
  Cuda lng, sht;
  // SPTC groups
  wvec<int32_t> s_col;
  wvec<uint8_t> s_mask;
  wvec<float> s_val;
  wvec<int8_t> s_pos;
  // tiles (tile_group holds the window-local first group)
  wvec<int32_t> tile_group, tile_cols, packed_a, packed_meta;
  // spill
  wvec<int32_t> sp_row, sp_col;
  wvec<float> sp_val;
  bool canonical = true;
  explicit Win(std::pmr::memory_resource* r)
      : t_parts(r), t_subcnt(r), t_col(r), t_atomic(r), t_bin(r), t_val(r), lng(r), sht(r), s_col(r), s_mask(r),
        s_val(r), s_pos(r), tile_group(r), tile_cols(r), packed_a(r), packed_meta(r), sp_row(r), sp_col(r),
        sp_val(r) {}
};

struct Params {
  int part_t, part_c, short_size, density, window, skip_tc, unit_min_nnz;
  float tc_min_util;
};

inline bool compatible(uint32_t a, uint32_t b) {
  const uint32_t c = a | b;
  return (((a & b) | ((c << 1) & c)) & 0xaaaaaaaau) == 0;
}

// Scratch reused across the windows one thread builds.
struct Scratch {
  struct Key { uint64_t k; int64_t e; };   // k = col << 5 | local_row
  std::vector<Key> keys;
  std::vector<int32_t> ucol, ucount, first_beg;   // per distinct column
  std::vector<uint32_t> uvec;
  std::vector<int32_t> first_lr;                  // first occurrence per (column, row)
  std::vector<int64_t> first_e;
  std::vector<int32_t> ecol;                      // edge (window-local) -> distinct column index
  std::vector<int32_t> status;                    // per distinct column: >=0 TC slot, -2 SPTC, -1 residual
  std::vector<uint8_t> covered;                   // per window-local edge
  std::vector<int32_t> cand, order;
  std::vector<int32_t> u1, u2, unnz;
  std::vector<uint32_t> uvec_unit;
  std::vector<char> matched;
  std::vector<std::vector<int32_t>> bucket;
  std::vector<size_t> cursor;
};

// Order distinct-column indices by (count desc, column asc) -- the total order of
// block_online.cpp:226-230 and :281-285.  Indices ascend with the column, so a counting sort on
// the count that keeps index order within a count gives exactly that order.
void sort_by_count(Scratch& S, std::vector<int32_t>& v) {
  int maxc = 0;
  for (int u : v) maxc = std::max(maxc, S.ucount[u]);
  std::vector<int32_t> start(maxc + 2, 0);
  for (int u : v) start[maxc - S.ucount[u] + 1]++;
  for (int i = 0; i <= maxc; ++i) start[i + 1] += start[i];
  std::vector<int32_t> out(v.size());
  for (int u : v) out[start[maxc - S.ucount[u]]++] = u;
  v.swap(out);
}

void split_residual_row(int row, int base_atomic, const Params& P, const int32_t* cols, const float* vals,
                        int n, Win& W) {
  // block_online.cpp:397-439
  auto emit = [&](Cuda& d, int atomic, int off, int cnt) {
    d.cnt.push_back(cnt);
    d.row.push_back(row);
    d.atomic.push_back(atomic);
    d.col.insert(d.col.end(), cols + off, cols + off + cnt);
    d.val.insert(d.val.end(), vals + off, vals + off + cnt);
  };
  if (n <= 0) return;
  if (n <= P.short_size) { emit(W.sht, base_atomic, 0, n); return; }
  if (n <= P.part_c) { emit(W.lng, base_atomic, 0, n); return; }
  const int full = n / P.part_c;
  int off = 0;
  for (int i = 0; i < full; ++i, off += P.part_c) emit(W.lng, 1, off, P.part_c);
  const int rem = n % P.part_c;
  if (rem > 0) emit(rem <= P.short_size ? W.sht : W.lng, 1, off, rem);
}

// Greedy max-degree matching when every pair of units is compatible (see file comment).
void match_all_compatible(Scratch& S, int n, std::vector<std::pair<int, int>>& pairs) {
  auto& order = S.order;
  order.resize(n);
  std::iota(order.begin(), order.end(), 0);
  const int32_t* nnz = S.unnz.data();
  std::sort(order.begin(), order.end(), [nnz](int a, int b) { return nnz[a] > nnz[b]; });
  int maxv = 0;
  for (int i = 0; i < n; ++i) maxv = std::max(maxv, nnz[i]);
  if ((int)S.bucket.size() < maxv + 1) S.bucket.resize(maxv + 1);
  for (int v = 0; v <= maxv; ++v) S.bucket[v].clear();
  for (int i = 0; i < n; ++i) S.bucket[nnz[i]].push_back(i);
  S.cursor.assign(maxv + 1, 0);
  S.matched.assign(n, 0);
  for (int idx : order) {
    if (S.matched[idx]) continue;
    int best = -1;
    for (int v = maxv; v >= 0 && best < 0; --v) {
      auto& B = S.bucket[v];
      size_t& c = S.cursor[v];
      while (c < B.size() && S.matched[B[c]]) ++c;
      size_t k = c;
      while (k < B.size() && (S.matched[B[k]] || B[k] == idx)) ++k;
      if (k < B.size()) best = B[k];
    }
    if (best >= 0) {
      S.matched[idx] = S.matched[best] = 1;
      pairs.push_back({idx, best});
    }
  }
}

// Literal rules of block_online.cpp:332-392 with the graph evaluated on the fly.
void match_literal(Scratch& S, int n, std::vector<std::pair<int, int>>& pairs) {
  std::vector<int> deg(n, 0);
  for (int i = 0; i < n; ++i)
    for (int j = i + 1; j < n; ++j)
      if (compatible(S.uvec_unit[i], S.uvec_unit[j])) { deg[i]++; deg[j]++; }
  auto& order = S.order;
  order.resize(n);
  std::iota(order.begin(), order.end(), 0);
  const int32_t* nnz = S.unnz.data();
  std::sort(order.begin(), order.end(), [&](int a, int b) {
    if (deg[a] != deg[b]) return deg[a] > deg[b];
    return nnz[a] > nnz[b];
  });
  S.matched.assign(n, 0);
  for (int idx : order) {
    if (S.matched[idx]) continue;
    int best = -1, bdeg = -1;
    for (int j = 0; j < n; ++j) {
      if (j == idx || S.matched[j] || !compatible(S.uvec_unit[idx], S.uvec_unit[j])) continue;
      if (deg[j] > bdeg || (deg[j] == bdeg && nnz[j] > nnz[best])) { best = j; bdeg = deg[j]; }
    }
    if (best >= 0) {
      S.matched[idx] = S.matched[best] = 1;
      pairs.push_back({idx, best});
    }
  }
}

void load_chunk(const Win& W, int g, int gend, int lr, int window, float& v0, float& v1, int& p0, int& p1) {
  // block_online.cpp:190-210 (g is window-local)
  v0 = v1 = 0.f; p0 = 0; p1 = 1;
  if (g >= gend || lr >= window) return;
  const size_t b = ((size_t)g * window + lr) * 2;
  const int q0 = W.s_pos[b], q1 = W.s_pos[b + 1];
  const float a0 = W.s_val[b], a1 = W.s_val[b + 1];
  if (q0 < 0 && q1 < 0) return;
  if (q0 >= 0 && q1 >= 0) {
    if (q0 <= q1) { p0 = q0; p1 = q1; v0 = a0; v1 = a1; } else { p0 = q1; p1 = q0; v0 = a1; v1 = a0; }
    return;
  }
  const int rp = q0 >= 0 ? q0 : q1;
  const float rv = q0 >= 0 ? a0 : a1;
  const int dummy = rp == 0 ? 1 : 0;
  if (dummy < rp) { p0 = dummy; p1 = rp; v0 = 0.f; v1 = rv; } else { p0 = rp; p1 = dummy; v0 = rv; v1 = 0.f; }
}

void build_window(const int32_t* rowptr, const int32_t* col, const float* val, int rows, int w,
                  const Params& P, Scratch& S, Win& W) {
  const int window = P.window;
  const int r0 = w * window, r1 = std::min(r0 + window, rows);
  const int64_t e0 = rowptr[r0], e1 = rowptr[r1];
  const int64_t ne = e1 - e0;

  // ---- per-column statistics (block_online.cpp:588-603) ----
  S.keys.resize(ne);
  for (int r = r0; r < r1; ++r) {
    const uint64_t lr = (uint64_t)(r - r0);
    int32_t prev = -1;
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      const int32_t c = col[e];
      if (c <= prev) W.canonical = false;
      prev = c;
      S.keys[e - e0] = {((uint64_t)(uint32_t)c << 5) | lr, e};
    }
  }
  std::sort(S.keys.begin(), S.keys.end(), [](const Scratch::Key& a, const Scratch::Key& b) {
    return a.k != b.k ? a.k < b.k : a.e < b.e;
  });
  S.ucol.clear(); S.ucount.clear(); S.uvec.clear(); S.first_beg.clear();
  S.first_lr.clear(); S.first_e.clear();
  S.ecol.resize(ne);
  for (int64_t i = 0; i < ne; ++i) {
    const uint64_t k = S.keys[i].k;
    const int32_t c = (int32_t)(k >> 5);
    const int lr = (int)(k & 31);
    if (S.ucol.empty() || S.ucol.back() != c) {
      S.ucol.push_back(c); S.ucount.push_back(0); S.uvec.push_back(0);
      S.first_beg.push_back((int32_t)S.first_lr.size());
    }
    const int u = (int)S.ucol.size() - 1;
    S.ecol[S.keys[i].e - e0] = u;
    if (i > 0 && S.keys[i - 1].k == k) continue;   // duplicate (row, column): first edge counts
    S.ucount[u]++;
    S.uvec[u] += 1u << ((2 * lr) & 31);             // 32-bit shift wraps for rows >= 16 (x86)
    S.first_lr.push_back(lr);
    S.first_e.push_back(S.keys[i].e);
  }
  const int nu = (int)S.ucol.size();
  S.first_beg.push_back((int32_t)S.first_lr.size());
  S.status.assign(nu, -1);

  // ---- stage 1: TC column chunks of 8 (block_online.cpp:215-253, 611) ----
  std::vector<std::vector<int>> tc_groups;   // distinct-column indices, ascending column
  if (!P.skip_tc) {
    S.cand.clear();
    for (int u = 0; u < nu; ++u) if (S.ucount[u] >= P.density) S.cand.push_back(u);
    sort_by_count(S, S.cand);
    for (size_t s = 0; s < S.cand.size(); s += 8) {
      const size_t e = std::min(s + 8, S.cand.size());
      int nnz = 0;
      for (size_t i = s; i < e; ++i) nnz += S.ucount[S.cand[i]];
      const float util = (float)nnz / (float)(window * 8);
      if (util < P.tc_min_util) continue;
      std::vector<int> g(S.cand.begin() + s, S.cand.begin() + e);
      std::sort(g.begin(), g.end());   // distinct-column index order == column order
      tc_groups.push_back(std::move(g));
    }
    for (size_t b = 0; b < tc_groups.size(); ++b)
      for (size_t p = 0; p < tc_groups[b].size(); ++p) S.status[tc_groups[b][p]] = (int32_t)(b * 8 + p);
  }

  // ---- stage 2: units (block_online.cpp:267-328) ----
  S.cand.clear();
  bool simple = true;   // every column vector has 0/1 row fields
  for (int u = 0; u < nu; ++u) {
    if (S.status[u] >= 0) continue;
    S.cand.push_back(u);
    if (S.uvec[u] & 0xaaaaaaaau) simple = false;
  }
  sort_by_count(S, S.cand);
  S.u1.clear(); S.u2.clear(); S.unnz.clear(); S.uvec_unit.clear();
  if (simple) {
    for (size_t i = 0; i < S.cand.size(); i += 2) {
      const int a = S.cand[i];
      const int b = i + 1 < S.cand.size() ? S.cand[i + 1] : -1;
      S.u1.push_back(a); S.u2.push_back(b);
      S.unnz.push_back(S.ucount[a] + (b >= 0 ? S.ucount[b] : 0));
      S.uvec_unit.push_back(S.uvec[a] | (b >= 0 ? S.uvec[b] : 0));
    }
  } else {
    std::vector<char> used(S.cand.size(), 0);
    for (size_t i = 0; i < S.cand.size(); ++i) {
      if (used[i]) continue;
      used[i] = 1;
      const int a = S.cand[i];
      int b = -1;
      for (size_t j = i + 1; j < S.cand.size(); ++j)
        if (!used[j] && compatible(S.uvec[a], S.uvec[S.cand[j]])) { used[j] = 1; b = S.cand[j]; break; }
      S.u1.push_back(a); S.u2.push_back(b);
      S.unnz.push_back(S.ucount[a] + (b >= 0 ? S.ucount[b] : 0));
      S.uvec_unit.push_back(S.uvec[a] | (b >= 0 ? S.uvec[b] : 0));
    }
  }
  const int nunits = (int)S.u1.size();
  std::vector<std::pair<int, int>> pairs;
  if (simple) match_all_compatible(S, nunits, pairs);
  else match_literal(S, nunits, pairs);

  // ---- groups (block_online.cpp:629-666) ----
  auto emit_group = [&](int* cols, int k) {   // cols: distinct-column indices
    std::sort(cols, cols + k);
    for (int i = 0; i < 4; ++i) {
      if (i < k) { S.status[cols[i]] = -2; W.s_col.push_back(S.ucol[cols[i]]); }
      else W.s_col.push_back(-1);
    }
  };
  std::vector<int32_t> gmembers;   // 4 distinct-column indices per group (-1 pad)
  for (auto& pr : pairs) {
    int c[4], k = 0;
    c[k++] = S.u1[pr.first];
    if (S.u2[pr.first] >= 0) c[k++] = S.u2[pr.first];
    c[k++] = S.u1[pr.second];
    if (S.u2[pr.second] >= 0) c[k++] = S.u2[pr.second];
    emit_group(c, k);
    for (int i = 0; i < 4; ++i) gmembers.push_back(i < k ? c[i] : -1);
  }
  for (int i = 0; i < nunits; ++i) {
    if (S.matched[i] || S.unnz[i] < P.unit_min_nnz) continue;
    int c[4], k = 0;
    c[k++] = S.u1[i];
    if (S.u2[i] >= 0) c[k++] = S.u2[i];
    emit_group(c, k);
    for (int j = 0; j < 4; ++j) gmembers.push_back(j < k ? c[j] : -1);
  }
  const int ng = (int)gmembers.size() / 4;

  // ---- 2:4 metadata (block_online.cpp:669-703) ----
  S.covered.assign(ne, 0);
  W.s_mask.assign((size_t)ng * window, 0);
  W.s_val.assign((size_t)ng * window * 2, 0.f);
  W.s_pos.assign((size_t)ng * window * 2, (int8_t)-1);
  std::vector<uint8_t> kept(window);
  std::vector<int64_t> dropped;
  for (int g = 0; g < ng; ++g) {
    std::fill(kept.begin(), kept.end(), 0);
    for (int q = 0; q < 4; ++q) {
      const int u = gmembers[g * 4 + q];
      if (u < 0) continue;
      for (int32_t f = S.first_beg[u]; f < S.first_beg[u + 1]; ++f) {
        const int lr = S.first_lr[f];
        const size_t mi = (size_t)g * window + lr;
        W.s_mask[mi] |= (uint8_t)(1u << q);
        if (kept[lr] < 2) {
          W.s_val[mi * 2 + kept[lr]] = val[S.first_e[f]];
          W.s_pos[mi * 2 + kept[lr]] = (int8_t)q;
          S.covered[S.first_e[f] - e0] = 1;
        }
        kept[lr]++;
      }
    }
  }

  // ---- residual + TC part (block_online.cpp:705-733, 444-540) ----
  bool fallback = false;
  for (int u = 0; u < nu; ++u) if (S.status[u] == -1) { fallback = true; break; }
  const int nsub = (int)tc_groups.size();
  if (nsub > 0) {
    std::vector<uint64_t> lo(nsub, 0), hi(nsub, 0);
    std::vector<std::vector<float>> sv(nsub);
    for (int r = r0; r < r1; ++r) {
      const int lr = r - r0;
      for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
        const int32_t st = S.status[S.ecol[e - e0]];
        if (st < 0) continue;
        const int sub = st / 8, k = st % 8;
        if (lr >= 8) hi[sub] |= 1ull << (((lr - 8) * 8 + k) & 63);
        else lo[sub] |= 1ull << ((lr * 8 + k) & 63);
        sv[sub].push_back(val[e]);
        S.covered[e - e0] = 1;
      }
    }
    for (int s = 0; s < nsub; ++s) {
      for (int q = 0; q < 8; ++q)
        W.t_col.push_back(q < (int)tc_groups[s].size() ? S.ucol[tc_groups[s][q]] : -1);
      W.t_bin.push_back((int64_t)lo[s]);
      W.t_bin.push_back((int64_t)hi[s]);
      W.t_subcnt.push_back((int32_t)sv[s].size());
      W.t_val.insert(W.t_val.end(), sv[s].begin(), sv[s].end());
    }
    if (nsub <= P.part_t) {
      W.t_parts.push_back(nsub);
      W.t_atomic.push_back(fallback ? 1 : 0);
    } else {
      for (int q = 0; q < nsub / P.part_t; ++q) { W.t_parts.push_back(P.part_t); W.t_atomic.push_back(1); }
      if (nsub % P.part_t) { W.t_parts.push_back(nsub % P.part_t); W.t_atomic.push_back(1); }
    }
  }
  const int base_atomic = nsub > 0 ? 1 : 0;
  std::vector<int32_t> rc;
  std::vector<float> rv;
  for (int r = r0; r < r1; ++r) {
    rc.clear(); rv.clear();
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      if (S.status[S.ecol[e - e0]] != -1) continue;
      rc.push_back(col[e]); rv.push_back(val[e]);
      S.covered[e - e0] = 1;
    }
    split_residual_row(r, base_atomic, P, rc.data(), rv.data(), (int)rc.size(), W);
  }
  for (int r = r0; r < r1; ++r)
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e)
      if (!S.covered[e - e0]) { W.sp_row.push_back(r); W.sp_col.push_back(col[e]); W.sp_val.push_back(val[e]); }

  // ---- tiles of 4 groups (block_online.cpp:796-841) ----
  const int ntile = (ng + 3) / 4;
  W.tile_group.resize(ntile);
  W.tile_cols.resize((size_t)ntile * 16);
  W.packed_meta.resize((size_t)ntile * 8);
  W.packed_a.resize((size_t)ntile * 64);
  for (int ti = 0; ti < ntile; ++ti) {
    const int base = ti * 4;
    W.tile_group[ti] = base;
    for (int k = 0; k < 16; ++k) {
      const int g = base + k / 4;
      W.tile_cols[(size_t)ti * 16 + k] = g < ng ? W.s_col[g * 4 + k % 4] : -1;
    }
    for (int rg = 0; rg < 8; ++rg) {
      // per chunk c: the two values of row rg, then the two of row rg + 8 (one int32 word each,
      // low half first)
      float a[16];
      uint32_t meta = 0;
      for (int c = 0; c < 4; ++c) {
        int p0, p1;
        load_chunk(W, base + c, ng, rg, window, a[4 * c], a[4 * c + 1], p0, p1);
        meta |= ((uint32_t)(p0 & 3) | ((uint32_t)(p1 & 3) << 2)) << (4 * c);
        load_chunk(W, base + c, ng, rg + 8, window, a[4 * c + 2], a[4 * c + 3], p0, p1);
        meta |= ((uint32_t)(p0 & 3) | ((uint32_t)(p1 & 3) << 2)) << (16 + 4 * c);
      }
      W.packed_meta[(size_t)ti * 8 + rg] = (int32_t)meta;
      uint16_t h[16];
      trs::half_bits_n(a, h, 16);
      std::memcpy(&W.packed_a[((size_t)ti * 8 + rg) * 8], h, sizeof(h));
    }
  }
}

bool env_flag(const char* name, bool dflt) {   // block_online.cpp:118-122
  const char* v = std::getenv(name);
  if (!v) return dflt;
  return !std::strcmp(v, "1") || !std::strcmp(v, "true") || !std::strcmp(v, "TRUE");
}
int env_int(const char* name, int dflt) {       // block_online.cpp:124-128
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : dflt;
}

template <class T, class A, class B>
void append_at(std::vector<T, A>& dst, size_t at, const std::vector<T, B>& src) {
  if (!src.empty()) std::memcpy(dst.data() + at, src.data(), src.size() * sizeof(T));
}

}  // namespace

namespace trs {
uint16_t half_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  return half_bits_of(x);
}

namespace {
// 8 conversions with the x86 F16C instruction (IEEE round to nearest even, like half_bits_of for
// every input but NaN, whose payload the instruction keeps: those lanes are redone by
// half_bits_of).
__attribute__((target("avx,f16c"))) void half_bits8_f16c(const float* src, uint16_t* dst) {
  const __m256 x = _mm256_loadu_ps(src);
  _mm_storeu_si128(reinterpret_cast<__m128i*>(dst), _mm256_cvtps_ph(x, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
  const __m256 nan = _mm256_cmp_ps(x, x, _CMP_UNORD_Q);
  if (!_mm256_testz_ps(nan, nan))
    for (int i = 0; i < 8; ++i)
      if (src[i] != src[i]) dst[i] = half_bits(src[i]);
}
const bool has_f16c = __builtin_cpu_supports("f16c") && __builtin_cpu_supports("avx");
}  // namespace

void half_bits_n(const float* src, uint16_t* dst, int64_t n) {
  int64_t i = 0;
  if (has_f16c)
    for (; i + 8 <= n; i += 8) half_bits8_f16c(src + i, dst + i);
  for (; i < n; ++i) dst[i] = half_bits(src[i]);
}
}  // namespace trs

extern "C" {

void trs_build_params_default(trs_build_params* p) {
  if (!p) return;
  p->struct_size = (int32_t)sizeof(trs_build_params);
  // spmm/spmm_3090_fp16_test.py:30-40 defaults
  p->part_size_t = 32;
  p->part_size_c = 32;
  p->short_size = 3;
  p->density = 8;
  p->window = 16;
  p->wide = 16;
  p->tc_min_util = 0.0f;
  p->sptc_min_util = 0.5f;
  p->sptc_threshold = 12;
  p->skip_tc = -1;
  p->sptc_unit_min_nnz = -1;
  p->num_threads = 0;
}

int trs_build_online(const int32_t* rowptr, const int32_t* col, const float* val, int32_t rows,
                     int64_t nnz, const trs_build_params* prm, trs_format** out) {
  if (!out) { trs::set_error("trs_build_online: out is NULL"); return TRS_EINVAL; }
  *out = nullptr;
  if (!prm) { trs::set_error("trs_build_online: params is NULL"); return TRS_EINVAL; }
  if (prm->struct_size != (int32_t)sizeof(trs_build_params)) {
    trs::set_error("trs_build_online: trs_build_params.struct_size is " + std::to_string(prm->struct_size) +
                   ", this library's is " + std::to_string(sizeof(trs_build_params)) +
                   " (initialise the parameters with trs_build_params_default of the same trspmm.h)");
    return TRS_EINVAL;
  }
  // block_online.cpp:551-553
  if (!(prm->window > 0 && prm->window <= 32 && prm->wide > 0 && prm->wide <= 32)) {
    trs::set_error("trs_build_online: requires 0 < window <= 32 and 0 < wide <= 32");
    return TRS_EINVAL;
  }
  if (rows < 0 || !rowptr || (nnz > 0 && (!col || !val))) {
    trs::set_error("trs_build_online: bad CSR arguments");
    return TRS_EINVAL;
  }
  if (rowptr[0] != 0 || (int64_t)rowptr[rows] != nnz) {
    trs::set_error("trs_build_online: rowptr must start at 0 and end at nnz");
    return TRS_EINVAL;
  }
  for (int32_t r = 0; r < rows; ++r)
    if (rowptr[r + 1] < rowptr[r]) { trs::set_error("trs_build_online: rowptr must be non-decreasing"); return TRS_EINVAL; }
  for (int64_t e = 0; e < nnz; ++e)
    if (col[e] < 0) { trs::set_error("trs_build_online: negative column index"); return TRS_EINVAL; }

  const auto t0 = std::chrono::high_resolution_clock::now();
  Params P;
  P.part_t = prm->part_size_t;
  P.part_c = prm->part_size_c;
  P.short_size = prm->short_size;
  P.density = prm->density;
  P.window = prm->window;
  P.tc_min_util = prm->tc_min_util;
  P.skip_tc = prm->skip_tc >= 0 ? (prm->skip_tc != 0) : env_flag("LIBRA_SKIP_TC", false);
  P.unit_min_nnz = prm->sptc_unit_min_nnz >= 0 ? prm->sptc_unit_min_nnz : env_int("LIBRA_SPTC_UNIT_MIN_NNZ", 2);
  if (P.part_t <= 0 || P.part_c <= 0) {
    trs::set_error("trs_build_online: partSize_t and partSize_c must be positive");
    return TRS_EINVAL;
  }

  const int nwin = (rows + P.window - 1) / P.window;
  const int nthreads = prm->num_threads > 0 ? prm->num_threads : omp_get_max_threads();
  // declared before the windows, so that windows still held on an early return are destroyed
  // while their arenas exist
  std::vector<std::unique_ptr<std::pmr::monotonic_buffer_resource>> arena(nthreads);
  std::vector<std::optional<Win>> wins(nwin);
#pragma omp parallel num_threads(nthreads)
  {
    Scratch S;
    auto& a = arena[omp_get_thread_num()];
    a = std::make_unique<std::pmr::monotonic_buffer_resource>(size_t(4) << 20);
#pragma omp for schedule(dynamic, 16)
    for (int w = 0; w < nwin; ++w) {
      wins[w].emplace(a.get());
      build_window(rowptr, col, val, rows, w, P, S, *wins[w]);
    }
  }

  // ---- serialisation in window order (block_online.cpp:736-776, 789-794, 840, 844-870) ----
  trs_format* F = new trs_format();
  F->rows = rows;
  F->window = P.window;
  struct Off { size_t parts, subs, tval, cl, clv, cs, csv, g, tiles, sp; };
  std::vector<Off> off(nwin + 1);
  off[0] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  bool canonical = true;
  for (int w = 0; w < nwin; ++w) {
    const Win& W = *wins[w];
    Off o = off[w];
    o.parts += W.t_parts.size();
    o.subs += W.t_subcnt.size();
    o.tval += W.t_val.size();
    o.cl += W.lng.cnt.size();
    o.clv += W.lng.col.size();
    o.cs += W.sht.cnt.size();
    o.csv += W.sht.col.size();
    o.g += W.s_col.size() / 4;
    o.tiles += W.tile_group.size();
    o.sp += W.sp_row.size();
    off[w + 1] = o;
    canonical = canonical && W.canonical;
  }
  F->canonical = canonical;
  const Off& T = off[nwin];
  if (T.subs > (size_t)INT32_MAX || T.g > (size_t)INT32_MAX / 32 || T.tiles > (size_t)INT32_MAX / 64) {
    delete F;
    trs::set_error("trs_build_online: output exceeds int32 index range");
    return TRS_ERANGE;
  }
  try {
    F->t_rowoff.resize(T.parts + 1); F->t_blockoff.resize(T.subs + 1); F->t_col.resize(T.subs * 8);
    F->t_val.resize(T.tval); F->t_winrow.resize(T.parts); F->t_atomic.resize(T.parts); F->t_bin.resize(T.subs * 2);
    F->c_off.resize(T.cl + 1); F->c_row.resize(T.cl); F->c_atomic.resize(T.cl); F->c_col.resize(T.clv); F->c_val.resize(T.clv);
    F->cs_off.resize(T.cs + 1); F->cs_row.resize(T.cs); F->cs_atomic.resize(T.cs); F->cs_col.resize(T.csv); F->cs_val.resize(T.csv);
    F->s_col.resize(T.g * 4); F->s_mask.resize(T.g * P.window); F->s_val.resize(T.g * P.window * 2);
    F->s_pos.resize(T.g * P.window * 2); F->s_win.resize(T.g); F->s_offsets.resize(nwin + 1);
    F->tile_win.resize(T.tiles); F->tile_group.resize(T.tiles); F->tile_cols.resize(T.tiles * 16);
    F->packed_a.resize(T.tiles * 64); F->packed_meta.resize(T.tiles * 8); F->win_tile_off.resize(nwin + 1);
    F->spill_row.resize(T.sp); F->spill_col.resize(T.sp); F->spill_val.resize(T.sp);
  } catch (const std::bad_alloc&) {
    delete F;
    trs::set_error("trs_build_online: out of host memory");
    return TRS_ENOMEM;
  }
  F->t_rowoff[0] = 0; F->t_blockoff[0] = 0; F->c_off[0] = 0; F->cs_off[0] = 0;
  for (int w = 0; w <= nwin; ++w) {
    F->s_offsets[w] = (int32_t)off[w].g;
    F->win_tile_off[w] = (int32_t)off[w].tiles;
  }
#pragma omp parallel for schedule(dynamic, 64) num_threads(nthreads)
  for (int w = 0; w < nwin; ++w) {
    const Win& W = *wins[w];
    const Off& o = off[w];
    // TC
    int32_t acc = (int32_t)o.subs;
    for (size_t i = 0; i < W.t_parts.size(); ++i) {
      acc += W.t_parts[i];
      F->t_rowoff[o.parts + 1 + i] = acc;
      F->t_winrow[o.parts + i] = w * 16;   // block_online.cpp:494 (window id * 16 for every window size)
      F->t_atomic[o.parts + i] = W.t_atomic[i];
    }
    int32_t vacc = (int32_t)o.tval;
    for (size_t i = 0; i < W.t_subcnt.size(); ++i) {
      vacc += W.t_subcnt[i];
      F->t_blockoff[o.subs + 1 + i] = vacc;
    }
    append_at(F->t_col, o.subs * 8, W.t_col);
    append_at(F->t_val, o.tval, W.t_val);
    append_at(F->t_bin, o.subs * 2, W.t_bin);
    // residual
    int32_t c = (int32_t)o.clv;
    for (size_t i = 0; i < W.lng.cnt.size(); ++i) { c += W.lng.cnt[i]; F->c_off[o.cl + 1 + i] = c; }
    append_at(F->c_row, o.cl, W.lng.row); append_at(F->c_atomic, o.cl, W.lng.atomic);
    append_at(F->c_col, o.clv, W.lng.col); append_at(F->c_val, o.clv, W.lng.val);
    c = (int32_t)o.csv;
    for (size_t i = 0; i < W.sht.cnt.size(); ++i) { c += W.sht.cnt[i]; F->cs_off[o.cs + 1 + i] = c; }
    append_at(F->cs_row, o.cs, W.sht.row); append_at(F->cs_atomic, o.cs, W.sht.atomic);
    append_at(F->cs_col, o.csv, W.sht.col); append_at(F->cs_val, o.csv, W.sht.val);
    // SPTC
    append_at(F->s_col, o.g * 4, W.s_col);
    append_at(F->s_mask, o.g * P.window, W.s_mask);
    append_at(F->s_val, o.g * P.window * 2, W.s_val);
    append_at(F->s_pos, o.g * P.window * 2, W.s_pos);
    for (size_t i = 0; i < W.s_col.size() / 4; ++i) F->s_win[o.g + i] = w;
    for (size_t i = 0; i < W.tile_group.size(); ++i) {
      F->tile_win[o.tiles + i] = w;
      F->tile_group[o.tiles + i] = (int32_t)o.g + W.tile_group[i];
    }
    append_at(F->tile_cols, o.tiles * 16, W.tile_cols);
    append_at(F->packed_a, o.tiles * 64, W.packed_a);
    append_at(F->packed_meta, o.tiles * 8, W.packed_meta);
    append_at(F->spill_row, o.sp, W.sp_row); append_at(F->spill_col, o.sp, W.sp_col);
    append_at(F->spill_val, o.sp, W.sp_val);
    wins[w].reset();
  }
  // keep the input CSR for device-side plan lowering (counted in the build time)
  if (canonical) {
    try {
      F->csr_rowptr.assign(rowptr, rowptr + (size_t)rows + 1);
      F->csr_col.resize((size_t)nnz);
      F->csr_val.resize((size_t)nnz);
    } catch (const std::bad_alloc&) {
      F->csr_rowptr.clear(); F->csr_col.clear(); F->csr_val.clear();
      F->csr_col.shrink_to_fit(); F->csr_val.shrink_to_fit();
      F->elapsed = std::chrono::duration<double>(std::chrono::high_resolution_clock::now() - t0).count();
      *out = F;
      return TRS_OK;   // the plan then lowers on the host
    }
    const int64_t chunk = 1 << 20;
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t b = 0; b < nnz; b += chunk) {
      const int64_t e = std::min<int64_t>(nnz, b + chunk);
      std::memcpy(F->csr_col.data() + b, col + b, (size_t)(e - b) * sizeof(int32_t));
      std::memcpy(F->csr_val.data() + b, val + b, (size_t)(e - b) * sizeof(float));
    }
  }
  F->elapsed = std::chrono::duration<double>(std::chrono::high_resolution_clock::now() - t0).count();
  *out = F;
  return TRS_OK;
}

int trs_format_slot(const trs_format* F, int32_t slot, const void** data, int64_t* numel) {
  if (!F || !data || !numel) { trs::set_error("trs_format_slot: NULL argument"); return TRS_EINVAL; }
#define TRS_SLOT(v) do { *data = (v).data(); *numel = (int64_t)(v).size(); return TRS_OK; } while (0)
  switch (slot) {
    case 0: TRS_SLOT(F->t_rowoff); case 1: TRS_SLOT(F->t_blockoff); case 2: TRS_SLOT(F->t_col);
    case 3: TRS_SLOT(F->t_val); case 4: TRS_SLOT(F->t_winrow); case 5: TRS_SLOT(F->t_atomic);
    case 6: TRS_SLOT(F->t_bin); case 7: TRS_SLOT(F->c_off); case 8: TRS_SLOT(F->c_row);
    case 9: TRS_SLOT(F->c_atomic); case 10: TRS_SLOT(F->c_col); case 11: TRS_SLOT(F->c_val);
    case 12: TRS_SLOT(F->cs_off); case 13: TRS_SLOT(F->cs_row); case 14: TRS_SLOT(F->cs_atomic);
    case 15: TRS_SLOT(F->cs_col); case 16: TRS_SLOT(F->cs_val); case 17: TRS_SLOT(F->s_col);
    case 18: TRS_SLOT(F->s_mask); case 19: TRS_SLOT(F->s_val); case 20: TRS_SLOT(F->s_pos);
    case 21: TRS_SLOT(F->s_win); case 22: TRS_SLOT(F->s_offsets); case 23: TRS_SLOT(F->tile_win);
    case 24: TRS_SLOT(F->tile_group); case 25: TRS_SLOT(F->tile_cols); case 26: TRS_SLOT(F->packed_a);
    case 27: TRS_SLOT(F->packed_meta); case 28: TRS_SLOT(F->win_tile_off);
    case 29: TRS_SLOT(F->spill_row); case 30: TRS_SLOT(F->spill_col); case 31: TRS_SLOT(F->spill_val);
    default: break;
  }
#undef TRS_SLOT
  trs::set_error("trs_format_slot: slot out of range 0..31");
  return TRS_EINVAL;
}

double trs_format_elapsed(const trs_format* F) { return F ? F->elapsed : 0.0; }
int32_t trs_format_window(const trs_format* F) { return F ? F->window : 0; }
int32_t trs_format_rows(const trs_format* F) { return F ? F->rows : 0; }
int32_t trs_format_canonical(const trs_format* F) { return F && F->canonical ? 1 : 0; }
void trs_format_free(trs_format* F) { delete F; }

}  // extern "C"
