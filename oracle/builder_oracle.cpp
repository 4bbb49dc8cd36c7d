// TEST INFRASTRUCTURE ONLY -- never linked into, loaded by, or called from the product.
//
// Literal CPU restatement of the reference "online" format builder
// (TR-source/Block/block_online.cpp:545-871, `block_sptc_2to4_online`), kept deliberately naive:
// an explicit O(n^2) compatibility graph per window and libstdc++ std::sort with the reference's
// comparators, so that the tie order of the non-total unit sort (block_online.cpp:358-363) comes out
// the same.  It additionally records every input edge that no output array carries (the "spill",
// values the 2:4 step drops), which the reference does not report.
//
// Pinned by: tests/test_oracle_builder.py (bit-exact against the committed golden fixtures written
// by the compiled reference, and against oracle/_ref directly when it is built), plus partition
// invariants (TC + SPTC-kept + CUDA + spill == input multiset).
//
// Slot numbering follows the reference return list (block_online.cpp:844-870); slots 29..31 are the
// spill rows / columns / values (CSR edge order).
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <numeric>
#include <vector>

namespace {

struct Column {            // per distinct column of a window (block_online.cpp:20-25, 588-603)
  int count = 0;
  uint32_t vec = 0;        // 2-bit count per local row
  std::vector<std::pair<int, int64_t>> first;  // (local_row, edge) first occurrence per row
};

struct Unit {              // block_online.cpp:28-34
  int c1 = -1, c2 = -1;
  uint32_t vec = 0;
  int nnz = 0;
};

bool compatible(uint32_t a, uint32_t b) {   // block_online.cpp:83-88
  uint32_t c = a | b;
  return (((a & b) | ((c << 1) & c)) & 0xaaaaaaaau) == 0;
}

uint16_t half_bits(float f) {  // IEEE binary16, round to nearest even
  uint32_t x; std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);       // NaN
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);      // overflow / inf
  if (ax < 0x38800000u) {                                        // subnormal half or zero
    // value = ax as float; half subnormal unit is 2^-24
    float a; std::memcpy(&a, &ax, 4);
    double scaled = (double)a * 16777216.0;                      // exact in double
    double fl = (double)(int64_t)scaled;
    double rem = scaled - fl;
    int64_t q = (int64_t)fl;
    if (rem > 0.5 || (rem == 0.5 && (q & 1))) q++;
    return (uint16_t)(sign | (uint32_t)q);
  }
  uint32_t e = (ax >> 23) - 127 + 15;
  uint32_t m = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  uint32_t rest = m & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1))) h++;
  return (uint16_t)(sign | h);
}

struct Out {
  std::vector<int32_t> t_rowoff{0}, t_blockoff{0}, t_col, t_winrow, t_atomic;
  std::vector<float> t_val;
  std::vector<int64_t> t_bin;
  std::vector<int32_t> c_off{0}, c_row, c_atomic, c_col;
  std::vector<float> c_val;
  std::vector<int32_t> cs_off{0}, cs_row, cs_atomic, cs_col;
  std::vector<float> cs_val;
  std::vector<int32_t> s_col, s_win, s_offsets{0};
  std::vector<uint8_t> s_mask;
  std::vector<float> s_val;
  std::vector<int8_t> s_pos;
  std::vector<int32_t> tile_win, tile_group, tile_cols, packed_a, packed_meta, win_tile_off{0};
  std::vector<int32_t> spill_row, spill_col;
  std::vector<float> spill_val;
  float elapsed = 0.f;
};

struct CudaPart { int row, atomic; std::vector<int32_t> cols; std::vector<float> vals; };

// block_online.cpp:397-439
void split_row(int row, int base_atomic, int part, int shrt, const std::vector<int32_t>& cols,
               const std::vector<float>& vals, std::vector<CudaPart>& lng, std::vector<CudaPart>& sht) {
  int n = (int)cols.size();
  auto emit = [&](int atomic, int off, int cnt, bool is_short) {
    CudaPart p{row, atomic, {cols.begin() + off, cols.begin() + off + cnt},
               {vals.begin() + off, vals.begin() + off + cnt}};
    (is_short ? sht : lng).push_back(std::move(p));
  };
  if (n <= 0) return;
  if (n <= shrt) { emit(base_atomic, 0, n, true); return; }
  if (n <= part) { emit(base_atomic, 0, n, false); return; }
  int full = n / part, off = 0;
  for (int i = 0; i < full; ++i, off += part) emit(1, off, part, false);
  int rem = n % part;
  if (rem > 0) emit(1, off, rem, rem <= shrt);
}

}  // namespace

extern "C" {

void* orc_build(const int32_t* rowptr, const int32_t* col, const float* val, int32_t rows,
                int32_t part_t, int32_t part_c, int32_t short_size, int32_t density, int32_t window,
                float tc_min_util, int32_t skip_tc, int32_t unit_min_nnz) {
  if (window <= 0 || window > 32) return nullptr;
  Out* o = new Out();
  const int nwin = (rows + window - 1) / window;
  std::vector<uint8_t> covered(rows > 0 ? rowptr[rows] : 0, 0);

  for (int w = 0; w < nwin; ++w) {
    const int r0 = w * window, r1 = std::min(r0 + window, rows);
    std::map<int, Column> info;
    for (int r = r0; r < r1; ++r) {
      const int lr = r - r0;
      std::vector<int> seen;
      for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
        int c = col[e];
        if (std::find(seen.begin(), seen.end(), c) != seen.end()) continue;
        seen.push_back(c);
        Column& ci = info[c];
        ci.count++;
        ci.vec += 1u << ((2 * lr) & 31);     // x86 shift-count masking for window > 16
        ci.first.push_back({lr, e});
      }
    }
    auto by_count = [&](int a, int b) {
      int ca = info[a].count, cb = info[b].count;
      return ca != cb ? ca > cb : a < b;
    };

    // Stage 1: TC columns (block_online.cpp:215-253), chunk width fixed at 8 (:611)
    std::vector<std::vector<int>> tc_groups;
    std::map<int, int> tc_slot;  // column -> block*8 + pos
    if (!skip_tc) {
      std::vector<int> cand;
      for (auto& kv : info) if (kv.second.count >= density) cand.push_back(kv.first);
      std::sort(cand.begin(), cand.end(), by_count);
      for (size_t s = 0; s < cand.size(); s += 8) {
        size_t e = std::min(s + 8, cand.size());
        int nnz = 0;
        std::vector<int> g;
        for (size_t i = s; i < e; ++i) { nnz += info[cand[i]].count; g.push_back(cand[i]); }
        float util = (float)nnz / (float)(window * 8);
        if (util < tc_min_util) continue;
        std::sort(g.begin(), g.end());
        tc_groups.push_back(g);
      }
      for (size_t b = 0; b < tc_groups.size(); ++b)
        for (size_t p = 0; p < tc_groups[b].size(); ++p) tc_slot[tc_groups[b][p]] = (int)(b * 8 + p);
    }

    // Stage 2a: units (block_online.cpp:267-328)
    std::vector<int> cand;
    for (auto& kv : info) if (!tc_slot.count(kv.first)) cand.push_back(kv.first);
    std::sort(cand.begin(), cand.end(), by_count);
    std::vector<Unit> units;
    std::vector<char> used(cand.size(), 0);
    for (size_t i = 0; i < cand.size(); ++i) {
      if (used[i]) continue;
      used[i] = 1;
      Unit u; u.c1 = cand[i]; u.vec = info[cand[i]].vec; u.nnz = info[cand[i]].count;
      for (size_t j = i + 1; j < cand.size(); ++j) {
        if (used[j] || !compatible(u.vec, info[cand[j]].vec)) continue;
        used[j] = 1; u.c2 = cand[j]; u.vec |= info[cand[j]].vec; u.nnz += info[cand[j]].count;
        break;
      }
      units.push_back(u);
    }

    // Stage 2b: max-degree greedy matching on the explicit graph (block_online.cpp:332-392)
    const int n = (int)units.size();
    std::vector<std::vector<int>> adj(n);
    std::vector<int> deg(n, 0);
    for (int i = 0; i < n; ++i)
      for (int j = i + 1; j < n; ++j)
        if (compatible(units[i].vec, units[j].vec)) {
          adj[i].push_back(j); adj[j].push_back(i); deg[i]++; deg[j]++;
        }
    std::vector<int> order(n);
    std::iota(order.begin(), order.end(), 0);
    std::sort(order.begin(), order.end(), [&](int a, int b) {
      if (deg[a] != deg[b]) return deg[a] > deg[b];
      return units[a].nnz > units[b].nnz;
    });
    std::vector<char> matched(n, 0);
    std::vector<std::pair<int, int>> pairs;
    for (int idx : order) {
      if (matched[idx]) continue;
      int best = -1, bdeg = -1;
      for (int nb : adj[idx]) {
        if (matched[nb]) continue;
        if (deg[nb] > bdeg || (deg[nb] == bdeg && units[nb].nnz > units[best].nnz)) { best = nb; bdeg = deg[nb]; }
      }
      if (best >= 0) { matched[idx] = matched[best] = 1; pairs.push_back({idx, best}); }
    }

    // Stage 2c: groups (block_online.cpp:629-666)
    std::map<int, int> in_sptc;
    const int g_begin = (int)o->s_win.size();
    auto emit_group = [&](std::vector<int> g) {
      std::sort(g.begin(), g.end());
      for (int c : g) in_sptc[c] = 1;
      while (g.size() < 4) g.push_back(-1);
      o->s_win.push_back(w);
      o->s_col.insert(o->s_col.end(), g.begin(), g.end());
    };
    for (auto& pr : pairs) {
      const Unit& a = units[pr.first];
      const Unit& b = units[pr.second];
      std::vector<int> g{a.c1};
      if (a.c2 >= 0) g.push_back(a.c2);
      g.push_back(b.c1);
      if (b.c2 >= 0) g.push_back(b.c2);
      emit_group(g);
    }
    for (int i = 0; i < n; ++i) {
      if (matched[i] || units[i].nnz < unit_min_nnz) continue;
      std::vector<int> g{units[i].c1};
      if (units[i].c2 >= 0) g.push_back(units[i].c2);
      emit_group(g);
    }

    // Stage 2d: per-row 2:4 metadata (block_online.cpp:669-703)
    for (int g = g_begin; g < (int)o->s_win.size(); ++g) {
      for (int lr = 0; lr < window; ++lr) {
        uint8_t mask = 0;
        int kept = 0;
        float v[2] = {0.f, 0.f};
        int8_t p[2] = {-1, -1};
        for (int q = 0; q < 4; ++q) {
          int c = o->s_col[g * 4 + q];
          if (c < 0) continue;
          const auto& fr = info[c].first;
          auto it = std::find_if(fr.begin(), fr.end(), [&](const std::pair<int, int64_t>& x) { return x.first == lr; });
          if (it == fr.end()) continue;
          mask |= (uint8_t)(1u << q);
          if (kept < 2) { v[kept] = val[it->second]; p[kept] = (int8_t)q; covered[it->second] = 1; }
          kept++;
        }
        o->s_mask.push_back(mask);
        o->s_val.push_back(v[0]); o->s_val.push_back(v[1]);
        o->s_pos.push_back(p[0]); o->s_pos.push_back(p[1]);
      }
    }
    o->s_offsets.push_back((int32_t)o->s_win.size());

    // Stage 3: residual (block_online.cpp:705-733)
    bool fallback = false;
    for (auto& kv : info) if (!tc_slot.count(kv.first) && !in_sptc.count(kv.first)) fallback = true;

    // TC part (block_online.cpp:444-540)
    if (!tc_groups.empty()) {
      const int nsub = (int)tc_groups.size();
      std::vector<uint64_t> lo(nsub, 0), hi(nsub, 0);
      std::vector<std::vector<float>> sv(nsub);
      for (int r = r0; r < r1; ++r) {
        const int lr = r - r0;
        for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
          auto it = tc_slot.find(col[e]);
          if (it == tc_slot.end()) continue;
          int sub = it->second / 8, k = it->second % 8;
          if (lr >= 8) hi[sub] |= 1ull << (((lr - 8) * 8 + k) & 63);
          else lo[sub] |= 1ull << ((lr * 8 + k) & 63);
          sv[sub].push_back(val[e]);
          covered[e] = 1;
        }
      }
      for (int s = 0; s < nsub; ++s) {
        for (int q = 0; q < 8; ++q) o->t_col.push_back(q < (int)tc_groups[s].size() ? tc_groups[s][q] : -1);
        o->t_bin.push_back((int64_t)lo[s]);
        o->t_bin.push_back((int64_t)hi[s]);
        o->t_val.insert(o->t_val.end(), sv[s].begin(), sv[s].end());
      }
      auto add_part = [&](int first, int cnt, int atomic) {
        o->t_rowoff.push_back(o->t_rowoff.back() + cnt);
        for (int b = first; b < first + cnt; ++b) o->t_blockoff.push_back(o->t_blockoff.back() + (int)sv[b].size());
        o->t_winrow.push_back(w * 16);
        o->t_atomic.push_back(atomic);
      };
      if (nsub <= part_t) add_part(0, nsub, fallback ? 1 : 0);
      else {
        int full = nsub / part_t;
        for (int q = 0; q < full; ++q) add_part(q * part_t, part_t, 1);
        if (nsub % part_t) add_part(full * part_t, nsub % part_t, 1);
      }
    }

    std::vector<CudaPart> lng, sht;
    const int base_atomic = tc_slot.empty() ? 0 : 1;
    for (int r = r0; r < r1; ++r) {
      std::vector<int32_t> cc; std::vector<float> cv;
      for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
        if (tc_slot.count(col[e]) || in_sptc.count(col[e])) continue;
        cc.push_back(col[e]); cv.push_back(val[e]); covered[e] = 1;
      }
      split_row(r, base_atomic, part_c, short_size, cc, cv, lng, sht);
    }
    for (auto& p : lng) {
      o->c_off.push_back(o->c_off.back() + (int)p.cols.size());
      o->c_row.push_back(p.row); o->c_atomic.push_back(p.atomic);
      o->c_col.insert(o->c_col.end(), p.cols.begin(), p.cols.end());
      o->c_val.insert(o->c_val.end(), p.vals.begin(), p.vals.end());
    }
    for (auto& p : sht) {
      o->cs_off.push_back(o->cs_off.back() + (int)p.cols.size());
      o->cs_row.push_back(p.row); o->cs_atomic.push_back(p.atomic);
      o->cs_col.insert(o->cs_col.end(), p.cols.begin(), p.cols.end());
      o->cs_val.insert(o->cs_val.end(), p.vals.begin(), p.vals.end());
    }
  }

  // Tile packing (block_online.cpp:796-841, 178-210)
  auto chunk = [&](int g, int gend, int lr, float& v0, float& v1, int& p0, int& p1) {
    v0 = v1 = 0.f; p0 = 0; p1 = 1;
    if (g >= gend || lr >= window) return;
    size_t b = ((size_t)g * window + lr) * 2;
    int q0 = o->s_pos[b], q1 = o->s_pos[b + 1];
    float a0 = o->s_val[b], a1 = o->s_val[b + 1];
    if (q0 < 0 && q1 < 0) return;
    if (q0 >= 0 && q1 >= 0) {
      if (q0 <= q1) { p0 = q0; p1 = q1; v0 = a0; v1 = a1; } else { p0 = q1; p1 = q0; v0 = a1; v1 = a0; }
      return;
    }
    int rp = q0 >= 0 ? q0 : q1;
    float rv = q0 >= 0 ? a0 : a1;
    int dummy = rp == 0 ? 1 : 0;
    if (dummy < rp) { p0 = dummy; p1 = rp; v0 = 0.f; v1 = rv; } else { p0 = rp; p1 = dummy; v0 = rv; v1 = 0.f; }
  };
  auto pack = [](float lo, float hi) { return (int32_t)((uint32_t)half_bits(lo) | ((uint32_t)half_bits(hi) << 16)); };
  for (int w = 0; w < nwin; ++w) {
    int gb = o->s_offsets[w], ge = o->s_offsets[w + 1];
    for (int base = gb; base < ge; base += 4) {
      o->tile_win.push_back(w);
      o->tile_group.push_back(base);
      for (int k = 0; k < 16; ++k) {
        int g = base + k / 4;
        o->tile_cols.push_back(g < ge ? o->s_col[g * 4 + k % 4] : -1);
      }
      for (int rg = 0; rg < 8; ++rg) {
        float a0[8], a1[8];
        uint32_t meta = 0;
        for (int c = 0; c < 4; ++c) {
          float v0, v1; int p0, p1;
          chunk(base + c, ge, rg, v0, v1, p0, p1);
          a0[2 * c] = v0; a0[2 * c + 1] = v1;
          meta |= ((uint32_t)(p0 & 3) | ((uint32_t)(p1 & 3) << 2)) << (4 * c);
          chunk(base + c, ge, rg + 8, v0, v1, p0, p1);
          a1[2 * c] = v0; a1[2 * c + 1] = v1;
          meta |= ((uint32_t)(p0 & 3) | ((uint32_t)(p1 & 3) << 2)) << (16 + 4 * c);
        }
        o->packed_meta.push_back((int32_t)meta);
        for (int t = 0; t < 4; ++t) {
          o->packed_a.push_back(pack(a0[2 * t], a0[2 * t + 1]));
          o->packed_a.push_back(pack(a1[2 * t], a1[2 * t + 1]));
        }
      }
    }
    o->win_tile_off.push_back((int32_t)o->tile_win.size());
  }

  for (int r = 0; r < rows; ++r)
    for (int64_t e = rowptr[r]; e < rowptr[r + 1]; ++e)
      if (!covered[e]) { o->spill_row.push_back(r); o->spill_col.push_back(col[e]); o->spill_val.push_back(val[e]); }
  return o;
}

static const void* slot_ptr(Out* o, int s, int64_t* n) {
#define S(v) do { *n = (int64_t)(v).size(); return (v).data(); } while (0)
  switch (s) {
    case 0: S(o->t_rowoff); case 1: S(o->t_blockoff); case 2: S(o->t_col); case 3: S(o->t_val);
    case 4: S(o->t_winrow); case 5: S(o->t_atomic); case 6: S(o->t_bin);
    case 7: S(o->c_off); case 8: S(o->c_row); case 9: S(o->c_atomic); case 10: S(o->c_col); case 11: S(o->c_val);
    case 12: S(o->cs_off); case 13: S(o->cs_row); case 14: S(o->cs_atomic); case 15: S(o->cs_col); case 16: S(o->cs_val);
    case 17: S(o->s_col); case 18: S(o->s_mask); case 19: S(o->s_val); case 20: S(o->s_pos);
    case 21: S(o->s_win); case 22: S(o->s_offsets); case 23: S(o->tile_win); case 24: S(o->tile_group);
    case 25: S(o->tile_cols); case 26: S(o->packed_a); case 27: S(o->packed_meta); case 28: S(o->win_tile_off);
    case 29: S(o->spill_row); case 30: S(o->spill_col); case 31: S(o->spill_val);
  }
#undef S
  *n = -1;
  return nullptr;
}

int64_t orc_len(void* h, int slot) { int64_t n; slot_ptr((Out*)h, slot, &n); return n; }
const void* orc_ptr(void* h, int slot) { int64_t n; return slot_ptr((Out*)h, slot, &n); }
void orc_free(void* h) { delete (Out*)h; }
uint16_t orc_half_bits(float f) { return half_bits(f); }

}  // extern "C"
