// Plans: lower format arrays to the device layout the kernels read, validate, upload once.
//
// Meaning of the arrays (the semantics every lowering below follows):
//   TC sub-block s of part p (TR-source/SpMM/mGCNkernel_online.cu:54-241): rows t_window_row[p] +
//     0..15, columns t_column[8s .. 8s+7] (-1 = empty); bit (r*8 + k) of t_binary[2s] (rows 0-7)
//     or t_binary[2s+1] (rows 8-15) marks a stored value; values sit at t_blockNew_offset[s] in
//     ascending bit order, the rows 8-15 after the rows 0-7.
//   2:4 group g (mGCNkernel_online.cu:248-337): rows window_of(g) * window + lr, up to two values
//     s_value[g][lr][q] at columns s_column[g][s_pos[g][lr][q]] (pos -1 = empty).
//   packed tile t (block_online.cpp:796-841, mGCNkernel_online.cu:812-933): rows w*window + rg and
//     + rg + 8; chunk c holds two fp16 values (s_packed_a) at 2-bit positions (s_packed_meta) of
//     columns s_tile_column[t][4c .. 4c+3].
//   residual part i (mGCNkernel.cu:976-1171): row c_row[i], entries c_row_offsets[i] .. [i+1].
// Output rows >= m are dropped, as the reference kernels guard `row < mOri`.  Column indices must
// lie in [0, n): the reference reads out of bounds there, this library rejects the plan instead.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <numeric>
#include <string>
#include <thread>
#include <vector>

#include "dformat.hpp"
#include "format.hpp"
#include "kernels.hpp"

namespace {
thread_local std::string g_error;
}

namespace trs {
void set_error(const std::string& msg) { g_error = msg; }
}  // namespace trs

struct trs_plan {
  trs::DevicePlan dp;
  void* dmem = nullptr;
  void* hmem = nullptr;   // hot-row staging: renumbered column ids and the hot column list
  size_t dbytes = 0;
  int device = 0;
  bool csr_only = false;
  trs_plan_stats stats{};
  ~trs_plan() {
    if (dmem) (void)hipFree(dmem);
    if (hmem) (void)hipFree(hmem);
  }
};

namespace {

struct Status {
  int code = TRS_OK;
  std::string msg;
  bool ok() const { return code == TRS_OK; }
};

Status fail(int code, const std::string& m) { return Status{code, m}; }

// Internal status of the device lowering: the format's tiles and its input CSR disagree (a tile
// entry the CSR does not hold, or two tiles holding one entry) or its temporaries could not be
// allocated; the caller then lowers on the host.
constexpr int kLowerOnHost = -100;

// Default XCD column split thresholds (rows with at least this many residual entries).  SpMM, R-MAT
// 2^20 step at K = 32 / 64 / 128 / 256: -16% / -6% / -18% / -19% against no split (128 and 512
// entries measured slower at K = 128).  SDDMM, K = 128 / 256: -14% / -20% (its launcher keeps the
// unsplit layout below K = 128, where the split measured slower: K = 32 / 64 / 96 +65% / +20% / +8%).
constexpr int32_t kSpmmSplitMin = 256;
constexpr int32_t kSddmmSplitMin = 512;
// ... and only when those rows' entries are at least this many times their distinct columns:
// R-MAT's rows of >= 256 entries gather 20.0M times from 0.60M columns (33x), the 64 hubs of the
// grid+hubs graph 6.4M times from 3.3M columns (1.9x), where the split measured +9% at K = 128
// (1.144 -> 1.249 ms) and +3% at K = 64.
constexpr int32_t kSplitMinReuse = 4;

// A tile-owning window goes back to the residual kernel when its longest residual row exceeds
// window_row_cap and this many times the mean of its rows: the window kernel walks each row with
// one lane group, so only a row far longer than its neighbours stalls the workgroup (R-MAT hub
// windows).  Windows of uniformly long rows keep their tiles: a block graph of 2048-node
// communities (p_in 0.2, 54.7M entries, ~280 residual entries in every row) ran at 0.924 / 2.082 ms
// (K = 128 / 256) with every window handed back under the length rule alone, 0.796 / 1.473 ms with
// this one; R-MAT, SBM and grid+hubs plans are unchanged (ratio 4 measured the same as 2).
constexpr int32_t kWindowRowRatio = 2;
// ... and whatever its neighbours, when that row is longer than this many times window_row_cap:
// windows of 16 uniformly long hub rows, which a row reorder (TCA) puts together on power-law
// graphs, each walked by one lane group (R-MAT 2^20 reordered, K = 128: 5.44 ms with such windows
// kept; the task kernel cuts those rows into pieces and XCD sub-rows instead).
constexpr int64_t kWindowRowHardFactor = 4;

// Hot-row staging (option hot_rows = 0): the kHotRows most gathered columns of the task kernels,
// at most one in kHotColumnShare of all columns, and only when they take at least
// kHotMinShare10 / 10 of the gathers.  R-MAT 2^20 (16,384 rows, 56.7% of the entries), K = 128:
// 0.741 -> 0.699 ms per step plus ~0.007 ms for the copy; 4,096 rows 0.709, 65,536 rows 0.694
// (+0.017 copy).  With 4 entries per batch in the task kernel, same box, twice each, 16,384 /
// 32,768 / 65,536 rows: SpMM K = 128 0.615 / 0.609-0.612 / 0.612-0.613 ms, K = 256 1.265 / 1.267
// / 1.271, SDDMM K = 128 0.707 / 0.697 / 0.699, K = 256 1.459 / 1.461 / 1.465.  SBM 1M and the
// grid+hubs graph: 2.3% and 0.7% of the entries, not staged.
constexpr int32_t kHotRows = 32768;
constexpr int32_t kHotColumnShare = 16;
constexpr int64_t kHotMinShare10 = 3;
constexpr int64_t kHotMaxColumnsPerEntry = 4;
// The column counts are taken in up to kCountCopies histograms (workgroup b into copy b mod
// copies), at most kCountCopyBytes in all, and summed.
constexpr int64_t kCountCopies = 8;
constexpr int64_t kCountCopyBytes = 64ll << 20;

// Host threads for plan lowering (std::thread: this object does not use an OpenMP runtime).
int lowering_threads() {
  const unsigned h = std::thread::hardware_concurrency();
  return (int)std::max(1u, std::min(h, 32u));
}

// fn(begin, end, t) on `parts` contiguous pieces of [0, n) given by cut(t) (cut(0) = 0,
// cut(parts) = n), one thread each; serial below `serial_below` elements.
template <class Cut, class Fn>
void parallel_parts(int parts, int64_t n, int64_t serial_below, Cut&& cut, Fn&& fn) {
  if (parts <= 1 || n < serial_below) {
    fn((int64_t)0, n, 0);
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(parts);
  for (int t = 0; t < parts; ++t) pool.emplace_back([&, t] { fn(cut(t), cut(t + 1), t); });
  for (auto& th : pool) th.join();
}
template <class Fn>
void parallel_chunks(int64_t n, Fn&& fn) {
  const int T = lowering_threads();
  parallel_parts(T, n, 1 << 16, [&](int t) { return n * t / T; }, fn);
}

// fn over [0, n) tiles (about 1 KB each) in parallel pieces.
template <class Fn>
void parallel_tiles(int64_t n, Fn&& fn) {
  const int T = lowering_threads();
  parallel_parts(T, n, 1024, [&](int t) { return n * t / T; }, fn);
}

// Host-side staging of one plan.
struct Lowering {
  int32_t m = 0, n = 0;
  std::vector<int32_t> row, col;
  std::vector<float> val;
  // MFMA tiles: row0, 16 columns, dense 16x16 values
  struct Tile { int32_t row0; int32_t cols[16]; float a[256]; uint64_t present[4]; int nnz; };
  // (tiles are over 1 KB each and written whole: no zero-fill on resize)
  trs::array<Tile> tiles;
  Status st;
  // Tiles only: entries outside tiles are not collected (the device lowering takes the residual
  // from the input CSR instead).
  bool tiles_only = false;

  bool check_col(int64_t c) {
    if (c < 0 || c >= n) {
      if (st.ok()) st = fail(TRS_ERANGE, "column index " + std::to_string(c) + " outside [0, " + std::to_string(n) + ")");
      return false;
    }
    return true;
  }
  void add(int64_t r, int64_t c, float v) {
    if (tiles_only) return;
    if (r < 0 || r >= m) return;   // reference kernels drop rows >= mOri
    if (!check_col(c)) return;
    row.push_back((int32_t)r);
    col.push_back((int32_t)c);
    val.push_back(v);
  }
  // Tile entry; -1 columns never carry values.
  void tile_add(Tile& t, int r, int k, float v) {
    t.a[r * 16 + k] += v;
    t.present[r / 4] |= 1ull << ((r % 4) * 16 + k);
    t.nnz++;
  }
  static void tile_init(Tile& t, int32_t row0) {
    t.row0 = row0;
    std::fill(t.cols, t.cols + 16, -1);
    std::fill(t.a, t.a + 256, 0.f);
    std::fill(t.present, t.present + 4, 0ull);
    t.nnz = 0;
  }
  static bool tile_has(const Tile& t, int r, int k) { return (t.present[r / 4] >> ((r % 4) * 16 + k)) & 1; }
};


using TileVec = trs::array<Lowering::Tile>;

float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// The private results of parallel lowering pieces, appended in piece order (sized once: a tile is
// over 1 KB).  stop_at_error: stop at the first failed piece (nothing after it is needed).
void append_parts(Lowering& L, std::vector<Lowering>& part, bool stop_at_error) {
  size_t nr = L.row.size(), nt = L.tiles.size();
  for (const auto& q : part) {
    nr += q.row.size();
    nt += q.tiles.size();
  }
  L.row.reserve(nr);
  L.col.reserve(nr);
  L.val.reserve(nr);
  // the pieces' tiles land at their offsets, copied in parallel (a tile is over 1 KB)
  std::vector<size_t> at;
  size_t t0 = L.tiles.size();
  for (auto& q : part) {
    if (!q.st.ok() && L.st.ok()) L.st = q.st;
    if (!q.st.ok() && stop_at_error) break;
    L.row.insert(L.row.end(), q.row.begin(), q.row.end());
    L.col.insert(L.col.end(), q.col.begin(), q.col.end());
    L.val.insert(L.val.end(), q.val.begin(), q.val.end());
    at.push_back(t0);
    t0 += q.tiles.size();
  }
  L.tiles.resize(t0);
  parallel_parts((int)at.size(), (int64_t)at.size(), 2, [&](int t) { return (int64_t)t; },
                 [&](int64_t b, int64_t e, int) {
                   for (int64_t i = b; i < e; ++i) {
                     std::copy(part[i].tiles.begin(), part[i].tiles.end(), L.tiles.begin() + at[i]);
                     TileVec().swap(part[i].tiles);
                   }
                 });
}

// TC sub-blocks of parts [p_begin, p_end) -> MFMA tiles (pairs of sub-blocks of one part, 16
// columns) or entries.
void lower_tc_range(Lowering& L, const int32_t* t_rowoff, int64_t p_begin, int64_t p_end, const int32_t* t_blockoff,
                    const int32_t* t_col, const float* vals_f32, const uint16_t* vals_f16, int64_t nvals,
                    const int32_t* t_winrow, const int64_t* t_bin, bool to_mfma) {
  for (int64_t p = p_begin; p < p_end && L.st.ok(); ++p) {
    const int32_t s0 = t_rowoff[p], s1 = t_rowoff[p + 1];
    const int32_t row0 = t_winrow[p];
    const bool mfma = to_mfma && row0 % 16 == 0 && row0 >= 0;
    for (int32_t s = s0; s < s1 && L.st.ok(); s += (mfma ? 2 : 1)) {
      // MFMA tiles are built in place (a tile is over 1 KB)
      Lowering::Tile scratch;
      Lowering::Tile& T = mfma ? L.tiles.emplace_back() : scratch;
      if (mfma) Lowering::tile_init(T, row0);
      const int nsub = mfma ? std::min(2, s1 - s) : 1;
      for (int h = 0; h < nsub; ++h) {
        const int32_t sb = s + h;
        const uint64_t lo = (uint64_t)t_bin[2 * (int64_t)sb], hi = (uint64_t)t_bin[2 * (int64_t)sb + 1];
        int64_t vi = t_blockoff[sb];
        const int pop = __builtin_popcountll(lo) + __builtin_popcountll(hi);
        if (vi < 0 || vi + pop > nvals) {
          L.st = fail(TRS_EINVAL, "t_blockNew_offset / t_binary describe values beyond t_value");
          if (mfma) L.tiles.pop_back();
          return;
        }
        for (int k = 0; k < 8 && mfma; ++k) {
          const int32_t c = t_col[(int64_t)sb * 8 + k];
          if (c >= 0 && !L.check_col(c)) {
            L.tiles.pop_back();
            return;
          }
          T.cols[h * 8 + k] = c;
        }
        for (int half = 0; half < 2; ++half) {
          uint64_t bits = half ? hi : lo;
          while (bits) {
            const int b = __builtin_ctzll(bits);
            bits &= bits - 1;
            const int r = half * 8 + b / 8, k = b % 8;
            const int32_t c = t_col[(int64_t)sb * 8 + k];
            const float v = vals_f32 ? vals_f32[vi] : f16_to_f32(vals_f16[vi]);
            ++vi;
            if (c < 0) continue;   // value at an empty column: the reference reads B[-1]; skip
            if (mfma) {
              if (row0 + r < L.m) L.tile_add(T, r, h * 8 + k, v);
            } else {
              L.add((int64_t)row0 + r, c, v);
            }
          }
        }
      }
    }
  }
}

// Parts are independent: ranges of parts are lowered in parallel into private buffers and appended
// in part order, so the result (and the first error) equals the serial one.
void lower_tc(Lowering& L, const int32_t* t_rowoff, int64_t nparts, const int32_t* t_blockoff, const int32_t* t_col,
              const float* vals_f32, const uint16_t* vals_f16, int64_t nvals, const int32_t* t_winrow,
              const int64_t* t_bin, bool to_mfma) {
  const int T = lowering_threads();
  if (nparts < 4096 || T <= 1) {
    lower_tc_range(L, t_rowoff, 0, nparts, t_blockoff, t_col, vals_f32, vals_f16, nvals, t_winrow, t_bin, to_mfma);
    return;
  }
  std::vector<Lowering> part(T);
  for (auto& q : part) {
    q.m = L.m;
    q.n = L.n;
    q.tiles_only = L.tiles_only;
  }
  parallel_parts(T, nparts, 0, [&](int t) { return nparts * t / T; }, [&](int64_t pb, int64_t pe, int t) {
    lower_tc_range(part[t], t_rowoff, pb, pe, t_blockoff, t_col, vals_f32, vals_f16, nvals, t_winrow, t_bin, to_mfma);
  });
  append_parts(L, part, true);
}

void lower_residual(Lowering& L, const int32_t* off, const int32_t* rows, int64_t nparts, const int32_t* cols,
                    const float* vf32, const uint16_t* vf16, int64_t ncols) {
  for (int64_t i = 0; i < nparts && L.st.ok(); ++i) {
    if (off[i] < 0 || off[i + 1] < off[i] || off[i + 1] > ncols) {
      L.st = fail(TRS_EINVAL, "residual offsets out of range");
      return;
    }
    for (int32_t e = off[i]; e < off[i + 1]; ++e) L.add(rows[i], cols[e], vf32 ? vf32[e] : f16_to_f32(vf16[e]));
  }
}

// 2:4 groups (s_column / s_value / s_pos) grouped in tiles of 4 per window as the reference packs them.
void lower_groups_range(Lowering& L, const int32_t* s_col, const float* s_val, const int8_t* s_pos, int64_t groups,
                        const int32_t* s_win, const int32_t* s_off, int64_t w_begin, int64_t w_end, int window,
                        bool to_mfma, float min_fill);

// Windows are independent: ranges of windows (balanced by group count) are lowered in parallel
// into private buffers and appended in window order, so the result equals the serial one.
void lower_groups(Lowering& L, const int32_t* s_col, const float* s_val, const int8_t* s_pos, int64_t groups,
                  const int32_t* s_win, const int32_t* s_off, int64_t nwin, int window, bool to_mfma,
                  float min_fill) {
  if (s_off)
    for (int64_t w = 0; w < nwin; ++w)
      if (s_off[w] < 0 || s_off[w + 1] < s_off[w] || s_off[w + 1] > groups) {
        L.st = fail(TRS_EINVAL, "s_offsets out of range");
        return;
      }
  if (!s_off || groups < (1 << 16)) {
    lower_groups_range(L, s_col, s_val, s_pos, groups, s_win, s_off, 0, nwin, window, to_mfma, min_fill);
    return;
  }
  const int T = lowering_threads();
  std::vector<int64_t> wcut(T + 1, nwin);
  wcut[0] = 0;
  for (int t = 1; t < T; ++t)
    wcut[t] = std::upper_bound(s_off, s_off + nwin + 1, (int32_t)(groups * t / T)) - s_off - 1;
  for (int t = 1; t <= T; ++t) wcut[t] = std::max(wcut[t], wcut[t - 1]);
  std::vector<Lowering> part(T);
  for (auto& q : part) {
    q.m = L.m;
    q.n = L.n;
    q.tiles_only = L.tiles_only;
  }
  parallel_parts(T, nwin, 0, [&](int t) { return wcut[t]; }, [&](int64_t wb, int64_t we, int t) {
    lower_groups_range(part[t], s_col, s_val, s_pos, groups, s_win, s_off, wb, we, window, to_mfma, min_fill);
  });
  append_parts(L, part, false);
}

void lower_groups_range(Lowering& L, const int32_t* s_col, const float* s_val, const int8_t* s_pos, int64_t groups,
                        const int32_t* s_win, const int32_t* s_off, int64_t w_begin, int64_t w_end, int window,
                        bool to_mfma, float min_fill) {
  auto group_row0 = [&](int64_t g, int64_t w) { return (int64_t)(s_win ? s_win[g] : w) * window; };
  auto emit_group = [&](int64_t g, int64_t row0) {
    if (L.tiles_only) return;
    for (int lr = 0; lr < window; ++lr)
      for (int q = 0; q < 2; ++q) {
        const int p = s_pos[(g * window + lr) * 2 + q];
        if (p < 0) continue;
        if (p > 3) { if (L.st.ok()) L.st = fail(TRS_EINVAL, "s_pos entry outside 0..3"); return; }
        const int32_t c = s_col[g * 4 + p];
        if (c < 0) continue;   // value at a padded column slot (scalar kernel skips it)
        L.add(row0 + lr, c, s_val[(g * window + lr) * 2 + q]);
      }
  };
  if (!s_off || !to_mfma || window != 16) {
    if (L.tiles_only) return;
    if (s_off) {
      for (int64_t w = w_begin; w < w_end && L.st.ok(); ++w)
        for (int64_t g = s_off[w]; g < s_off[w + 1]; ++g) emit_group(g, group_row0(g, w));
    } else {
      for (int64_t g = 0; g < groups && L.st.ok(); ++g) emit_group(g, group_row0(g, 0));
    }
    return;
  }
  for (int64_t w = w_begin; w < w_end && L.st.ok(); ++w) {
    for (int64_t base = s_off[w]; base < s_off[w + 1] && L.st.ok(); base += 4) {
      const int64_t end = std::min<int64_t>(base + 4, s_off[w + 1]);
      int kept = 0;
      for (int64_t g = base; g < end; ++g)
        for (int i = 0; i < window * 2; ++i) kept += s_pos[g * window * 2 + i] >= 0;
      const int64_t row0 = group_row0(base, w);
      if (kept < min_fill * 256.f || row0 % 16 != 0) {
        for (int64_t g = base; g < end; ++g) emit_group(g, group_row0(g, w));
        continue;
      }
      Lowering::Tile T;
      Lowering::tile_init(T, (int32_t)row0);
      for (int64_t g = base; g < end; ++g) {
        const int gi = (int)(g - base);
        for (int p = 0; p < 4; ++p) {
          const int32_t c = s_col[g * 4 + p];
          if (c >= 0 && !L.check_col(c)) return;
          T.cols[gi * 4 + p] = c;
        }
        for (int lr = 0; lr < window; ++lr)
          for (int q = 0; q < 2; ++q) {
            const int p = s_pos[(g * window + lr) * 2 + q];
            if (p < 0) continue;
            if (p > 3) { L.st = fail(TRS_EINVAL, "s_pos entry outside 0..3"); return; }
            if (s_col[g * 4 + p] < 0) continue;
            if (row0 + lr < L.m) L.tile_add(T, lr, gi * 4 + p, s_val[(g * window + lr) * 2 + q]);
          }
      }
      L.tiles.push_back(T);
    }
  }
}

// Packed 2:4 tiles (s_tile_column / s_packed_a / s_packed_meta) -> entries or MFMA tiles.
void lower_packed(Lowering& L, const int32_t* tcol, const int32_t* pa, const int32_t* pm, int64_t tiles,
                  const int32_t* wto, int64_t nwin, int window, bool to_mfma, float min_fill) {
  for (int64_t w = 0; w < nwin && L.st.ok(); ++w) {
    if (wto[w] < 0 || wto[w + 1] < wto[w] || wto[w + 1] > tiles) {
      L.st = fail(TRS_EINVAL, "s_window_tile_offset out of range");
      return;
    }
    for (int64_t t = wto[w]; t < wto[w + 1] && L.st.ok(); ++t) {
      struct E { int r, k; float v; };
      std::vector<E> es;
      for (int rg = 0; rg < 8; ++rg) {
        const uint32_t meta = (uint32_t)pm[t * 8 + rg];
        for (int hsel = 0; hsel < 2; ++hsel) {
          const int lr = rg + 8 * hsel;
          if (lr >= window) continue;
          for (int c = 0; c < 4; ++c) {
            const uint32_t word = (uint32_t)pa[((t * 8 + rg) * 4 + c) * 2 + hsel];
            const uint32_t m4 = (meta >> (16 * hsel + 4 * c)) & 15u;
            const int p0 = m4 & 3, p1 = (m4 >> 2) & 3;
            const float v0 = f16_to_f32((uint16_t)(word & 0xffffu));
            const float v1 = f16_to_f32((uint16_t)(word >> 16));
            if (v0 != 0.f) es.push_back({lr, c * 4 + p0, v0});
            if (v1 != 0.f) es.push_back({lr, c * 4 + p1, v1});
          }
        }
      }
      const int64_t row0 = w * (int64_t)window;
      const bool mfma = to_mfma && window == 16 && row0 % 16 == 0 && (float)es.size() >= min_fill * 256.f;
      Lowering::Tile T;
      if (mfma) {
        Lowering::tile_init(T, (int32_t)row0);
        for (int k = 0; k < 16; ++k) {
          const int32_t c = tcol[t * 16 + k];
          if (c >= 0 && !L.check_col(c)) return;
          T.cols[k] = c;
        }
      }
      for (const E& e : es) {
        const int32_t c = tcol[t * 16 + e.k];
        if (c < 0) continue;
        if (mfma) {
          if (row0 + e.r < L.m) L.tile_add(T, e.r, e.k, e.v);
        } else {
          L.add(row0 + e.r, c, e.v);
        }
      }
      if (mfma) L.tiles.push_back(T);
    }
  }
}

// Layout of a plan's single device allocation: arrays at 256-byte aligned offsets, copied from
// their host vectors by upload() (which must run while the vectors are alive).
struct Blob {
  struct Piece {
    const void* src;
    size_t off, bytes;
  };
  std::vector<Piece> pieces;
  size_t total = 0;
  template <class T, class A>
  size_t add(const std::vector<T, A>& v) {
    return add_raw(v.data(), v.size() * sizeof(T));
  }
  // src = nullptr: a region the device fills (left as allocated)
  size_t add_raw(const void* src, size_t bytes) {
    const size_t off = (total + 255) & ~size_t(255);
    pieces.push_back({src, off, bytes});
    total = off + bytes;
    return off;
  }
  // 256 bytes past the last array: kernels may read whole 16-byte chunks that end past an array
  size_t size() const { return total + 256; }
};

// Residual work items of a plan.
//
// Main part: tasks over the rows of `rowptr` that no MFMA window owns (owned: per 16-row block,
// empty = none), spread over the chip by xcd_remap: runs of whole rows (<= S entries, <= kTaskRows
// rows) and equal pieces of rows longer than piece_max.  SpMM pieces sum into partial slots that
// the fixup kernel adds up in a fixed order; SDDMM pieces write their own outputs.
//
// XCD column split (split part): workgroup i runs on XCD i mod 8 (measured on MI355X for every
// grid size and workload), and each XCD has its own 4 MB L2.  The columns are divided among the 8
// XCDs and rows with at least split_min entries are cut into sub-rows, one per XCD, laid out
// XCD-major after the main part; XCD x's sub-rows are packed into tasks like ordinary rows and
// queued for XCD x, so each L2 caches B rows of one eighth of the columns only.  An SpMM sub-row's
// sum goes to a partial slot (sub-row j -> slot j; pieces of long sub-rows get slots of their own
// after those), and the fixup adds a split row's slots in XCD order, so the result is
// deterministic.  SDDMM sub-rows are copies of the split rows' column ids, with the output index
// of each entry (x_pos); since the split only pays from K = 128 on, an SDDMM plan also keeps the
// unsplit task list of all rows (full) for narrower widths.
//
// The work is split in three: place_entries decides where every residual entry goes (from the
// row lengths and the split rows' columns alone), move_entries puts them there (on the host here;
// the device lowering does it with kernels), build_tasks cuts the placed rows into tasks.

// The input CSR a device lowering reads: row pointers on the host; columns and values on the host
// (a trs_format built in this process), in device memory (a trs_dformat), or both.
struct CsrSource {
  int32_t rows = 0;
  const int32_t* rowptr = nullptr;   // host, rows + 1
  const int32_t* col = nullptr;      // host (null: device only)
  const float* val = nullptr;
  const int32_t* d_col = nullptr;    // device (null: uploaded from the host arrays when needed)
  const float* d_val = nullptr;
};

CsrSource csr_of(const trs_format& f) {
  CsrSource c;
  c.rows = f.rows;
  c.rowptr = f.csr_rowptr.data();
  c.col = f.csr_col.data();
  c.val = f.csr_val.data();
  return c;
}

// Where the residual entries go in the plan's entry arrays.
struct Placement {
  bool compact = false;               // SpMM: split rows leave the main part (else they stay, SDDMM)
  std::vector<int32_t> main_rowptr;   // [m + 1] main part
  std::vector<uint8_t> split;         // per row
  std::vector<int32_t> split_rows;    // ascending
  std::vector<int32_t> cursor;        // [split row i][XCD x]: first position of sub-row (i, x), -1 = none
  std::vector<int32_t> xrowptr;       // [J + 1] sub-rows, XCD-major
  std::vector<int32_t> sub_row;       // [J] row of each sub-row
  int32_t xfirst[trs::kXcds + 1] = {};
  int64_t total = 0;                  // length of the plan's entry arrays
  int32_t J() const { return (int32_t)sub_row.size(); }
};

// Split-row statistics from device-resident columns (defined with the device lowering below).
Status split_stats_device(const int32_t* d_col, const int32_t* col_rowptr, const std::vector<int32_t>& rowptr,
                          const std::vector<int32_t>& split_rows, int32_t n, bool need_distinct, int64_t& total,
                          int64_t& distinct, std::vector<int32_t>& cnt);

// rowptr: the residual CSR's row pointers; owned: per 16-row block (empty = none).  The columns of
// a split row r are col[col_rowptr[r] ..] (col_rowptr = rowptr for the residual CSR itself; the
// input CSR's row pointers when the residual is built on the device, where split rows -- owned by
// no window, so no tile took entries from them -- equal their input rows).
//
// min_reuse > 0 (the automatic split): split only when the candidate rows' entries are at least
// min_reuse times their distinct columns.  The split buys L2 reuse of B rows; columns the long rows
// read once or twice each (uniformly random hub rows) have none to buy, and the split's extra
// launch and partial slots then cost time.
// d_col (device lowering of a device-resident CSR; col is then unused): the candidates' statistics
// are counted on the device instead.
Placement place_entries(const std::vector<int32_t>& rowptr, const int32_t* col, const int32_t* col_rowptr, int32_t m,
                        int32_t n, const std::vector<uint8_t>& owned, bool compact, int32_t split_min,
                        int32_t min_reuse = 0, const int32_t* d_col = nullptr, Status* st = nullptr) {
  Placement P;
  P.compact = compact;
  const int64_t nent = rowptr[m];
  P.split.assign((size_t)m, 0);
  if (split_min > 0 && n > 0)
    for (int32_t r = 0; r < m; ++r)
      if (!(!owned.empty() && owned[r / 16]) && rowptr[r + 1] - rowptr[r] >= split_min) {
        P.split[r] = 1;
        P.split_rows.push_back(r);
      }
  std::vector<int32_t> dev_cnt;
  if (d_col && !P.split_rows.empty()) {
    int64_t total = 0, distinct = 0;
    const Status ds = split_stats_device(d_col, col_rowptr, rowptr, P.split_rows, n, min_reuse > 0, total, distinct,
                                         dev_cnt);
    if (!ds.ok()) {
      if (st) *st = ds;
      return P;
    }
    if (min_reuse > 0 && total < (int64_t)min_reuse * distinct) {
      for (int32_t r : P.split_rows) P.split[r] = 0;
      P.split_rows.clear();
      dev_cnt.clear();
    }
  } else if (min_reuse > 0 && !P.split_rows.empty()) {
    // distinct columns of the candidate rows: per-thread bitmaps, OR-ed
    const int T = lowering_threads();
    const size_t ns = P.split_rows.size();
    const size_t words = ((size_t)n + 63) / 64;
    std::vector<std::vector<uint64_t>> seen(T);
    std::vector<int64_t> entries(T, 0);
    parallel_parts(T, (int64_t)ns, 256, [&](int t) { return (int64_t)ns * t / T; }, [&](int64_t b, int64_t e, int t) {
      std::vector<uint64_t>& bits = seen[t];
      bits.assign(words, 0);
      for (int64_t i = b; i < e; ++i) {
        const int32_t r = P.split_rows[i];
        const int32_t* c = col + col_rowptr[r];
        const int32_t len = rowptr[r + 1] - rowptr[r];
        for (int32_t q = 0; q < len; ++q) bits[(uint32_t)c[q] >> 6] |= 1ull << (c[q] & 63);
        entries[t] += len;
      }
    });
    int64_t distinct = 0, total = 0;
    for (int t = 0; t < T; ++t) total += entries[t];
    for (size_t w = 0; w < words; ++w) {
      uint64_t x = 0;
      for (int t = 0; t < T; ++t)
        if (!seen[t].empty()) x |= seen[t][w];
      distinct += __builtin_popcountll(x);
    }
    if (total < (int64_t)min_reuse * distinct) {
      for (int32_t r : P.split_rows) P.split[r] = 0;
      P.split_rows.clear();
    }
  }
  const size_t ns = P.split_rows.size();
  // entries per (split row, XCD), counted by the column hash on a few threads
  std::vector<int32_t> cnt(ns * trs::kXcds, 0);
  if (d_col) cnt.swap(dev_cnt);
  else parallel_parts(lowering_threads(), (int64_t)ns, 256, [&](int t) { return (int64_t)ns * t / lowering_threads(); },
                 [&](int64_t b, int64_t e, int) {
                   for (int64_t i = b; i < e; ++i) {
                     const int32_t r = P.split_rows[i];
                     const int32_t* c = col + col_rowptr[r];
                     for (int32_t q = 0; q < rowptr[r + 1] - rowptr[r]; ++q) cnt[i * trs::kXcds + trs::xcd_of_column(c[q])]++;
                   }
                 });
  P.main_rowptr.resize((size_t)m + 1);
  int64_t w = 0;
  for (int32_t r = 0; r < m; ++r) {
    P.main_rowptr[r] = (int32_t)w;
    if (!(compact && P.split[r])) w += rowptr[r + 1] - rowptr[r];
  }
  P.main_rowptr[m] = (int32_t)w;
  if (!compact) w = nent;   // SDDMM: copies after the whole main part
  P.cursor.assign(ns * trs::kXcds, -1);
  for (int y = 0; y < trs::kXcds; ++y) {
    P.xfirst[y] = (int32_t)P.sub_row.size();
    for (size_t i = 0; i < ns; ++i) {
      const int32_t c = cnt[i * trs::kXcds + y];
      if (c == 0) continue;
      P.cursor[i * trs::kXcds + y] = (int32_t)w;
      P.sub_row.push_back(P.split_rows[i]);
      P.xrowptr.push_back((int32_t)w);
      w += c;
    }
  }
  P.xfirst[trs::kXcds] = (int32_t)P.sub_row.size();
  P.xrowptr.push_back((int32_t)w);
  P.total = w;
  return P;
}

// The entries of the residual CSR (rowptr / col / val) in their placed order: col_out / val_out
// of P.total entries; x_pos (SDDMM) gets the residual index of each sub-row entry.
void move_entries(const Placement& P, const std::vector<int32_t>& rowptr, const int32_t* col, const uint16_t* val,
                  int32_t m, std::vector<int32_t>& col_out, std::vector<uint16_t>* val_out,
                  std::vector<int32_t>* x_pos, std::vector<int32_t>* x_src = nullptr,
                  const std::vector<int32_t>* merge_off = nullptr) {
  const int64_t nent = rowptr[m];
  col_out.resize((size_t)P.total);
  if (val_out) val_out->resize((size_t)P.total);
  if (x_pos) x_pos->resize((size_t)(P.total - (P.compact ? 0 : nent)));
  if (x_src) x_src->resize((size_t)(P.total - (P.compact ? 0 : nent)));
  // main part, in row order
  parallel_parts(lowering_threads(), (int64_t)m, 1 << 14, [&](int t) { return (int64_t)m * t / lowering_threads(); },
                 [&](int64_t rb, int64_t re, int) {
                   for (int64_t r = rb; r < re; ++r) {
                     if (P.compact && P.split[r]) continue;
                     const int32_t d = P.main_rowptr[r];
                     for (int32_t q = rowptr[r]; q < rowptr[r + 1]; ++q) {
                       col_out[d + q - rowptr[r]] = col[q];
                       if (val_out) (*val_out)[d + q - rowptr[r]] = val[q];
                     }
                   }
                 });
  // sub-rows: each split row's entries by the XCD of their column, in column order
  const size_t ns = P.split_rows.size();
  const int64_t xbase = P.compact ? 0 : nent;
  parallel_parts(lowering_threads(), (int64_t)ns, 256, [&](int t) { return (int64_t)ns * t / lowering_threads(); },
                 [&](int64_t b, int64_t e, int) {
                   int32_t cur[trs::kXcds];
                   for (int64_t i = b; i < e; ++i) {
                     std::copy(P.cursor.begin() + i * trs::kXcds, P.cursor.begin() + (i + 1) * trs::kXcds, cur);
                     const int32_t r = P.split_rows[i];
                     for (int32_t q = rowptr[r]; q < rowptr[r + 1]; ++q) {
                       const int32_t o = cur[trs::xcd_of_column(col[q])]++;
                       col_out[o] = col[q];
                       if (val_out) (*val_out)[o] = val[q];
                       if (x_pos) (*x_pos)[o - xbase] = q;
                       if (x_src) (*x_src)[(*merge_off)[i] + (q - rowptr[r])] = (int32_t)(o - xbase);
                     }
                   }
                 });
}

struct Tasks {
  std::vector<trs::Task> tasks;      // main part
  std::vector<trs::Task> xtasks;     // split part: queue x = xtasks [xq[x], xq[x + 1])
  int32_t xq[trs::kXcds + 1] = {};
  std::vector<trs::Task> full;       // SDDMM with a split part: the unsplit layout of every row
  std::vector<trs::Task> narrow;     // SDDMM: the unsplit layout with pieces of S entries (lane
                                     // groups of <= 8 lanes), where some row is longer than S
  std::vector<trs::Fixup> fix, wfix; // SpMM: {row, first index into slot_list, slots}
  std::vector<int32_t> slot_list;
  int32_t slots = 0;
  int64_t split_rows = 0;
  int32_t task_nnz = 0;              // entries per packed task (S)
  int32_t task_max = 0, xtask_max = 0;
  Status st;
};

// Residual tasks a plan aims at when the automatic task size leaves fewer (small matrices).
constexpr int64_t kMinTasks = 16384;
// Rows per chunk of the main part's task packing (a multiple of 16: MFMA windows stay whole).
constexpr int64_t kPackRows = 1 << 16;

// Longest tasks first (a stable counting sort on the entry count, which never exceeds the piece
// length): a workgroup's lane groups then carry tasks of similar length, so none idles while a
// longer one finishes (R-MAT K = 32 / 64 / 128: -9% / -11% / -5%).  Among tasks of one length,
// pieces go by their index in their row (the first pieces of all long rows, then the second ones,
// ...): a row's entries are in column order, so the pieces that run together cover the same part
// of the column range in every long row, and their B (Y) rows are shared in the L2 and read from
// nearby addresses, where row by row the concurrent pieces gathered across the whole of B.
// Same-box A/B against row order: grid+hubs K = 32 / 64 SpMM 0.366 / 0.588 -> 0.348 / 0.580 ms
// (its 64 hub rows of 100K random columns), SDDMM K = 32 0.433 -> 0.422; R-MAT SDDMM K = 32
// 0.368 -> 0.352, SpMM K = 64 / 128 / 256 0.442 / 0.599 / 1.243 -> 0.440 / 0.597 / 1.239.
void sort_longest_first(std::vector<trs::Task>::iterator first, std::vector<trs::Task>::iterator last) {
  const size_t n = (size_t)(last - first);
  if (n == 0) return;
  int32_t most = 0;
  for (auto it = first; it != last; ++it) most = std::max(most, it->nz_end - it->nz_begin);
  // a piece's index in its row: the pieces of a row are consecutive here (row_end < 0 marks them)
  std::vector<int32_t> piece(n, 0);
  int32_t pieces = 0;
  for (size_t i = 1; i < n; ++i) {
    const trs::Task& a = first[(ptrdiff_t)i - 1];
    const trs::Task& b = first[(ptrdiff_t)i];
    if (a.row_end < 0 && b.row_end < 0 && a.row_begin == b.row_begin) {
      piece[i] = piece[i - 1] + 1;
      pieces = std::max(pieces, piece[i]);
    }
  }
  // two stable counting sorts (by piece index, then by length, longest first): the order is
  // (length desc, piece index asc, input order), in O(n + pieces + most) memory
  std::vector<size_t> idx(n), by_piece(n);
  {
    std::vector<int64_t> start((size_t)pieces + 2, 0);
    for (size_t i = 0; i < n; ++i) start[(size_t)piece[i] + 1]++;
    for (size_t i = 1; i < start.size(); ++i) start[i] += start[i - 1];
    for (size_t i = 0; i < n; ++i) by_piece[(size_t)start[(size_t)piece[i]]++] = i;
  }
  {
    auto len_key = [&](size_t i) { return (size_t)(most - (first[(ptrdiff_t)i].nz_end - first[(ptrdiff_t)i].nz_begin)); };
    std::vector<int64_t> start((size_t)most + 2, 0);
    for (size_t i = 0; i < n; ++i) start[len_key(i) + 1]++;
    for (size_t i = 1; i < start.size(); ++i) start[i] += start[i - 1];
    for (size_t j = 0; j < n; ++j) idx[(size_t)start[len_key(by_piece[j])]++] = by_piece[j];
  }
  std::vector<trs::Task> out(n);
  for (size_t i = 0; i < n; ++i) out[i] = first[(ptrdiff_t)idx[i]];
  std::copy(out.begin(), out.end(), first);
}

// Tasks over the placed rows (the residual row lengths are rowptr's, before placement).
Tasks build_tasks(const Placement& P, const std::vector<int32_t>& rowptr, int32_t m, const std::vector<uint8_t>& owned,
                  bool with_fixup, const trs_plan_options& opt) {
  Tasks T;
  const int64_t nent = rowptr[m];
  // Entries per packed task: short rows want small tasks (more lane groups in flight, fewer row
  // flushes per group), long rows want larger ones.  Measured on MI355X: 32 for a degree-4 mesh,
  // 128 for R-MAT (mean non-empty row ~49) -- about four mean rows per task.
  int S = opt.task_nnz;
  if (S <= 0) {
    int64_t nonempty = 0;
    for (int32_t q = 0; q < m; ++q) nonempty += rowptr[q + 1] > rowptr[q];
    const double mean = nonempty ? (double)nent / (double)nonempty : 1.0;
    S = (int)std::min(128.0, std::max(32.0, 4.0 * mean));
  }
  // Small matrices: fewer than kMinTasks tasks leave most lane groups of the chip idle while the
  // rest walk long task streams one batch round trip after another, so automatic sizes shrink to
  // reach kMinTasks (tasks of at least 16 entries, pieces of 64).  Measured on MI355X, R-MAT 2^14
  // (426K entries) K = 64: 75 -> 42 us per call; R-MAT 2^20 (31.4M entries) is far above the bar.
  const bool small = nent / S < kMinTasks;
  if (opt.task_nnz <= 0 && small) S = (int)std::max<int64_t>(16, std::min<int64_t>(S, nent / kMinTasks));
  T.task_nnz = S;
  const int piece_max = std::max(S, opt.piece_nnz > 0 ? opt.piece_nnz : small ? 64 : 256);
  const int rows_cap = trs::kTaskRows;
  auto is_owned = [&](int32_t r) { return !owned.empty() && owned[r / 16]; };
  const int32_t J = P.J();
  if (with_fixup) T.slots = J;   // sub-row j sums into slot j; piece slots follow

  // equal pieces of at most piece_max entries of [b, e) of (sub-)row r
  auto cut_pieces = [&](int32_t r, int32_t b, int32_t e, std::vector<trs::Task>& outv, std::vector<int32_t>* slots_of,
                        int32_t pmax) {
    const int32_t d = e - b;
    const int np = (d + pmax - 1) / pmax;
    for (int q = 0; q < np; ++q) {
      const int32_t pb = b + (int32_t)((int64_t)d * q / np), pe = b + (int32_t)((int64_t)d * (q + 1) / np);
      outv.push_back({r, with_fixup ? ~T.slots : -1, pb, pe});
      if (with_fixup) {
        if (slots_of) slots_of->push_back(T.slots);
        ++T.slots;
      }
    }
  };
  auto add_fixup = [&](int32_t r, const std::vector<int32_t>& sl) {
    if (!with_fixup) return;
    (sl.size() > (size_t)trs::kWideFixupSlots ? T.wfix : T.fix)
        .push_back({r, (int32_t)T.slot_list.size(), (int32_t)sl.size(), 0});
    T.slot_list.insert(T.slot_list.end(), sl.begin(), sl.end());
    ++T.split_rows;
  };
  // runs of whole (sub-)rows [r, r1) of rp, row r1 - r <= rows_cap, entries <= S, none longer
  // than piece_max; stop(r) ends a run before row r
  auto pack = [&](const std::vector<int32_t>& rp, int32_t r, int32_t end, auto&& stop) {
    int32_t r1 = r + 1;
    int32_t tot = rp[r + 1] - rp[r];
    while (r1 < end && r1 - r < rows_cap && !stop(r1)) {
      const int32_t d = rp[r1 + 1] - rp[r1];
      if (d > piece_max || tot + d > S) break;
      tot += d;
      ++r1;
    }
    return r1;
  };

  // main part (skip_split: without the split rows), longest tasks first.  Runs of rows are packed
  // in chunks of kPackRows rows, in parallel (a run never crosses a chunk boundary, so the tasks do
  // not depend on the thread count); rows longer than piece_max are collected and cut afterwards,
  // in row order, which numbers their slots.
  const std::vector<int32_t>& rp = P.main_rowptr;
  auto build_main = [&](bool skip_split, std::vector<trs::Task>& outv, int32_t pmax) {
    const int64_t nchunks = ((int64_t)m + kPackRows - 1) / kPackRows;
    std::vector<std::vector<trs::Task>> packed((size_t)nchunks);
    std::vector<std::vector<int32_t>> longer((size_t)nchunks);
    const int T = (int)std::min<int64_t>(lowering_threads(), nchunks);
    parallel_parts(T, nchunks, 2, [&](int t) { return nchunks * t / T; }, [&](int64_t cb, int64_t ce, int) {
      for (int64_t ch = cb; ch < ce; ++ch) {
        const int32_t end = (int32_t)std::min<int64_t>(m, (ch + 1) * kPackRows);
        int32_t r = (int32_t)(ch * kPackRows);
        while (r < end) {
          if (is_owned(r)) { r = std::min(end, (r / 16 + 1) * 16); continue; }
          if (skip_split && P.split[r]) { ++r; continue; }
          if (rp[r + 1] - rp[r] > pmax) {
            longer[(size_t)ch].push_back(r);
            ++r;
            continue;
          }
          const int32_t r1 = pack(rp, r, end, [&](int32_t q) { return is_owned(q) || (skip_split && P.split[q] != 0); });
          packed[(size_t)ch].push_back({r, r1, rp[r], rp[r1]});
          r = r1;
        }
      }
    });
    std::vector<trs::Task> pieces;
    std::vector<int32_t> sl;
    for (const auto& rows : longer)
      for (int32_t r : rows) {
        sl.clear();
        cut_pieces(r, rp[r], rp[r + 1], pieces, &sl, pmax);
        add_fixup(r, sl);
      }
    size_t np = pieces.size();
    for (const auto& v : packed) np += v.size();
    outv.reserve(np);
    outv.insert(outv.end(), pieces.begin(), pieces.end());
    for (const auto& v : packed) outv.insert(outv.end(), v.begin(), v.end());
    sort_longest_first(outv.begin(), outv.end());
  };
  build_main(true, T.tasks, piece_max);
  if (!with_fixup && J > 0) build_main(false, T.full, piece_max);   // SDDMM: no slots, no fixups to repeat
  // SDDMM lane groups of <= 8 lanes walk the unsplit layout in pieces of S entries: with 8 lanes
  // to a group a wave holds 8 tasks, and the long rows' pieces should not hold them for 256
  // entries (same-box A/B on R-MAT 2^20, pieces of 128 against 256: K = 16 0.302 -> 0.288 ms, K =
  // 32 0.359 -> 0.337; 16-lane groups lose with them, K = 64 0.443 -> 0.454, K = 96 0.651 ->
  // 0.668, and keep the 256-entry pieces)
  if (!with_fixup && opt.piece_nnz <= 0 && piece_max > S) {
    bool longer = false;
    for (int32_t r = 0; r < m && !longer; ++r) longer = !is_owned(r) && rp[r + 1] - rp[r] > S;
    if (longer) build_main(false, T.narrow, S);
  }

  // split part: per XCD, pieces of long sub-rows and runs of the others, longest first
  if (J > 0) {
    // sub-row j cut into pieces: their slots are pfirst[j] .. pfirst[j] + pn[j] (consecutive)
    std::vector<int32_t> pfirst((size_t)J, 0), pn((size_t)J, 0);
    for (int y = 0; y < trs::kXcds; ++y) {
      T.xq[y] = (int32_t)T.xtasks.size();
      int32_t j = P.xfirst[y];
      while (j < P.xfirst[y + 1]) {
        const int32_t d = P.xrowptr[j + 1] - P.xrowptr[j];
        if (d > piece_max) {
          pfirst[j] = T.slots;
          cut_pieces(j, P.xrowptr[j], P.xrowptr[j + 1], T.xtasks, nullptr, piece_max);
          pn[j] = T.slots - pfirst[j];
          ++j;
          continue;
        }
        const int32_t j1 = pack(P.xrowptr, j, P.xfirst[y + 1], [&](int32_t) { return false; });
        T.xtasks.push_back({j, j1, P.xrowptr[j], P.xrowptr[j1]});
        j = j1;
      }
      sort_longest_first(T.xtasks.begin() + T.xq[y], T.xtasks.end());
    }
    T.xq[trs::kXcds] = (int32_t)T.xtasks.size();
    if (with_fixup) {
      // a split row's slots in XCD order: sub-row j's own slot, or its pieces' slots.  Sub-rows are
      // numbered XCD by XCD, split rows in order within each (place_entries), and split row i has
      // a sub-row of XCD y exactly where P.cursor[i * kXcds + y] >= 0; the split rows are in row
      // order, and so are their fixups
      const size_t ns = P.split_rows.size();
      std::vector<int32_t> nsl(ns + 1, 0);
      int32_t j = 0;
      for (int y = 0; y < trs::kXcds; ++y)
        for (size_t i = 0; i < ns; ++i)
          if (P.cursor[i * trs::kXcds + y] >= 0) {
            nsl[i] += pn[(size_t)j] > 0 ? pn[(size_t)j] : 1;
            ++j;
          }
      std::vector<int32_t> sbeg(ns + 1, 0);
      for (size_t i = 0; i < ns; ++i) sbeg[i + 1] = sbeg[i] + nsl[i];
      std::vector<int32_t> flat((size_t)sbeg[ns]), fill(sbeg.begin(), sbeg.end() - 1);
      j = 0;
      for (int y = 0; y < trs::kXcds; ++y)
        for (size_t i = 0; i < ns; ++i) {
          if (P.cursor[i * trs::kXcds + y] < 0) continue;
          if (pn[(size_t)j] > 0)
            for (int32_t k = 0; k < pn[(size_t)j]; ++k) flat[(size_t)fill[i]++] = pfirst[(size_t)j] + k;
          else
            flat[(size_t)fill[i]++] = j;
          ++j;
        }
      T.slot_list.reserve(T.slot_list.size() + flat.size());
      for (size_t i = 0; i < ns; ++i) {
        const int32_t cntv = nsl[i];
        (cntv > trs::kWideFixupSlots ? T.wfix : T.fix)
            .push_back({P.split_rows[i], (int32_t)T.slot_list.size(), cntv, 0});
        T.slot_list.insert(T.slot_list.end(), flat.begin() + sbeg[i], flat.begin() + sbeg[i + 1]);
        ++T.split_rows;
      }
    }
  }
  for (const trs::Task& t : T.tasks) T.task_max = std::max(T.task_max, t.nz_end - t.nz_begin);
  for (const trs::Task& t : T.full) T.task_max = std::max(T.task_max, t.nz_end - t.nz_begin);
  for (const trs::Task& t : T.xtasks) T.xtask_max = std::max(T.xtask_max, t.nz_end - t.nz_begin);
  if (T.tasks.size() + T.xtasks.size() + T.full.size() + T.narrow.size() > (size_t)INT32_MAX / 64)
    T.st = fail(TRS_ERANGE, "too many tasks");
  return T;
}

// Residual CSR of a lowering: row pointers and the permutation of entries into row order, each
// row sorted by column (ties in insertion order) unless keep_order.  Stable counting sort by row
// with per-thread histograms, then the rows sorted in parallel (pieces balanced by entries).
void residual_csr(const Lowering& L, bool keep_order, std::vector<int32_t>& rowptr, std::vector<int64_t>& perm) {
  const int32_t m = L.m;
  const int64_t nent = (int64_t)L.row.size();
  const int T = nent >= (1 << 20) ? lowering_threads() : 1;
  auto cut = [&](int t) { return nent * t / T; };
  std::vector<std::vector<int32_t>> cnt(T, std::vector<int32_t>((size_t)m, 0));
  parallel_parts(T, nent, 0, cut, [&](int64_t b, int64_t e, int t) {
    int32_t* c = cnt[t].data();
    for (int64_t i = b; i < e; ++i) c[L.row[i]]++;
  });
  // rows in order; inside a row, thread pieces in order: entries keep their insertion order
  rowptr.assign((size_t)m + 1, 0);
  int64_t acc = 0;
  for (int32_t r = 0; r < m; ++r) {
    rowptr[r] = (int32_t)acc;
    for (int t = 0; t < T; ++t) {
      const int32_t c = cnt[t][r];
      cnt[t][r] = (int32_t)acc;
      acc += c;
    }
  }
  rowptr[m] = (int32_t)acc;
  perm.resize((size_t)nent);
  parallel_parts(T, nent, 0, cut, [&](int64_t b, int64_t e, int t) {
    int32_t* c = cnt[t].data();
    for (int64_t i = b; i < e; ++i) perm[(size_t)c[L.row[i]]++] = i;
  });
  std::vector<std::vector<int32_t>>().swap(cnt);
  if (keep_order) return;
  // rows split into pieces of about nent / T entries
  std::vector<int32_t> row_cut(T + 1, m);
  row_cut[0] = 0;
  for (int t = 1; t < T; ++t)
    row_cut[t] = (int32_t)(std::upper_bound(rowptr.begin(), rowptr.end(), (int32_t)(nent * t / T)) - rowptr.begin() - 1);
  for (int t = 1; t <= T; ++t) row_cut[t] = std::max(row_cut[t], row_cut[t - 1]);
  parallel_parts(T, (int64_t)m, 0, [&](int t) { return (int64_t)row_cut[t]; }, [&](int64_t rb, int64_t re, int) {
    for (int64_t r = rb; r < re; ++r) {
      auto b = perm.begin() + rowptr[r], e = perm.begin() + rowptr[r + 1];
      auto less = [&](int64_t x, int64_t y) { return L.col[x] != L.col[y] ? L.col[x] < L.col[y] : x < y; };
      if (!std::is_sorted(b, e, less)) std::sort(b, e, less);
    }
  });
}

// Blob pieces with a source into device memory at dmem.
bool copy_pieces(const Blob& blob, void* dmem) {
  for (const auto& pc : blob.pieces) {
    if (pc.bytes == 0 || !pc.src) continue;
    if (hipMemcpy(static_cast<unsigned char*>(dmem) + pc.off, pc.src, pc.bytes, hipMemcpyHostToDevice) != hipSuccess)
      return false;
  }
  return true;
}

// Entries per (split candidate, XCD class) -- cnt, as place_entries counts them -- and, with
// need_distinct, the candidates' distinct columns, counted on the device from the input columns
// d_col (candidate i = split_rows[i] holds d_col[col_rowptr[r] ..] of length rowptr[r + 1] - rowptr[r]).
Status split_stats_device(const int32_t* d_col, const int32_t* col_rowptr, const std::vector<int32_t>& rowptr,
                          const std::vector<int32_t>& split_rows, int32_t n, bool need_distinct, int64_t& total,
                          int64_t& distinct, std::vector<int32_t>& cnt) {
  const size_t ns = split_rows.size();
  // chunks of at most kChunk entries, one wave each
  constexpr int32_t kChunk = 2048;
  std::vector<int32_t> start, len, row;
  start.reserve(ns);
  len.reserve(ns);
  row.reserve(ns);
  total = 0;
  for (size_t i = 0; i < ns; ++i) {
    const int32_t r = split_rows[i];
    const int32_t b = col_rowptr[r], d = rowptr[r + 1] - rowptr[r];
    for (int32_t q = 0; q < d; q += kChunk) {
      start.push_back(b + q);
      len.push_back(std::min(kChunk, d - q));
      row.push_back((int32_t)i);
    }
    total += d;
  }
  const size_t flag_bytes = need_distinct ? ((size_t)n + 3) / 4 * 4 : 0;
  Blob tmp;
  const size_t o_start = tmp.add(start);
  const size_t o_len = tmp.add(len);
  const size_t o_row = tmp.add(row);
  const size_t o_cnt = tmp.add_raw(nullptr, ns * trs::kXcds * 4);
  const size_t o_pop = tmp.add_raw(nullptr, 8 + flag_bytes);   // the count, then the column flags
  void* dmem = nullptr;
  if (hipMalloc(&dmem, tmp.size()) != hipSuccess) {
    (void)hipGetLastError();
    return fail(kLowerOnHost, "device lowering temporaries: hipMalloc failed");
  }
  unsigned char* base = static_cast<unsigned char*>(dmem);
  auto done = [&](Status st) {
    (void)hipFree(dmem);
    return st;
  };
  unsigned long long* d_pop = reinterpret_cast<unsigned long long*>(base + o_pop);
  uint8_t* d_seen = need_distinct ? base + o_pop + 8 : nullptr;
  int32_t* d_cnt = reinterpret_cast<int32_t*>(base + o_cnt);
  if (!copy_pieces(tmp, dmem) || hipMemset(d_cnt, 0, ns * trs::kXcds * 4) != hipSuccess ||
      hipMemset(base + o_pop, 0, 8 + flag_bytes) != hipSuccess ||
      trs::launch_split_stats(d_col, reinterpret_cast<const int32_t*>(base + o_start),
                              reinterpret_cast<const int32_t*>(base + o_len),
                              reinterpret_cast<const int32_t*>(base + o_row), (int32_t)start.size(), d_cnt, d_seen,
                              nullptr) != hipSuccess ||
      (need_distinct && trs::launch_count_flags(d_seen, (int64_t)flag_bytes, d_pop, nullptr) != hipSuccess))
    return done(fail(TRS_EDEVICE, "device lowering: split statistics launch failed"));
  cnt.resize(ns * trs::kXcds);
  unsigned long long pop = 0;
  if (hipMemcpy(cnt.data(), d_cnt, cnt.size() * 4, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(&pop, d_pop, 8, hipMemcpyDeviceToHost) != hipSuccess)
    return done(fail(TRS_EDEVICE, "device lowering: split statistics failed"));
  distinct = (int64_t)pop;
  return done(Status{});
}

// One hipMalloc holding the whole plan, filled array by array.
Status upload(const Blob& blob, trs_plan*& P) {
  P = new trs_plan();
  if (hipGetDevice(&P->device) != hipSuccess) {
    delete P;
    P = nullptr;
    return fail(TRS_EDEVICE, "no HIP device available");
  }
  if (hipMalloc(&P->dmem, blob.size()) != hipSuccess) {
    P->dmem = nullptr;
    delete P;
    P = nullptr;
    (void)hipGetLastError();
    return fail(TRS_ENOMEM, "hipMalloc of " + std::to_string(blob.size()) + " plan bytes failed");
  }
  P->dbytes = blob.size();
  if (!copy_pieces(blob, P->dmem)) {
    delete P;
    P = nullptr;
    return fail(TRS_EDEVICE, "plan upload failed");
  }
  return Status{};
}

// Tiles by row0, equal row0 in their order: a stable sort of indices, then one gather (a tile is
// over 1 KB, too large to move around in a sort).
void sort_tiles(TileVec& tiles) {
  auto less = [&](const Lowering::Tile& a, const Lowering::Tile& b) { return a.row0 < b.row0; };
  const auto run = std::is_sorted_until(tiles.begin(), tiles.end(), less);
  if (run == tiles.end()) return;
  std::vector<int32_t> order(tiles.size());
  std::iota(order.begin(), order.end(), 0);
  auto by_row0 = [&](int32_t a, int32_t b) { return tiles[a].row0 < tiles[b].row0; };
  const size_t k = (size_t)(run - tiles.begin());
  if (std::is_sorted(run, tiles.end(), less)) {
    // two sorted runs (TC tiles, then the 2:4 group tiles): a stable merge of their indices
    std::vector<int32_t> merged(tiles.size());
    std::merge(order.begin(), order.begin() + k, order.begin() + k, order.end(), merged.begin(), by_row0);
    order.swap(merged);
  } else {
    std::stable_sort(order.begin(), order.end(), by_row0);
  }
  TileVec sorted(tiles.size());
  parallel_tiles((int64_t)tiles.size(), [&](int64_t b, int64_t e, int) {
    for (int64_t i = b; i < e; ++i) sorted[i] = tiles[order[i]];
  });
  tiles.swap(sorted);
}

// A tile whose every row holds at most 2 entries in each group of 4 columns (2:4 structured).
bool is_two_four(const Lowering::Tile& t) {
  for (int r = 0; r < 16; ++r) {
    const uint64_t bits = (t.present[r / 4] >> ((r % 4) * 16)) & 0xffffull;
    for (int g = 0; g < 4; ++g)
      if (__builtin_popcountll((bits >> (4 * g)) & 0xfull) > 2) return false;
  }
  return true;
}

// Sparse-MFMA operands of 2:4 tiles, four tiles (a quad, 64 columns) at a time, in the lane layout
// of v_smfmac_f32_16x16x64_f16 (kernels.hpp, DevicePlan::quad_*).
struct Quads {
  std::vector<int32_t> cols;    // [quad][64]
  std::vector<uint16_t> a;      // [quad][64 lanes][8] fp16
  std::vector<uint16_t> idx;    // [quad][64 lanes]: 2-bit positions, value j at bits 2j .. 2j + 1
  int32_t count = 0;
};

// Tiles [b, e) (at most 4) as the next quad; missing tiles are empty.  In each (row, group of 4
// columns) the present entries, at most 2, take the group's two slots in column order; a single
// entry is paired with a zero at another position (position 1 if it sits at 0, else 0), an empty
// group with zeros at 0 and 1, so every slot pair names two distinct positions in ascending order.
void add_quad(Quads& Q, const TileVec& tiles, size_t b, size_t e) {
  const size_t q = (size_t)Q.count++;
  Q.cols.resize((q + 1) * 64, -1);
  Q.a.resize((q + 1) * 64 * 8, 0);
  Q.idx.resize((q + 1) * 64, 0);
  for (size_t lb = 0; lb < 4 && b + lb < e; ++lb) {
    const Lowering::Tile& t = tiles[b + lb];
    for (int k = 0; k < 16; ++k) Q.cols[q * 64 + lb * 16 + k] = t.cols[k];
    for (int r = 0; r < 16; ++r) {
      const size_t lane = q * 64 + lb * 16 + r;
      uint32_t ix = 0;
      for (int g = 0; g < 4; ++g) {
        int pos[2] = {0, 1};
        float val[2] = {0.f, 0.f};
        int n = 0;
        for (int p = 0; p < 4; ++p)
          if (Lowering::tile_has(t, r, 4 * g + p)) {
            pos[n] = p;
            val[n] = t.a[r * 16 + 4 * g + p];
            ++n;
          }
        if (n == 1 && pos[0] != 0) {   // one entry at p > 0: a zero at 0 first
          pos[1] = pos[0];
          val[1] = val[0];
          pos[0] = 0;
          val[0] = 0.f;
        } else if (n == 1) {
          pos[1] = 1;
          val[1] = 0.f;
        }
        for (int h = 0; h < 2; ++h) {
          Q.a[lane * 8 + 2 * g + h] = trs::half_bits(val[h]);
          ix |= (uint32_t)pos[h] << (2 * (2 * g + h));
        }
      }
      Q.idx[lane] = (uint16_t)ix;
    }
  }
}

// Entries stored by tile t, rows < m: the present bits (tile_add sets each once per entry).
int64_t tile_present(const Lowering::Tile& t) {
  int64_t c = 0;
  for (int i = 0; i < 4; ++i) c += __builtin_popcountll(t.present[i]);
  return c;
}

// Tile entries in row r (0..15) of tile t.
int tile_row_entries(const Lowering::Tile& t, int r) {
  return __builtin_popcountll((t.present[r / 4] >> ((r % 4) * 16)) & 0xffffull);
}

// Where the device lowering writes (device addresses inside the plan; null = not in this plan).
struct DeviceOut {
  const int32_t* main_rowptr = nullptr;
  int32_t* col = nullptr;
  uint16_t* val = nullptr;        // SpMM: fp16 values
  int32_t* res_pos = nullptr;     // SDDMM with tiles: output index of each residual entry
  int32_t* x_pos = nullptr;       // SDDMM split part: output index of each sub-row entry
  int64_t x_base = 0;             // x_pos[i] belongs to entry x_base + i
  int32_t* tile_pos = nullptr;    // SDDMM with tiles: output index of each stored tile slot, else -1
  bool compact = true;            // SpMM: split rows only in their sub-rows
  int32_t* x_src = nullptr;       // SDDMM split part: its buffer index of each split-row entry ...
  const std::vector<int32_t>* merge_off = nullptr;   // ... counted from merge_off[split row index]
};

// Device half of the device lowering: the input CSR of rows [0, m) goes up once, the kept tiles'
// entries are flagged in it, and every row is written to its placed position -- main rows without
// their flagged entries, split rows scattered into their XCD sub-rows.  Outputs follow the input
// CSR order, so an entry's output index is its CSR index.  Temporaries live in one allocation
// freed before returning.
Status residual_on_device(const CsrSource& f, int32_t m, const TileVec& tiles,
                          int64_t expect_marked, const Placement& PL, const DeviceOut& o) {
  const int32_t rows = std::min(m, f.rows);
  const int64_t cnnz = f.rowptr[rows];
  std::vector<int32_t> rp((size_t)m + 1, (int32_t)cnnz);
  std::copy(f.rowptr, f.rowptr + rows + 1, rp.begin());
  std::vector<trs::TileEntries> te(tiles.size());
  for (size_t i = 0; i < tiles.size(); ++i) {
    te[i] = trs::TileEntries{};
    te[i].row0 = tiles[i].row0;
    std::copy(tiles[i].cols, tiles[i].cols + 16, te[i].cols);
    std::copy(tiles[i].present, tiles[i].present + 4, te[i].present);
  }
  std::vector<int32_t> split_index((size_t)m, -1);
  for (size_t i = 0; i < PL.split_rows.size(); ++i) split_index[PL.split_rows[i]] = (int32_t)i;
  Blob tmp;
  const size_t o_rp = tmp.add(rp);
  // columns and values go up unless they are on the device already
  const size_t o_col = tmp.add_raw(f.d_col ? nullptr : f.col, f.d_col ? 0 : (size_t)cnnz * 4);
  const bool up_val = o.val && !f.d_val;
  const size_t o_val = tmp.add_raw(up_val ? f.val : nullptr, up_val ? (size_t)cnnz * 4 : 0);
  const size_t o_te = tmp.add(te);
  const size_t o_si = tmp.add(split_index);
  const size_t o_cur = tmp.add(PL.cursor);
  const size_t o_moff = o.x_src ? tmp.add(*o.merge_off) : 0;
  // entry flags as bytes of 32-bit words (the marking kernel sets them with word atomics), then
  // the count of entries marked
  const size_t flag_bytes = ((size_t)cnnz + 3) & ~size_t(3);
  const size_t o_flag = tmp.add_raw(nullptr, flag_bytes + 256);
  void* dmem = nullptr;
  if (hipMalloc(&dmem, tmp.size()) != hipSuccess) {
    (void)hipGetLastError();
    return fail(kLowerOnHost, "device lowering temporaries: hipMalloc failed");
  }
  unsigned char* base = static_cast<unsigned char*>(dmem);
  auto done = [&](Status st) {
    (void)hipFree(dmem);
    return st;
  };
  if (!copy_pieces(tmp, dmem) || hipMemset(base + o_flag, 0, flag_bytes + 256) != hipSuccess)
    return done(fail(TRS_EDEVICE, "device lowering: upload failed"));
  const int32_t* d_rp = reinterpret_cast<const int32_t*>(base + o_rp);
  const int32_t* d_col = f.d_col ? f.d_col : reinterpret_cast<const int32_t*>(base + o_col);
  uint32_t* d_flag = reinterpret_cast<uint32_t*>(base + o_flag);
  uint32_t* d_marked = reinterpret_cast<uint32_t*>(base + o_flag + flag_bytes);
  if (!tiles.empty()) {
    if (o.tile_pos && hipMemset(o.tile_pos, 0xff, tiles.size() * 256 * sizeof(int32_t)) != hipSuccess)
      return done(fail(TRS_EDEVICE, "device lowering: tile slot clear failed"));
    if (trs::launch_mark_tile_entries(reinterpret_cast<const trs::TileEntries*>(base + o_te), (int32_t)tiles.size(), m,
                                      d_rp, d_col, d_flag, d_marked, o.tile_pos, nullptr) != hipSuccess)
      return done(fail(TRS_EDEVICE, "device lowering: tile marking launch failed"));
    uint32_t marked = 0;
    if (hipMemcpy(&marked, d_marked, 4, hipMemcpyDeviceToHost) != hipSuccess)
      return done(fail(TRS_EDEVICE, "device lowering: tile marking failed"));
    // every kept tile entry found once in the CSR: then each row loses exactly its tile entries
    // and the placement below stays inside the rows' ranges
    if ((int64_t)marked != expect_marked)
      return done(fail(kLowerOnHost, "device lowering: tiles and input CSR disagree"));
  }
  trs::PlaceEntries a;
  a.m = m;
  a.rowptr = d_rp;
  a.col = d_col;
  a.val = !o.val ? nullptr : f.d_val ? f.d_val : reinterpret_cast<const float*>(base + o_val);
  a.flag = tiles.empty() ? nullptr : reinterpret_cast<const uint8_t*>(d_flag);
  a.main_rowptr = o.main_rowptr;
  a.split_index = reinterpret_cast<const int32_t*>(base + o_si);
  a.cursor = reinterpret_cast<const int32_t*>(base + o_cur);
  a.col_out = o.col;
  a.val_out = o.val;
  a.res_pos = o.res_pos;
  a.x_pos = o.x_pos;
  a.x_base = o.x_base;
  a.compact = o.compact ? 1 : 0;
  if (o.x_src) {
    a.merge_off = reinterpret_cast<const int32_t*>(base + o_moff);
    a.x_src = o.x_src;
  }
  if (trs::launch_place_entries(a, nullptr) != hipSuccess || hipStreamSynchronize(nullptr) != hipSuccess)
    return done(fail(TRS_EDEVICE, "device lowering: entry placement failed"));
  return done(Status{});
}

// Device lowering, host side: the column range check the host lowering makes (a residual or tile
// column outside [0, n) is TRS_ERANGE) over the input CSR's rows [0, m), and their lengths (rows
// beyond the input's are empty).
Status input_rows(const CsrSource& src, Lowering& L, std::vector<int32_t>& csr_len) {
  const int32_t m = L.m;
  const int32_t rows = std::min(m, src.rows);
  const int64_t cnnz = src.rowptr[rows];
  if (src.col) {
    const int T = lowering_threads();
    std::vector<int64_t> bad((size_t)T, INT64_MAX);
    parallel_parts(T, cnnz, 1 << 16, [&](int t) { return cnnz * t / T; }, [&](int64_t b, int64_t e, int t) {
      for (int64_t q = b; q < e; ++q)
        if (src.col[q] < 0 || src.col[q] >= L.n) {
          bad[t] = q;
          break;
        }
    });
    const int64_t q = *std::min_element(bad.begin(), bad.end());
    if (q != INT64_MAX) L.check_col(src.col[q]);
  } else if (cnnz > 0) {
    // the first column outside [0, n), found where the columns are
    void* d = nullptr;
    if (hipMalloc(&d, 8) != hipSuccess) {
      (void)hipGetLastError();
      return fail(kLowerOnHost, "device lowering temporaries: hipMalloc failed");
    }
    unsigned long long first = ~0ull;
    int32_t c = 0;
    const bool ok = hipMemcpy(d, &first, 8, hipMemcpyHostToDevice) == hipSuccess &&
                    trs::launch_check_columns(src.d_col, cnnz, L.n, static_cast<unsigned long long*>(d), nullptr) ==
                        hipSuccess &&
                    hipMemcpy(&first, d, 8, hipMemcpyDeviceToHost) == hipSuccess &&
                    (first == ~0ull || hipMemcpy(&c, src.d_col + first, 4, hipMemcpyDeviceToHost) == hipSuccess);
    (void)hipFree(d);
    if (!ok) return fail(TRS_EDEVICE, "device lowering: column check failed");
    if (first != ~0ull) L.check_col(c);
  }
  if (!L.st.ok()) return L.st;
  csr_len.assign((size_t)m, 0);
  for (int32_t r = 0; r < rows; ++r) csr_len[r] = src.rowptr[r + 1] - src.rowptr[r];
  // a tile slot added twice (duplicate input entries) holds a sum the input CSR does not
  for (const auto& t : L.tiles)
    if (t.nnz != tile_present(t)) return fail(kLowerOnHost, "device lowering: a tile slot holds two entries");
  return Status{};
}

// Residual row pointers of the device lowering: the input rows minus the tiles' entries; a
// negative length means the tiles hold entries the input CSR lacks.
Status residual_rows(const std::vector<int32_t>& csr_len, const TileVec& tiles, int32_t m,
                     std::vector<int32_t>& rowptr, int64_t* tile_entries) {
  std::vector<int32_t> len(csr_len);
  int64_t te = 0;
  for (const auto& t : tiles) {
    te += tile_present(t);
    for (int r = 0; r < 16 && t.row0 + r < m; ++r) len[t.row0 + r] -= tile_row_entries(t, r);
  }
  rowptr.assign((size_t)m + 1, 0);
  for (int32_t r = 0; r < m; ++r) {
    if (len[r] < 0) return fail(kLowerOnHost, "device lowering: tiles hold entries the input CSR lacks");
    rowptr[r + 1] = rowptr[r] + len[r];
  }
  if (tile_entries) *tile_entries = te;
  return Status{};
}

// Hot-row staging of an uploaded plan whose entry arrays (task kernel column ids) are
// d.col[0, total): count the gathers of each column on the device (the residual entries of
// MFMA-window rows excluded: the window kernel gathers those through the plain ids), choose the hot
// columns on the host (most gathered first, ties by column), renumber their entries ~rank into a
// copy of the column ids (the plain ids stay for the window kernel and for widths that do not
// stage).
Status stage_hot_rows(trs_plan* P, int64_t total, const trs_plan_options& opt) {
  trs::DevicePlan& d = P->dp;
  if (opt.hot_rows < 0 || total <= 0 || d.n <= 0) return Status{};
  const int32_t n = d.n;
  const int32_t want = opt.hot_rows > 0 ? std::min(opt.hot_rows, n) : std::min(kHotRows, n / kHotColumnShare);
  // the choice costs O(n) memory (a count per column, here and on the host): not for matrices with
  // far more columns than entries, whose columns are mostly unused anyway
  if (want <= 0 || (int64_t)n > kHotMaxColumnsPerEntry * total) return Status{};
  // histogram copies against atomic contention on hot columns, within kCountCopyBytes
  const int copies = (int)std::max<int64_t>(1, std::min<int64_t>(kCountCopies, kCountCopyBytes / ((int64_t)n * 4)));
  int32_t* counts = nullptr;
  if (hipMalloc(&counts, (size_t)n * 4 * copies) != hipSuccess) {
    (void)hipGetLastError();
    return fail(TRS_ENOMEM, "hot rows: hipMalloc of the column counts failed");
  }
  auto done = [&](Status st) {
    (void)hipFree(counts);
    return st;
  };
  std::vector<int32_t> cnt((size_t)n);
  if (hipMemset(counts, 0, (size_t)n * 4 * copies) != hipSuccess ||
      trs::launch_count_columns(d.col, total, n, counts, copies, nullptr) != hipSuccess ||
      trs::launch_uncount_windows(d.mwin, d.nmwin, d.m, d.rowptr, d.col, n, counts, nullptr) != hipSuccess ||
      hipMemcpy(cnt.data(), counts, (size_t)n * 4, hipMemcpyDeviceToHost) != hipSuccess)
    return done(fail(TRS_EDEVICE, "hot rows: column count failed"));
  // the task kernels' gathers: every entry but the window rows' residual entries
  const int64_t task_entries = total - P->stats.window_csr_nnz;
  // The `want` first columns in the order (count desc, column asc) among those gathered at least
  // twice (a column gathered once gains nothing from a copy), found through a histogram of the
  // counts: every column above the cut count t, then those at t in column order, each placed in
  // its count's bucket in one pass over the columns (ascending, so each bucket is in column
  // order).  Counts from kCountCap on share the histogram's last bucket and are ordered by a sort
  // of their own.
  constexpr int32_t kCountCap = 1 << 16;
  std::vector<int32_t> hc((size_t)kCountCap + 1, 0);
  int64_t capped_entries = 0;
  for (int32_t c = 0; c < n; ++c) {
    const int32_t v = cnt[c];
    if (v >= kCountCap) capped_entries += v;
    if (v >= 2) hc[(size_t)(v < kCountCap ? v : kCountCap)]++;
  }
  // the automatic choice stages nothing when the chosen columns take too few of the gathers
  auto too_few = [&](int64_t entries) {
    return opt.hot_rows == 0 && entries * 10 < task_entries * kHotMinShare10;
  };
  int64_t taken = 0, hot_entries = 0;
  int32_t t = kCountCap;   // the lowest count taken in full is above t
  for (; t >= 2 && taken + hc[(size_t)t] <= want; --t) taken += hc[(size_t)t];
  auto before = [&](int32_t a, int32_t b) { return cnt[a] != cnt[b] ? cnt[a] > cnt[b] : a < b; };
  std::vector<int32_t> hot;
  if (t == kCountCap && hc[(size_t)kCountCap] > want) {
    // more capped columns than wanted: take them all and cut by the exact order
    for (int32_t c = 0; c < n; ++c)
      if (cnt[c] >= kCountCap) hot.push_back(c);
    std::nth_element(hot.begin(), hot.begin() + want, hot.end(), before);
    hot.resize((size_t)want);
    std::sort(hot.begin(), hot.end(), before);
  } else {
    const int32_t lo = std::max(t, 2);               // lowest count taken
    int64_t at_t = t >= 2 ? want - taken : 0;        // columns of count t still taken, lowest ids first
    const int64_t ncap = t < kCountCap ? hc[(size_t)kCountCap] : 0;
    // their entries, from the histogram, before any column is placed
    int64_t chosen = capped_entries + (t >= 2 ? at_t * t : 0);
    for (int32_t v = std::max(t + 1, 2); v < kCountCap; ++v) chosen += (int64_t)v * hc[(size_t)v];
    if (taken + (t >= 2 ? at_t : 0) == 0 || too_few(chosen)) return done(Status{});
    std::vector<int64_t> off((size_t)kCountCap, 0);  // next slot of each count below the cap
    int64_t pos = ncap;
    for (int32_t v = kCountCap - 1; v >= lo; --v) {
      off[(size_t)v] = pos;
      pos += v == t ? at_t : hc[(size_t)v];
    }
    hot.resize((size_t)pos);
    std::vector<int32_t> capped;
    capped.reserve((size_t)ncap);
    for (int32_t c = 0; c < n; ++c) {
      const int32_t v = cnt[c];
      if (v < lo) continue;
      if (v >= kCountCap) capped.push_back(c);
      else if (v > t) hot[(size_t)off[(size_t)v]++] = c;
      else if (at_t > 0) {   // v == t
        hot[(size_t)off[(size_t)v]++] = c;
        --at_t;
      }
    }
    std::sort(capped.begin(), capped.end(), before);
    std::copy(capped.begin(), capped.end(), hot.begin());
  }
  for (int32_t c : hot) hot_entries += cnt[c];
  if (hot.empty() || too_few(hot_entries)) return done(Status{});
  std::vector<int32_t> rank((size_t)n, -1);
  for (size_t i = 0; i < hot.size(); ++i) rank[hot[i]] = (int32_t)i;
  // renumbered ids with the 256-byte tail every entry array has (staged streams read whole
  // 16-byte chunks that may end past it), then the hot list
  const size_t col_bytes = (((size_t)total * 4 + 255) & ~size_t(255)) + 256;
  const size_t bytes = col_bytes + hot.size() * 4;
  if (hipMalloc(&P->hmem, bytes) != hipSuccess) {
    P->hmem = nullptr;
    (void)hipGetLastError();
    return done(fail(TRS_ENOMEM, "hot rows: hipMalloc of " + std::to_string(bytes) + " bytes failed"));
  }
  int32_t* hot_col = static_cast<int32_t*>(P->hmem);
  int32_t* hot_rows = reinterpret_cast<int32_t*>(static_cast<unsigned char*>(P->hmem) + col_bytes);
  if (hipMemcpy(counts, rank.data(), (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(hot_rows, hot.data(), hot.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemset(static_cast<unsigned char*>(P->hmem) + (size_t)total * 4, 0, col_bytes - (size_t)total * 4) !=
          hipSuccess ||
      trs::launch_renumber_hot(d.col, total, n, counts, hot_col, nullptr) != hipSuccess ||
      hipStreamSynchronize(nullptr) != hipSuccess)
    return done(fail(TRS_EDEVICE, "hot rows: renumbering failed"));
  d.hot_col = hot_col;
  d.hot_rows = hot_rows;
  d.nhot = (int32_t)hot.size();
  P->stats.hot_rows = d.nhot;
  P->stats.hot_entries = hot_entries;
  P->stats.device_bytes += (int64_t)bytes;
  return done(Status{});
}

// Residual CSR + tasks + MFMA windows -> device plan.  With src (the format that holds its input
// CSR), L carries the tiles only and the residual -- the input CSR minus the kept tiles' entries --
// is built on the device; the plan equals the host lowering's (same arrays, same statistics).
// Tiles whose rows all lie at or past m hold no entries (the lowerings add none there: reference
// kernels drop rows >= mOri).  They come from windows past the plan's rows, and from formats of
// windows under 16 rows, whose t_window_row is the window id * 16 (block_online.cpp:494) and so
// runs to twice the rows and more.
void drop_tiles_past_m(Lowering& L) {
  L.tiles.erase(std::remove_if(L.tiles.begin(), L.tiles.end(), [&](const Lowering::Tile& t) { return t.row0 >= L.m; }),
                L.tiles.end());
}

Status finalize(Lowering& L, const trs_plan_options& opt, trs_plan** out, const CsrSource* src = nullptr) {
  if (!L.st.ok()) return L.st;
  drop_tiles_past_m(L);
  const int32_t m = L.m;
  // device lowering: row lengths of the input CSR (rows beyond its rows are empty)
  std::vector<int32_t> csr_len;
  if (src) {
    const Status is = input_rows(*src, L, csr_len);
    if (!is.ok()) return is;
  }

  // MFMA windows: 16-row blocks owning at least one tile (tile order inside a window kept).
  sort_tiles(L.tiles);
  const int32_t nblocks = (m + 15) / 16;
  std::vector<uint8_t> owned(nblocks, 0);
  for (const auto& t : L.tiles) owned[t.row0 / 16] = 1;

  // Hand a tile-owning block back to the residual path when one of its residual rows is long:
  // the window kernel walks each residual row with one lane group, so a long row would keep the
  // whole workgroup waiting (hub windows of power-law graphs).  Decided on the residual row
  // lengths before the demoted tiles' entries join the residual.
  const int row_cap = opt.window_row_cap > 0 ? opt.window_row_cap : 128;
  if (!L.tiles.empty()) {
    std::vector<int32_t> len((size_t)m, 0);
    if (src) {
      // input row length minus the tile entries of the row
      std::vector<int32_t> rp;
      const Status rs = residual_rows(csr_len, L.tiles, m, rp, nullptr);
      if (!rs.ok()) return rs;
      for (int32_t r = 0; r < m; ++r) len[r] = rp[r + 1] - rp[r];
    } else {
      for (int32_t r : L.row) len[r]++;
    }
    std::vector<uint8_t> demote(nblocks, 0);
    bool any_demote = false;
    for (int32_t b = 0; b < nblocks; ++b) {
      if (!owned[b]) continue;
      int64_t longest = 0, sum = 0, rows = 0;
      for (int32_t r = b * 16; r < std::min(m, b * 16 + 16); ++r) {
        longest = std::max<int64_t>(longest, len[r]);
        sum += len[r];
        ++rows;
      }
      // only a row much longer than its window's others stalls the workgroup
      demote[b] = longest > row_cap && (longest * rows > (int64_t)kWindowRowRatio * sum ||
                                        longest > kWindowRowHardFactor * row_cap);
      any_demote |= demote[b] != 0;
    }
    if (any_demote) {
      TileVec kept;
      for (const auto& t : L.tiles) {
        if (!demote[t.row0 / 16]) { kept.push_back(t); continue; }
        owned[t.row0 / 16] = 0;
        if (src) continue;   // its entries stay in the input CSR
        for (int r = 0; r < 16; ++r)
          for (int k = 0; k < 16; ++k)
            if (t.cols[k] >= 0 && Lowering::tile_has(t, r, k)) L.add((int64_t)t.row0 + r, t.cols[k], t.a[r * 16 + k]);
      }
      L.tiles.swap(kept);
      if (!L.st.ok()) return L.st;
    }
  }
  // residual CSR sorted by (row, column); equal keys keep insertion order
  std::vector<int32_t> rowptr;
  std::vector<int32_t> col;
  std::vector<uint16_t> val;
  int64_t nent = 0;
  int64_t expect_marked = 0;
  if (src) {
    // the input rows minus the kept tiles' entries (columns ascending, as the host sort leaves them)
    const Status rs = residual_rows(csr_len, L.tiles, m, rowptr, &expect_marked);
    if (!rs.ok()) return rs;
    nent = rowptr[m];
  } else {
    nent = (int64_t)L.row.size();
    if (nent > INT32_MAX) return fail(TRS_ERANGE, "more than 2^31 residual entries");
    col.resize((size_t)nent);
    val.resize((size_t)nent);
    std::vector<int64_t> perm;
    residual_csr(L, false, rowptr, perm);
    parallel_chunks(nent, [&](int64_t b, int64_t e, int) {
      for (int64_t i = b; i < e; ++i) {
        col[i] = L.col[perm[i]];
        val[i] = trs::half_bits(L.val[perm[i]]);
      }
    });
  }
  std::vector<trs::MfmaWindow> mwin;
  // sptc_sparse: a window's 2:4 tiles go behind its dense ones and into quads of four
  const bool sparse = opt.sptc_sparse != 0;
  std::vector<int32_t> win_quad(1, 0);
  Quads Q;
  int64_t sparse_tiles = 0;
  for (size_t i = 0; i < L.tiles.size();) {
    size_t j = i;
    while (j < L.tiles.size() && L.tiles[j].row0 == L.tiles[i].row0) ++j;
    size_t dense_end = j;
    if (sparse) {
      dense_end = (size_t)(std::stable_partition(L.tiles.begin() + i, L.tiles.begin() + j,
                                                 [](const Lowering::Tile& t) { return !is_two_four(t); }) -
                           L.tiles.begin());
      for (size_t b = dense_end; b < j; b += 4) add_quad(Q, L.tiles, b, std::min(j, b + 4));
      sparse_tiles += (int64_t)(j - dense_end);
      win_quad.push_back(Q.count);
    }
    mwin.push_back({L.tiles[i].row0, (int32_t)i, (int32_t)dense_end, 0});
    i = j;
  }
  trs::array<int32_t> tile_cols(L.tiles.size() * 16);   // written whole below, in parallel
  trs::array<uint16_t> tile_a(L.tiles.size() * 256);
  int64_t mfma_nnz = 0;
  for (const auto& t : L.tiles) mfma_nnz += t.nnz;
  parallel_tiles((int64_t)L.tiles.size(), [&](int64_t b, int64_t e, int) {
    for (int64_t t = b; t < e; ++t) {
      for (int k = 0; k < 16; ++k) tile_cols[t * 16 + k] = L.tiles[t].cols[k];
      trs::half_bits_n(L.tiles[t].a, &tile_a[t * 256], 256);   // F16C, the same bits as half_bits
    }
  });

  // residual tasks over rows not owned by an MFMA window
  // XCD column split for SpMM (each sub-row costs a partial slot of 4 K bytes written and read back)
  const int32_t split_min = opt.xcd_split < 0 ? 0 : opt.xcd_split > 0 ? opt.xcd_split : kSpmmSplitMin;
  const int32_t reuse = opt.xcd_split == 0 ? kSplitMinReuse : 0;
  Status pst;
  const Placement PL =
      src ? place_entries(rowptr, src->col, src->rowptr, m, L.n, owned, true, split_min, reuse,
                          src->col ? nullptr : src->d_col, &pst)
          : place_entries(rowptr, col.data(), rowptr.data(), m, L.n, owned, true, split_min, reuse);
  if (!pst.ok()) return pst;
  std::vector<int32_t> col2;
  std::vector<uint16_t> val2;
  if (!src) move_entries(PL, rowptr, col.data(), val.data(), m, col2, &val2, nullptr);
  Tasks T = build_tasks(PL, rowptr, m, owned, true, opt);
  if (!T.st.ok()) return T.st;
  const int32_t slots = T.slots;
  const int64_t split_rows = T.split_rows;

  // one device allocation
  Blob blob;
  const size_t o_rowptr = blob.add(PL.main_rowptr);
  const size_t o_col = src ? blob.add_raw(nullptr, (size_t)PL.total * 4) : blob.add(col2);
  const size_t o_val = src ? blob.add_raw(nullptr, (size_t)PL.total * 2) : blob.add(val2);
  const size_t o_tasks = blob.add(T.tasks);
  const size_t o_xtasks = blob.add(T.xtasks);
  const size_t o_xrowptr = blob.add(PL.xrowptr);
  const size_t o_fix = blob.add(T.fix);
  const size_t o_wfix = blob.add(T.wfix);
  const size_t o_slots = blob.add(T.slot_list);
  const size_t o_mwin = blob.add(mwin);
  const size_t o_tcol = blob.add(tile_cols);
  const size_t o_ta = blob.add(tile_a);
  const size_t o_wq = blob.add(win_quad);
  const size_t o_qcol = blob.add(Q.cols);
  const size_t o_qa = blob.add(Q.a);
  const size_t o_qidx = blob.add(Q.idx);
  trs_plan* P = nullptr;
  {
    const Status us = upload(blob, P);
    if (!us.ok()) return us;
  }
  unsigned char* base = static_cast<unsigned char*>(P->dmem);
  if (src) {
    DeviceOut o;
    o.main_rowptr = reinterpret_cast<const int32_t*>(base + o_rowptr);
    o.col = reinterpret_cast<int32_t*>(base + o_col);
    o.val = reinterpret_cast<uint16_t*>(base + o_val);
    const Status ds = residual_on_device(*src, m, L.tiles, expect_marked, PL, o);
    if (!ds.ok()) {
      delete P;
      return ds;
    }
  }
  trs::DevicePlan& d = P->dp;
  d.m = m;
  d.n = L.n;
  d.nnz_csr = nent;
  d.rowptr = reinterpret_cast<const int32_t*>(base + o_rowptr);
  d.col = reinterpret_cast<const int32_t*>(base + o_col);
  d.val = reinterpret_cast<const uint16_t*>(base + o_val);
  d.tasks = reinterpret_cast<const trs::Task*>(base + o_tasks);
  d.ntasks = (int32_t)T.tasks.size();
  d.x_tasks = reinterpret_cast<const trs::Task*>(base + o_xtasks);
  d.x_ntasks = (int32_t)T.xtasks.size();
  d.x_rowptr = reinterpret_cast<const int32_t*>(base + o_xrowptr);
  std::copy(T.xq, T.xq + trs::kXcds + 1, d.xq);
  d.x_task_max = T.xtask_max;
  d.fixups = reinterpret_cast<const trs::Fixup*>(base + o_fix);
  d.nfixups = (int32_t)T.fix.size();
  d.wfixups = reinterpret_cast<const trs::Fixup*>(base + o_wfix);
  d.nwfixups = (int32_t)T.wfix.size();
  d.slot_list = reinterpret_cast<const int32_t*>(base + o_slots);
  d.partial_slots = slots;
  d.mwin = reinterpret_cast<const trs::MfmaWindow*>(base + o_mwin);
  d.nmwin = (int32_t)mwin.size();
  d.tile_cols = reinterpret_cast<const int32_t*>(base + o_tcol);
  d.tile_a = reinterpret_cast<const uint16_t*>(base + o_ta);
  d.ntiles = (int32_t)L.tiles.size();
  if (Q.count > 0) {
    d.win_quad = reinterpret_cast<const int32_t*>(base + o_wq);
    d.quad_cols = reinterpret_cast<const int32_t*>(base + o_qcol);
    d.quad_a = reinterpret_cast<const uint16_t*>(base + o_qa);
    d.quad_idx = reinterpret_cast<const uint16_t*>(base + o_qidx);
    d.nquads = Q.count;
  }
  d.feature_lanes = opt.feature_lanes;
  d.split_dispatch = opt.split_dispatch != 0;
  // default: non-temporal C stores only (measured +3%); non-temporal A loads cost ~60% because
  // consecutive iterations re-read the same col/val cache lines
  d.task_nnz = T.task_nnz;
  d.task_max = T.task_max;
  d.streaming = opt.streaming < 0 ? 2 : opt.streaming;
  d.xcd_run = opt.xcd_run > 0 ? opt.xcd_run : 16;
  d.stage = opt.stage < 0 ? -1 : 0;
  d.occupancy = opt.occupancy < 0 ? -1 : opt.occupancy == 0 ? 0 : std::min(8, std::max(2, opt.occupancy));
  P->csr_only = false;
  trs_plan_stats& s = P->stats;
  s.m = m;
  s.n = L.n;
  s.csr_nnz = nent;
  s.mfma_tiles = (int64_t)L.tiles.size();
  s.mfma_nnz = mfma_nnz;
  s.nnz = nent + mfma_nnz;
  s.tasks = (int64_t)(T.tasks.size() + T.xtasks.size());
  s.split_rows = split_rows;
  s.partial_slots = slots;
  s.device_bytes = (int64_t)blob.size();
  s.mfma_windows = (int64_t)mwin.size();
  int64_t wnnz = 0;
  for (const auto& w : mwin)
    for (int32_t r = w.row0; r < std::min(m, w.row0 + 16); ++r) wnnz += rowptr[r + 1] - rowptr[r];
  s.window_csr_nnz = wnnz;
  s.device_lowered = src ? 1 : 0;
  s.sparse_tiles = sparse_tiles;
  const Status hs = stage_hot_rows(P, PL.total, opt);
  if (!hs.ok()) {
    delete P;
    return hs;
  }
  *out = P;
  return Status{};
}

// SDDMM plan: residual CSR (+ the output index of each entry when tiles exist) and independent
// tiles with the output index of each stored slot.  Outputs follow the (row, column) order of all
// entries, i.e. the input CSR order for canonical input; keep_order keeps a plain CSR as given.
//
// With src (the input CSR of the format), L carries the tiles only and the residual is
// built on the device as for SpMM plans; the output index of an entry is then its input CSR index.
Status finalize_sddmm(Lowering& L, const trs_plan_options& opt, bool keep_order, trs_plan** out,
                      const CsrSource* src = nullptr) {
  if (!L.st.ok()) return L.st;
  drop_tiles_past_m(L);
  std::vector<int32_t> csr_len;
  if (src) {
    const Status is = input_rows(*src, L, csr_len);
    if (!is.ok()) return is;
  }
  // Tiles pay for themselves only when they carry a real share of the entries: otherwise the
  // per-entry output index they force on the residual costs more than MFMA saves (measured on
  // R-MAT 2^20, K=128: tiles with 2.7% of the entries made SDDMM 15% slower).  Hand them back.
  {
    int64_t tile_entries = 0;
    for (const auto& t : L.tiles) tile_entries += t.nnz;
    const int64_t total = src ? (int64_t)std::accumulate(csr_len.begin(), csr_len.end(), (int64_t)0)
                              : tile_entries + (int64_t)L.row.size();
    if (!L.tiles.empty() && (double)tile_entries < 0.10 * (double)total) {
      if (src) L.tiles.clear();   // their entries stay in the input CSR
      for (const auto& t : L.tiles)
        for (int r = 0; r < 16; ++r)
          for (int k = 0; k < 16; ++k)
            if (t.cols[k] >= 0 && Lowering::tile_has(t, r, k)) L.add((int64_t)t.row0 + r, t.cols[k], t.a[r * 16 + k]);
      L.tiles.clear();
    }
  }
  const int32_t m = L.m;
  std::vector<int32_t> rowptr;
  std::vector<int32_t> col;
  int64_t nent = 0;
  int64_t expect_marked = 0;
  if (src) {
    const Status rs = residual_rows(csr_len, L.tiles, m, rowptr, &expect_marked);
    if (!rs.ok()) return rs;
    nent = rowptr[m];
  } else {
    nent = (int64_t)L.row.size();
    std::vector<int64_t> perm;
    residual_csr(L, keep_order && L.tiles.empty(), rowptr, perm);
    col.resize((size_t)nent);
    parallel_chunks(nent, [&](int64_t b, int64_t e, int) {
      for (int64_t i = b; i < e; ++i) col[i] = L.col[perm[i]];
    });
  }

  // tile entries in (row, column) order, merged with the residual rows
  struct TE { int32_t row, col, slot; };   // slot = tile * 256 + r * 16 + k
  std::vector<TE> te;
  for (size_t t = 0; t < L.tiles.size() && !src; ++t)
    for (int r = 0; r < 16; ++r)
      for (int k = 0; k < 16; ++k)
        if (L.tiles[t].cols[k] >= 0 && Lowering::tile_has(L.tiles[t], r, k) && L.tiles[t].row0 + r < m)
          te.push_back({L.tiles[t].row0 + r, L.tiles[t].cols[k], (int32_t)(t * 256 + r * 16 + k)});
  std::sort(te.begin(), te.end(), [](const TE& a, const TE& b) { return a.row != b.row ? a.row < b.row : a.col < b.col; });
  const int64_t tile_entries = src ? expect_marked : (int64_t)te.size();
  if (nent + tile_entries > INT32_MAX) return fail(TRS_ERANGE, "more than 2^31 entries");
  const bool with_pos = tile_entries > 0;
  std::vector<int32_t> res_pos, tile_pos, tile_row0, tile_cols;
  if (src && with_pos) {
    for (const auto& t : L.tiles) {
      tile_row0.push_back(t.row0);
      tile_cols.insert(tile_cols.end(), t.cols, t.cols + 16);
    }
  }
  if (!src && !te.empty()) {
    res_pos.resize(nent);
    tile_pos.assign(L.tiles.size() * 256, -1);
    int32_t next = 0;
    size_t ti = 0;
    for (int32_t r = 0; r < m; ++r) {
      int32_t j = rowptr[r];
      while (j < rowptr[r + 1] || (ti < te.size() && te[ti].row == r)) {
        const bool take_tile = ti < te.size() && te[ti].row == r && (j >= rowptr[r + 1] || te[ti].col < col[j]);
        if (take_tile) tile_pos[te[ti++].slot] = next++;
        else res_pos[j++] = next++;
      }
    }
    for (const auto& t : L.tiles) {
      tile_row0.push_back(t.row0);
      tile_cols.insert(tile_cols.end(), t.cols, t.cols + 16);
    }
  }
  // SDDMM sub-rows write their own outputs (no partial slot)
  const int32_t split_min = opt.xcd_split < 0 ? 0 : opt.xcd_split > 0 ? opt.xcd_split : kSddmmSplitMin;
  // the split part's outputs are contiguous runs of the residual order: only without tiles, whose
  // merge interleaves output positions
  // (device lowering: split rows hold no tile entries -- there are none -- so their columns are
  // the input rows')
  const int32_t split = with_pos ? 0 : split_min;
  const int32_t reuse = opt.xcd_split == 0 ? kSplitMinReuse : 0;
  Status pst;
  const Placement PL =
      src ? place_entries(rowptr, src->col, src->rowptr, m, L.n, {}, false, split, reuse,
                          src->col ? nullptr : src->d_col, &pst)
          : place_entries(rowptr, col.data(), rowptr.data(), m, L.n, {}, false, split, reuse);
  if (!pst.ok()) return pst;
  // the split rows' outputs merged from the split part's own buffer: merge_off[i] = entries of the
  // split rows before split row i; tasks of at most trs::kMergeTaskEntries output indices
  std::vector<int32_t> merge_off(PL.split_rows.size() + 1, 0);
  std::vector<trs::MergeTask> merge;
  for (size_t i = 0; i < PL.split_rows.size(); ++i) {
    const int32_t r = PL.split_rows[i];
    const int32_t b = rowptr[r], e = rowptr[r + 1];
    merge_off[i + 1] = merge_off[i] + (e - b);
    for (int32_t q = b; q < e; q += trs::kMergeTaskEntries)
      merge.push_back({q, std::min(e, q + trs::kMergeTaskEntries), merge_off[i] + (q - b), 0});
  }
  std::vector<int32_t> col2, x_pos, x_src;
  if (!src) move_entries(PL, rowptr, col.data(), nullptr, m, col2, nullptr, &x_pos, &x_src, &merge_off);
  Tasks T = build_tasks(PL, rowptr, m, {}, false, opt);
  if (!T.st.ok()) return T.st;

  Blob blob;
  const size_t n_xpos = (size_t)(PL.total - nent);
  const size_t o_rowptr = blob.add(rowptr);
  const size_t o_col = src ? blob.add_raw(nullptr, (size_t)PL.total * 4) : blob.add(col2);
  const size_t o_tasks = blob.add(T.tasks);
  const size_t o_xtasks = blob.add(T.xtasks);
  const size_t o_xrowptr = blob.add(PL.xrowptr);
  const size_t o_xpos = src ? blob.add_raw(nullptr, n_xpos * 4) : blob.add(x_pos);
  const size_t o_xsrc = src ? blob.add_raw(nullptr, n_xpos * 4) : blob.add(x_src);
  const size_t o_merge = blob.add(merge);
  const size_t o_srow = blob.add(PL.sub_row);
  const size_t o_full = blob.add(T.full);
  const size_t o_narrow = blob.add(T.narrow);
  const size_t o_rpos = src ? blob.add_raw(nullptr, with_pos ? (size_t)nent * 4 : 0) : blob.add(res_pos);
  const size_t o_trow = blob.add(tile_row0);
  const size_t o_tcol = blob.add(tile_cols);
  const size_t o_tpos = src ? blob.add_raw(nullptr, with_pos ? L.tiles.size() * 256 * 4 : 0) : blob.add(tile_pos);
  trs_plan* P = nullptr;
  {
    const Status us = upload(blob, P);
    if (!us.ok()) return us;
  }
  unsigned char* base = static_cast<unsigned char*>(P->dmem);
  if (src) {
    DeviceOut o;
    o.main_rowptr = reinterpret_cast<const int32_t*>(base + o_rowptr);
    o.col = reinterpret_cast<int32_t*>(base + o_col);
    o.res_pos = with_pos ? reinterpret_cast<int32_t*>(base + o_rpos) : nullptr;
    o.x_pos = n_xpos ? reinterpret_cast<int32_t*>(base + o_xpos) : nullptr;
    o.x_base = nent;
    o.x_src = n_xpos ? reinterpret_cast<int32_t*>(base + o_xsrc) : nullptr;
    o.merge_off = &merge_off;
    o.tile_pos = with_pos ? reinterpret_cast<int32_t*>(base + o_tpos) : nullptr;
    o.compact = false;
    const Status ds = residual_on_device(*src, m, with_pos ? L.tiles : TileVec{}, expect_marked, PL, o);
    if (!ds.ok()) {
      delete P;
      return ds;
    }
  }
  trs::DevicePlan& d = P->dp;
  d.m = m;
  d.n = L.n;
  d.nnz_csr = nent;
  d.rowptr = reinterpret_cast<const int32_t*>(base + o_rowptr);
  d.col = reinterpret_cast<const int32_t*>(base + o_col);
  d.tasks = reinterpret_cast<const trs::Task*>(base + o_tasks);
  d.ntasks = (int32_t)T.tasks.size();
  d.x_tasks = reinterpret_cast<const trs::Task*>(base + o_xtasks);
  d.x_ntasks = (int32_t)T.xtasks.size();
  d.x_rowptr = reinterpret_cast<const int32_t*>(base + o_xrowptr);
  d.x_pos = reinterpret_cast<const int32_t*>(base + o_xpos);
  d.x_sub_row = reinterpret_cast<const int32_t*>(base + o_srow);
  d.x_src = reinterpret_cast<const int32_t*>(base + o_xsrc);
  d.merge = reinterpret_cast<const trs::MergeTask*>(base + o_merge);
  d.nmerge = (int32_t)merge.size();
  d.x_entries = (int64_t)n_xpos;
  d.full_tasks = reinterpret_cast<const trs::Task*>(base + o_full);
  d.nfull_tasks = (int32_t)T.full.size();
  d.narrow_tasks = reinterpret_cast<const trs::Task*>(base + o_narrow);
  d.nnarrow_tasks = (int32_t)T.narrow.size();
  std::copy(T.xq, T.xq + trs::kXcds + 1, d.xq);
  d.x_task_max = T.xtask_max;
  d.res_pos = with_pos ? reinterpret_cast<const int32_t*>(base + o_rpos) : nullptr;
  d.tile_row0 = with_pos ? reinterpret_cast<const int32_t*>(base + o_trow) : nullptr;
  d.tile_cols = with_pos ? reinterpret_cast<const int32_t*>(base + o_tcol) : nullptr;
  d.tile_pos = with_pos ? reinterpret_cast<const int32_t*>(base + o_tpos) : nullptr;
  d.ntiles = with_pos ? (int32_t)L.tiles.size() : 0;
  d.feature_lanes = opt.feature_lanes;
  d.split_dispatch = opt.split_dispatch != 0;
  d.streaming = opt.streaming < 0 ? 2 : (opt.streaming & 2);
  d.xcd_run = opt.xcd_run > 0 ? opt.xcd_run : 16;
  d.sddmm_unroll = opt.sddmm_unroll == 4 || opt.sddmm_unroll == 8 ? opt.sddmm_unroll : 0;
  d.stage = opt.stage < 0 ? -1 : 0;
  d.occupancy = opt.occupancy < 0 ? -1 : opt.occupancy == 0 ? 0 : std::min(8, std::max(2, opt.occupancy));
  d.task_nnz = T.task_nnz;
  d.task_max = T.task_max;
  P->csr_only = true;
  trs_plan_stats& s = P->stats;
  s.m = m;
  s.n = L.n;
  s.csr_nnz = nent;
  s.mfma_tiles = d.ntiles;
  s.mfma_nnz = tile_entries;
  s.nnz = nent + tile_entries;
  s.tasks = (int64_t)(T.tasks.size() + T.xtasks.size());
  s.split_rows = (int64_t)PL.split_rows.size();
  s.device_bytes = (int64_t)blob.size();
  s.device_lowered = src ? 1 : 0;
  const Status hs = stage_hot_rows(P, PL.total, opt);
  if (!hs.ok()) {
    delete P;
    return hs;
  }
  *out = P;
  return Status{};
}

// Every share of a builder output: TC sub-blocks, residual parts, 2:4 groups, spill.
void lower_format(Lowering& L, const trs_format& f, const trs_plan_options& o) {
  lower_tc(L, f.t_rowoff.data(), (int64_t)f.t_winrow.size(), f.t_blockoff.data(), f.t_col.data(), f.t_val.data(),
           nullptr, (int64_t)f.t_val.size(), f.t_winrow.data(), f.t_bin.data(), o.mfma_tc != 0);
  lower_residual(L, f.c_off.data(), f.c_row.data(), (int64_t)f.c_row.size(), f.c_col.data(), f.c_val.data(), nullptr,
                 (int64_t)f.c_col.size());
  lower_residual(L, f.cs_off.data(), f.cs_row.data(), (int64_t)f.cs_row.size(), f.cs_col.data(), f.cs_val.data(),
                 nullptr, (int64_t)f.cs_col.size());
  lower_groups(L, f.s_col.data(), f.s_val.data(), f.s_pos.data(), (int64_t)f.s_win.size(), f.s_win.data(),
               f.s_offsets.data(), (int64_t)f.s_offsets.size() - 1, f.window, o.mfma_sptc != 0, o.sptc_min_fill);
  for (size_t i = 0; i < f.spill_row.size() && L.st.ok(); ++i) L.add(f.spill_row[i], f.spill_col[i], f.spill_val[i]);
}

// The tiles of a builder output only (L.tiles_only): the shares that can become MFMA tiles.
void lower_format_tiles(Lowering& L, const trs_format& f, const trs_plan_options& o) {
  // room for every tile (see lower_dformat_tiles)
  int64_t room = f.window == 16 && o.mfma_sptc ? (int64_t)f.tile_win.size() : 0;
  for (size_t p = 0; p < f.t_winrow.size() && o.mfma_tc; ++p)
    if (f.t_winrow[p] >= 0 && f.t_winrow[p] % 16 == 0) room += (f.t_rowoff[p + 1] - f.t_rowoff[p] + 1) / 2;
  L.tiles.reserve((size_t)room);
  lower_tc(L, f.t_rowoff.data(), (int64_t)f.t_winrow.size(), f.t_blockoff.data(), f.t_col.data(), f.t_val.data(),
           nullptr, (int64_t)f.t_val.size(), f.t_winrow.data(), f.t_bin.data(), o.mfma_tc != 0);
  lower_groups(L, f.s_col.data(), f.s_val.data(), f.s_pos.data(), (int64_t)f.s_win.size(), f.s_win.data(),
               f.s_offsets.data(), (int64_t)f.s_offsets.size() - 1, f.window, o.mfma_sptc != 0, o.sptc_min_fill);
}

// The tiles of a device-resident builder output, as lower_format_tiles finds them in the host
// one: the TC arrays (slots 0-4, 6) come to the host for lower_tc; the 2:4 group tiles that pass
// the fill rule are chosen and gathered on the device, and only those come over.
Status lower_dformat_tiles(Lowering& L, const trs_dformat& f, const trs_plan_options& o) {
  auto fetch = [&](int s, auto& v) {
    v.resize((size_t)f.slot[s].numel);
    return v.empty() ||
           hipMemcpy(v.data(), f.slot[s].ptr, v.size() * sizeof(v[0]), hipMemcpyDeviceToHost) == hipSuccess;
  };
  {
    std::vector<int32_t> t_rowoff, t_blockoff, t_col, t_winrow;
    std::vector<float> t_val;
    std::vector<int64_t> t_bin;
    if (!fetch(0, t_rowoff) || !fetch(1, t_blockoff) || !fetch(2, t_col) || !fetch(3, t_val) || !fetch(4, t_winrow) ||
        !fetch(6, t_bin))
      return fail(TRS_EDEVICE, "device format: TC array download failed");
    // room for every tile this lowering can make (pairs of sub-blocks of 16-row parts, and the
    // group tiles), so appending the group tiles does not move the TC tiles (over 1 KB each)
    int64_t room = f.window == 16 && o.mfma_sptc ? f.slot[23].numel : 0;
    for (size_t p = 0; p + 1 < t_rowoff.size() && o.mfma_tc; ++p)
      if (t_winrow[p] >= 0 && t_winrow[p] % 16 == 0) room += (t_rowoff[p + 1] - t_rowoff[p] + 1) / 2;
    L.tiles.reserve((size_t)room);
    lower_tc(L, t_rowoff.data(), (int64_t)t_winrow.size(), t_blockoff.data(), t_col.data(), t_val.data(), nullptr,
             (int64_t)t_val.size(), t_winrow.data(), t_bin.data(), o.mfma_tc != 0);
    if (!L.st.ok()) return L.st;
  }
  const int64_t ntiles = f.slot[23].numel;
  if (!o.mfma_sptc || f.window != 16 || ntiles == 0) return Status{};
  if (ntiles > INT32_MAX) return fail(TRS_ERANGE, "more than 2^31 group tiles");
  const int32_t* tile_win = static_cast<const int32_t*>(f.slot[23].ptr);
  const int32_t* tile_group = static_cast<const int32_t*>(f.slot[24].ptr);
  const int32_t* s_off = static_cast<const int32_t*>(f.slot[22].ptr);
  const int32_t* s_col = static_cast<const int32_t*>(f.slot[17].ptr);
  const float* s_val = static_cast<const float*>(f.slot[19].ptr);
  const int8_t* s_pos = static_cast<const int8_t*>(f.slot[20].ptr);
  void* dpass = nullptr;
  const size_t ids_off = ((size_t)ntiles + 3) & ~size_t(3);   // pass flags, then up to ntiles ids
  if (hipMalloc(&dpass, ids_off + (size_t)ntiles * 4) != hipSuccess) {
    (void)hipGetLastError();
    return fail(kLowerOnHost, "device lowering temporaries: hipMalloc failed");
  }
  uint8_t* d_pass = static_cast<uint8_t*>(dpass);
  int32_t* d_ids = reinterpret_cast<int32_t*>(d_pass + ids_off);
  std::vector<uint8_t> pass((size_t)ntiles);
  if (trs::launch_group_tile_fill(tile_win, tile_group, s_off, s_pos, (int32_t)ntiles, o.sptc_min_fill, d_pass,
                                  nullptr) != hipSuccess ||
      hipMemcpy(pass.data(), d_pass, pass.size(), hipMemcpyDeviceToHost) != hipSuccess) {
    (void)hipFree(dpass);
    return fail(TRS_EDEVICE, "device format: group tile fill failed");
  }
  std::vector<int32_t> ids;
  for (int64_t t = 0; t < ntiles; ++t)
    if (pass[t]) ids.push_back((int32_t)t);
  std::vector<trs::GroupTile> gt(ids.size());
  void* dgt = nullptr;
  bool ok = true;
  if (!ids.empty()) {
    ok = hipMalloc(&dgt, gt.size() * sizeof(trs::GroupTile)) == hipSuccess;
    if (!ok) {
      (void)hipGetLastError();
      (void)hipFree(dpass);
      return fail(kLowerOnHost, "device lowering temporaries: hipMalloc failed");
    }
    ok = hipMemcpy(d_ids, ids.data(), ids.size() * 4, hipMemcpyHostToDevice) == hipSuccess &&
         trs::launch_gather_group_tiles(d_ids, (int32_t)ids.size(), tile_win, tile_group, s_off, s_col, s_val, s_pos,
                                        static_cast<trs::GroupTile*>(dgt), nullptr) == hipSuccess &&
         hipMemcpy(gt.data(), dgt, gt.size() * sizeof(trs::GroupTile), hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(dgt);
  }
  (void)hipFree(dpass);
  if (!ok) return fail(TRS_EDEVICE, "device format: group tile gather failed");
  // lower_groups_range's tile step, per gathered tile: a tile with a column outside [0, n) or a
  // position outside 0..3 stops the lowering at the first such tile, in tile order
  auto make = [&](const trs::GroupTile& g, Lowering::Tile& T, Lowering& E) {
    Lowering::tile_init(T, g.row0);
    for (int gi = 0; gi < g.ngroups; ++gi) {
      for (int p = 0; p < 4; ++p) {
        const int32_t c = g.cols[gi * 4 + p];
        if (c >= 0 && !E.check_col(c)) return false;
        T.cols[gi * 4 + p] = c;
      }
      for (int j = 0; j < 32; ++j) {
        const int p = g.pos[gi][j];
        if (p < 0) continue;
        if (p > 3) {
          E.st = fail(TRS_EINVAL, "s_pos entry outside 0..3");
          return false;
        }
        if (g.cols[gi * 4 + p] < 0) continue;
        if (g.row0 + j / 2 < E.m) E.tile_add(T, j / 2, gi * 4 + p, g.val[gi][j]);
      }
    }
    return true;
  };
  const size_t t0 = L.tiles.size();
  L.tiles.resize(t0 + gt.size());
  std::vector<uint8_t> bad(gt.size(), 0);
  parallel_tiles((int64_t)gt.size(), [&](int64_t b, int64_t e, int) {
    Lowering E;
    E.m = L.m;
    E.n = L.n;
    for (int64_t i = b; i < e; ++i) bad[i] = !make(gt[i], L.tiles[t0 + i], E);
  });
  for (size_t i = 0; i < gt.size(); ++i)
    if (bad[i]) {
      Lowering::Tile T;
      make(gt[i], T, L);   // sets L.st as the serial lowering would
      L.tiles.resize(t0 + i);
      return L.st;
    }
  return Status{};
}

// The device lowering takes the residual from the input CSR, minus the entries of the kept tiles:
// for window 16 only, where a TC part's t_window_row (the window id * 16, block_online.cpp:494) is
// its window's first row.  Formats of other window sizes place TC entries at rows of their own.
bool device_lowering_applies(const trs_format& f, const trs_plan_options& o) {
  return !o.host_lowering && !f.csr_rowptr.empty() && f.window == 16;
}

int report(const Status& s) {
  if (!s.ok()) trs::set_error(s.msg);
  return s.code;
}

// The caller's options, or the defaults for NULL.  A struct_size other than this library's means
// the caller was compiled against another trspmm.h: only that first field is read, and the call
// fails.
Status resolve(const trs_plan_options* o, trs_plan_options& r, const char* where) {
  trs_plan_options_default(&r);
  if (!o) return Status{};
  if (o->struct_size != (int32_t)sizeof(trs_plan_options))
    return fail(TRS_EINVAL, std::string(where) + ": trs_plan_options.struct_size is " + std::to_string(o->struct_size) +
                                ", this library's is " + std::to_string(sizeof(trs_plan_options)) +
                                " (initialise the options with trs_plan_options_default of the same trspmm.h)");
  r = *o;
  return Status{};
}

bool bad_dims(int32_t m, int32_t n) { return m < 0 || n < 0; }

}  // namespace

extern "C" {

void trs_plan_options_default(trs_plan_options* o) {
  if (!o) return;
  o->struct_size = (int32_t)sizeof(trs_plan_options);
  o->mfma_tc = 1;
  o->mfma_sptc = 1;
  o->sptc_min_fill = 0.25f;
  o->task_nnz = 0;
  o->piece_nnz = 0;
  o->feature_lanes = 0;
  o->streaming = -1;
  o->window_row_cap = 0;
  o->xcd_run = 0;
  o->sddmm_unroll = 0;
  o->stage = 0;
  o->occupancy = 0;
  o->xcd_split = 0;
  o->host_lowering = 0;
  o->sptc_sparse = 1;
  o->hot_rows = 0;
  o->split_dispatch = 0;
}

const char* trs_last_error(void) { return g_error.c_str(); }

int32_t trs_abi_version(void) { return TRSPMM_ABI_VERSION; }

int trs_plan_create(const trs_format* f, int32_t m, int32_t n, const trs_plan_options* opt, trs_plan** out) {
  if (!f || !out) return report(fail(TRS_EINVAL, "trs_plan_create: NULL argument"));
  *out = nullptr;
  if (bad_dims(m, n)) return report(fail(TRS_EINVAL, "trs_plan_create: negative m or n"));
  if (!f->canonical)
    return report(fail(TRS_ENOTCANON, "trs_plan_create: input rows were not strictly increasing; the format "
                                      "arrays cannot describe duplicate or unsorted entries"));
  trs_plan_options o;
  if (const Status rs = resolve(opt, o, "trs_plan_create"); !rs.ok()) return report(rs);
  if (device_lowering_applies(*f, o)) {
    // device lowering: the tiles from the format, the residual from its input CSR
    Lowering D;
    D.m = m;
    D.n = n;
    D.tiles_only = true;
    lower_format_tiles(D, *f, o);
    const CsrSource cs = csr_of(*f);
    const Status ds = finalize(D, o, out, &cs);
    if (ds.code != kLowerOnHost) return report(ds);
  }
  Lowering L;
  L.m = m;
  L.n = n;
  const size_t approx = f->t_val.size() + f->c_val.size() + f->cs_val.size() + f->s_val.size() / 2 + f->spill_val.size();
  L.row.reserve(approx); L.col.reserve(approx); L.val.reserve(approx);
  lower_format(L, *f, o);
  return report(finalize(L, o, out));
}

int trs_plan_create_sddmm(const trs_format* f, int32_t m, int32_t n, const trs_plan_options* opt, trs_plan** out) {
  if (!f || !out) return report(fail(TRS_EINVAL, "trs_plan_create_sddmm: NULL argument"));
  *out = nullptr;
  if (bad_dims(m, n)) return report(fail(TRS_EINVAL, "trs_plan_create_sddmm: negative m or n"));
  if (!f->canonical)
    return report(fail(TRS_ENOTCANON, "trs_plan_create_sddmm: input rows were not strictly increasing"));
  trs_plan_options o;
  if (const Status rs = resolve(opt, o, "trs_plan_create_sddmm"); !rs.ok()) return report(rs);
  if (device_lowering_applies(*f, o)) {
    Lowering D;
    D.m = m;
    D.n = n;
    D.tiles_only = true;
    lower_format_tiles(D, *f, o);
    const CsrSource cs = csr_of(*f);
    const Status ds = finalize_sddmm(D, o, false, out, &cs);
    if (ds.code != kLowerOnHost) return report(ds);
  }
  Lowering L;
  L.m = m;
  L.n = n;
  lower_format(L, *f, o);
  return report(finalize_sddmm(L, o, false, out));
}

// Plans from a device-resident format: the tiles as lower_dformat_tiles finds them, the residual
// from the format's device copy of the input CSR (only its row pointers come to the host).  Host
// lowering (option host_lowering, or inputs the device lowering does not take) downloads the
// format and lowers it as trs_plan_create does.
static int plan_from_dformat(const trs_dformat* f, int32_t m, int32_t n, const trs_plan_options* opt, bool sddmm,
                             trs_plan** out, const char* where) {
  if (!f || !out) return report(fail(TRS_EINVAL, std::string(where) + ": NULL argument"));
  *out = nullptr;
  if (bad_dims(m, n)) return report(fail(TRS_EINVAL, std::string(where) + ": negative m or n"));
  trs_plan_options o;
  if (const Status rs = resolve(opt, o, where); !rs.ok()) return report(rs);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != f->device)
    return report(fail(TRS_EINVAL, std::string(where) + ": the format lives on device " + std::to_string(f->device) +
                                       ", not on the current device"));
  if (!o.host_lowering && f->window == 16) {
    std::vector<int32_t> rowptr((size_t)f->rows + 1);
    if (hipMemcpy(rowptr.data(), f->csr_rowptr, rowptr.size() * 4, hipMemcpyDeviceToHost) != hipSuccess)
      return report(fail(TRS_EDEVICE, std::string(where) + ": row pointer download failed"));
    CsrSource cs;
    cs.rows = f->rows;
    cs.rowptr = rowptr.data();
    cs.d_col = f->csr_col;
    cs.d_val = f->csr_val;
    Lowering D;
    D.m = m;
    D.n = n;
    D.tiles_only = true;
    Status ds = lower_dformat_tiles(D, *f, o);
    if (ds.ok()) ds = sddmm ? finalize_sddmm(D, o, false, out, &cs) : finalize(D, o, out, &cs);
    if (ds.code != kLowerOnHost) return report(ds);
  }
  trs_format* hf = nullptr;
  if (const int rc = trs_dformat_download(f, &hf); rc != TRS_OK) return rc;
  trs_plan_options h = o;
  h.host_lowering = 1;
  const int rc = sddmm ? trs_plan_create_sddmm(hf, m, n, &h, out) : trs_plan_create(hf, m, n, &h, out);
  trs_format_free(hf);
  return rc;
}

int trs_plan_create_dformat(const trs_dformat* f, int32_t m, int32_t n, const trs_plan_options* opt, trs_plan** out) {
  return plan_from_dformat(f, m, n, opt, false, out, "trs_plan_create_dformat");
}

int trs_plan_create_sddmm_dformat(const trs_dformat* f, int32_t m, int32_t n, const trs_plan_options* opt,
                                  trs_plan** out) {
  return plan_from_dformat(f, m, n, opt, true, out, "trs_plan_create_sddmm_dformat");
}

int trs_plan_create_parallel(const trs_parallel_arrays* a, const trs_plan_options* opt, trs_plan** out) {
  if (!a || !out) return report(fail(TRS_EINVAL, "trs_plan_create_parallel: NULL argument"));
  *out = nullptr;
  if (bad_dims(a->m, a->n)) return report(fail(TRS_EINVAL, "negative m or n"));
  trs_plan_options o;
  if (const Status rs = resolve(opt, o, "trs_plan_create_parallel"); !rs.ok()) return report(rs);
  // structural checks (mGCN_online.cpp:858-932)
  if (a->n_t_row_offset < 1 || a->n_t_row_offset - 1 > a->n_t_window_row || a->n_t_binary < 2 * (a->n_t_block_offset - 1))
    return report(fail(TRS_EINVAL, "TC arrays have inconsistent sizes"));
  const int64_t nparts = a->n_t_row_offset - 1;
  for (int64_t p = 0; p < nparts; ++p) {
    const int32_t s0 = a->t_row_offset[p], s1 = a->t_row_offset[p + 1];
    if (s0 < 0 || s1 < s0 || s1 >= a->n_t_block_offset || (int64_t)s1 * 8 > a->n_t_column)
      return report(fail(TRS_EINVAL, "t_row_offset out of range"));
  }
  if (a->n_c_row_offsets < a->n_c_row + 1 || a->n_cs_row_offsets < a->n_cs_row + 1)
    return report(fail(TRS_EINVAL, "residual offsets shorter than part lists"));
  // lower_residual reads a value for every column entry a part covers
  if (a->n_c_value < a->n_c_column || a->n_cs_value < a->n_cs_column)
    return report(fail(TRS_EINVAL, "residual value arrays shorter than their column arrays"));
  Lowering L;
  L.m = a->m;
  L.n = a->n;
  lower_tc(L, a->t_row_offset, nparts, a->t_block_offset, a->t_column, nullptr, a->t_value, a->n_t_value,
           a->t_window_row, a->t_binary, o.mfma_tc != 0);
  lower_residual(L, a->c_row_offsets, a->c_row, a->n_c_row, a->c_column, nullptr, a->c_value, a->n_c_column);
  lower_residual(L, a->cs_row_offsets, a->cs_row, a->n_cs_row, a->cs_column, nullptr, a->cs_value, a->n_cs_column);
  if (a->use_packed_tiles) {
    lower_packed(L, a->s_tile_column, a->s_packed_a, a->s_packed_meta, a->tiles, a->s_window_tile_offset,
                 a->n_s_window_tile_offset - 1, a->window, o.mfma_sptc != 0, o.sptc_min_fill);
  } else {
    lower_groups(L, a->s_column, a->s_value, a->s_pos, a->groups, nullptr, a->s_offsets, a->n_s_offsets - 1,
                 a->window, o.mfma_sptc != 0, o.sptc_min_fill);
  }
  for (int64_t i = 0; i < a->spill_count && L.st.ok(); ++i) L.add(a->spill_row[i], a->spill_col[i], a->spill_val[i]);
  return report(finalize(L, o, out));
}

int trs_plan_create_sptc(const int32_t* s_column, const float* s_value, const int8_t* s_pos, int64_t groups,
                         const int32_t* s_window, const int32_t* s_offsets, int64_t n_s_offsets, int32_t window,
                         int32_t m, int32_t n, const trs_plan_options* opt, trs_plan** out) {
  if (!out) return report(fail(TRS_EINVAL, "trs_plan_create_sptc: NULL out"));
  *out = nullptr;
  if (bad_dims(m, n) || window <= 0 || groups < 0 || (groups > 0 && (!s_column || !s_value || !s_pos)))
    return report(fail(TRS_EINVAL, "trs_plan_create_sptc: bad arguments"));
  if (!s_window && (!s_offsets || n_s_offsets < 1 || s_offsets[0] != 0 || s_offsets[n_s_offsets - 1] != groups))
    return report(fail(TRS_EINVAL, "s_offsets must start with 0 and end with the group count"));
  if (s_offsets && !s_window)
    for (int64_t w = 0; w + 1 < n_s_offsets; ++w)
      if (s_offsets[w + 1] < s_offsets[w]) return report(fail(TRS_EINVAL, "s_offsets must be non-decreasing"));
  trs_plan_options o;
  if (const Status rs = resolve(opt, o, "trs_plan_create_sptc"); !rs.ok()) return report(rs);
  Lowering L;
  L.m = m;
  L.n = n;
  lower_groups(L, s_column, s_value, s_pos, groups, s_window, s_window ? nullptr : s_offsets,
               s_window ? 0 : n_s_offsets - 1, window, o.mfma_sptc != 0 && !s_window, o.sptc_min_fill);
  return report(finalize(L, o, out));
}

int trs_plan_create_sptc_packed(const int32_t* s_tile_column, const int32_t* s_packed_a, const int32_t* s_packed_meta,
                                const int32_t* s_window_tile_offset, int64_t tiles, int64_t n_wto, int32_t window,
                                int32_t m, int32_t n, const trs_plan_options* opt, trs_plan** out) {
  if (!out) return report(fail(TRS_EINVAL, "trs_plan_create_sptc_packed: NULL out"));
  *out = nullptr;
  if (bad_dims(m, n) || window <= 0 || window > 16 || n_wto < 2 || !s_window_tile_offset)
    return report(fail(TRS_EINVAL, "trs_plan_create_sptc_packed: bad arguments"));
  trs_plan_options o;
  if (const Status rs = resolve(opt, o, "trs_plan_create_sptc_packed"); !rs.ok()) return report(rs);
  Lowering L;
  L.m = m;
  L.n = n;
  lower_packed(L, s_tile_column, s_packed_a, s_packed_meta, tiles, s_window_tile_offset, n_wto - 1, window,
               o.mfma_sptc != 0, o.sptc_min_fill);
  return report(finalize(L, o, out));
}

int trs_plan_create_csr(const int32_t* rowptr, const int32_t* col, const uint16_t* val, int32_t m, int32_t n,
                        const trs_plan_options* opt, trs_plan** out) {
  if (!out) return report(fail(TRS_EINVAL, "trs_plan_create_csr: NULL out"));
  *out = nullptr;
  if (bad_dims(m, n) || !rowptr) return report(fail(TRS_EINVAL, "trs_plan_create_csr: bad arguments"));
  if (rowptr[0] != 0) return report(fail(TRS_EINVAL, "rowptr must start at 0"));
  for (int32_t r = 0; r < m; ++r)
    if (rowptr[r + 1] < rowptr[r]) return report(fail(TRS_EINVAL, "rowptr must be non-decreasing"));
  const int64_t nnz = rowptr[m];
  if (nnz > 0 && (!col || !val)) return report(fail(TRS_EINVAL, "trs_plan_create_csr: NULL col/val"));
  trs_plan_options o;
  if (const Status rs = resolve(opt, o, "trs_plan_create_csr"); !rs.ok()) return report(rs);
  Lowering L;
  L.m = m;
  L.n = n;
  L.row.resize(nnz); L.col.resize(nnz); L.val.resize(nnz);
  for (int32_t r = 0; r < m; ++r)
    for (int32_t e = rowptr[r]; e < rowptr[r + 1]; ++e) {
      if (col[e] < 0 || col[e] >= n) return report(fail(TRS_ERANGE, "column index outside [0, n)"));
      L.row[e] = r; L.col[e] = col[e]; L.val[e] = f16_to_f32(val[e]);
    }
  return report(finalize_sddmm(L, o, true, out));
}

int trs_plan_stats_get(const trs_plan* p, trs_plan_stats* s, int64_t stats_bytes) {
  if (stats_bytes != (int64_t)sizeof(trs_plan_stats))
    return report(fail(TRS_EINVAL, "trs_plan_stats_get: stats_bytes is " + std::to_string(stats_bytes) +
                                       ", this library's trs_plan_stats has " + std::to_string(sizeof(trs_plan_stats)) +
                                       " bytes"));
  if (!p || !s) return report(fail(TRS_EINVAL, "trs_plan_stats_get: NULL argument"));
  *s = p->stats;
  return TRS_OK;
}

void trs_plan_free(trs_plan* p) { delete p; }

// SpMM workspace: the partial slots, then (256-byte aligned) the staged hot rows.
static int64_t partial_region_bytes(const trs_plan* p, int32_t K) {
  return (int64_t)p->dp.partial_slots * K * (int64_t)sizeof(float);
}

int64_t trs_spmm_workspace_bytes(const trs_plan* p, int32_t K) {
  if (!p || K <= 0 || p->csr_only) return 0;
  const int64_t hot = trs::hot_buffer_bytes(p->dp, K);
  const int64_t partial = partial_region_bytes(p, K);
  return hot > 0 ? ((partial + 255) & ~int64_t(255)) + hot : partial;
}

// SDDMM workspace: the split part's output buffer, then (256-byte aligned) the staged hot rows.
static int64_t merge_region_bytes(const trs_plan* p, int32_t K) {
  const int64_t b = trs::merge_buffer_bytes(p->dp, K);
  return trs::hot_buffer_bytes(p->dp, K) > 0 ? (b + 255) & ~int64_t(255) : b;
}

int64_t trs_sddmm_workspace_bytes(const trs_plan* p, int32_t K) {
  if (!p || K <= 0 || !p->csr_only) return 0;
  return merge_region_bytes(p, K) + trs::hot_buffer_bytes(p->dp, K);
}

static int check_call(const trs_plan* p, int32_t K) {
  if (!p) return report(fail(TRS_EINVAL, "NULL plan"));
  if (K < 0) return report(fail(TRS_EINVAL, "K must be non-negative"));
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev != p->device)
    return report(fail(TRS_EDEVICE, "the current HIP device is not the device the plan was created on"));
  return TRS_OK;
}

static int spmm_impl(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C, int64_t ldc, void* ws,
                     int64_t ws_bytes, void* stream, hipEvent_t* ev) {
  int rc = check_call(p, K);
  if (rc) return rc;
  if (p->csr_only) return report(fail(TRS_EINVAL, "trs_spmm_f16: plan was created for SDDMM"));
  if (K == 0 || p->dp.m == 0) return TRS_OK;
  if (!C || (p->dp.n > 0 && !B) || ldb < K || ldc < K)
    return report(fail(TRS_EINVAL, "trs_spmm_f16: NULL operand or leading dimension < K"));
  if (ldb > INT32_MAX) return report(fail(TRS_ERANGE, "trs_spmm_f16: leading dimension of B beyond 2^31 - 1"));
  const int64_t need = trs_spmm_workspace_bytes(p, K);
  if (ws_bytes < need || (need > 0 && !ws))
    return report(fail(TRS_EINVAL, "trs_spmm_f16: workspace smaller than trs_spmm_workspace_bytes"));
  const int64_t partial = partial_region_bytes(p, K);
  uint16_t* hot = trs::hot_buffer_bytes(p->dp, K) > 0
                      ? reinterpret_cast<uint16_t*>(static_cast<unsigned char*>(ws) + ((partial + 255) & ~int64_t(255)))
                      : nullptr;
  const hipError_t e = trs::launch_spmm(p->dp, B, ldb, K, C, ldc, static_cast<float*>(ws), hot,
                                        static_cast<hipStream_t>(stream), ev);
  if (e != hipSuccess) return report(fail(TRS_EDEVICE, std::string("kernel launch failed: ") + hipGetErrorString(e)));
  return TRS_OK;
}

int trs_spmm_f16(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C, int64_t ldc, void* ws,
                 int64_t ws_bytes, void* stream) {
  return spmm_impl(p, B, ldb, K, C, ldc, ws, ws_bytes, stream, nullptr);
}

int trs_spmm_f16_kernel_ms(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C, int64_t ldc,
                           void* ws, int64_t ws_bytes, void* stream, int32_t iters, float* ms) {
  if (!ms || iters <= 0) return report(fail(TRS_EINVAL, "trs_spmm_f16_kernel_ms: needs ms[3] and iters > 0"));
  ms[0] = ms[1] = ms[2] = 0.f;
  hipEvent_t ev[4];
  for (auto& e : ev)
    if (hipEventCreate(&e) != hipSuccess) return report(fail(TRS_EDEVICE, "hipEventCreate failed"));
  int rc = TRS_OK;
  for (int i = 0; i < iters && rc == TRS_OK; ++i) {
    rc = spmm_impl(p, B, ldb, K, C, ldc, ws, ws_bytes, stream, ev);
    if (rc) break;
    (void)hipEventSynchronize(ev[3]);
    for (int k = 0; k < 3; ++k) {
      float t = 0.f;
      (void)hipEventElapsedTime(&t, ev[k], ev[k + 1]);
      ms[k] += t / (float)iters;
    }
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  return rc;
}

int trs_spmm_f16_timed(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C, int64_t ldc, void* ws,
                       int64_t ws_bytes, void* stream, int32_t warmup, int32_t iters, float* ms_avg) {
  if (ms_avg) *ms_avg = 0.f;
  if (iters <= 0) return report(fail(TRS_EINVAL, "iters must be positive"));
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int i = 0; i < warmup; ++i) {
    int rc = trs_spmm_f16(p, B, ldb, K, C, ldc, ws, ws_bytes, stream);
    if (rc) return rc;
  }
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess)
    return report(fail(TRS_EDEVICE, "hipEventCreate failed"));
  (void)hipEventRecord(e0, s);
  int rc = TRS_OK;
  for (int i = 0; i < iters && rc == TRS_OK; ++i) rc = trs_spmm_f16(p, B, ldb, K, C, ldc, ws, ws_bytes, stream);
  (void)hipEventRecord(e1, s);
  (void)hipEventSynchronize(e1);
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc) return rc;
  if (ms_avg) *ms_avg = ms / (float)iters;
  return TRS_OK;
}

// ws: the staged hot Y rows (null: run without staging)
static int sddmm_impl(const trs_plan* p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy, int32_t K,
                      float* out, void* ws, int64_t ws_bytes, void* stream, hipEvent_t* ev) {
  int rc = check_call(p, K);
  if (rc) return rc;
  if (!p->csr_only)
    return report(fail(TRS_EINVAL, "trs_sddmm_f16: needs a plan from trs_plan_create_sddmm or trs_plan_create_csr"));
  if (p->stats.nnz == 0) return TRS_OK;
  if (!out) return report(fail(TRS_EINVAL, "trs_sddmm_f16: NULL output"));
  if (K == 0) {   // empty dot products; X and Y may be empty (NULL) then
    if (trs::launch_zero_fill(out, p->stats.nnz, static_cast<hipStream_t>(stream)) != hipSuccess)
      return report(fail(TRS_EDEVICE, "zero-fill launch failed"));
    return TRS_OK;
  }
  if (!X || !Y || ldx < K || ldy < K)
    return report(fail(TRS_EINVAL, "trs_sddmm_f16: NULL operand or leading dimension < K"));
  if (ldy > INT32_MAX) return report(fail(TRS_ERANGE, "trs_sddmm_f16: leading dimension of Y beyond 2^31 - 1"));
  const int64_t need = trs_sddmm_workspace_bytes(p, K);
  if (ws && ws_bytes < need)
    return report(fail(TRS_EINVAL, "trs_sddmm_f16_ws: workspace smaller than trs_sddmm_workspace_bytes"));
  float* xbuf = ws && trs::merge_buffer_bytes(p->dp, K) > 0 ? static_cast<float*>(ws) : nullptr;
  uint16_t* hot = ws && trs::hot_buffer_bytes(p->dp, K) > 0
                      ? reinterpret_cast<uint16_t*>(static_cast<unsigned char*>(ws) + merge_region_bytes(p, K))
                      : nullptr;
  const hipError_t e =
      trs::launch_sddmm(p->dp, X, ldx, Y, ldy, K, out, hot, xbuf, static_cast<hipStream_t>(stream), ev);
  if (e != hipSuccess) return report(fail(TRS_EDEVICE, std::string("kernel launch failed: ") + hipGetErrorString(e)));
  return TRS_OK;
}

int trs_sddmm_f16(const trs_plan* p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy, int32_t K,
                  float* out, void* stream) {
  return sddmm_impl(p, X, ldx, Y, ldy, K, out, nullptr, 0, stream, nullptr);
}

int trs_sddmm_f16_ws(const trs_plan* p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy, int32_t K,
                     float* out, void* ws, int64_t ws_bytes, void* stream) {
  return sddmm_impl(p, X, ldx, Y, ldy, K, out, ws, ws_bytes, stream, nullptr);
}

int trs_sddmm_f16_kernel_ms(const trs_plan* p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy,
                            int32_t K, float* out, void* ws, int64_t ws_bytes, void* stream, int32_t iters,
                            float* ms) {
  if (!ms || iters <= 0) return report(fail(TRS_EINVAL, "trs_sddmm_f16_kernel_ms: needs ms[2] and iters > 0"));
  ms[0] = ms[1] = 0.f;
  hipEvent_t ev[3];
  for (auto& e : ev)
    if (hipEventCreate(&e) != hipSuccess) return report(fail(TRS_EDEVICE, "hipEventCreate failed"));
  int rc = TRS_OK;
  for (int i = 0; i < iters && rc == TRS_OK; ++i) {
    rc = sddmm_impl(p, X, ldx, Y, ldy, K, out, ws, ws_bytes, stream, ev);
    if (rc) break;
    (void)hipEventSynchronize(ev[2]);
    for (int k = 0; k < 2; ++k) {
      float t = 0.f;
      (void)hipEventElapsedTime(&t, ev[k], ev[k + 1]);
      ms[k] += t / (float)iters;
    }
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  return rc;
}

}  // extern "C"
