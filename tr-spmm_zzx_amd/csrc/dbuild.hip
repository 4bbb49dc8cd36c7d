// Format builder on the GPU: the reference's 29-array "online" tuple plus the spill list, bit for
// bit what trs_build_online (csrc/builder.cpp) and the reference builder produce
// (TR-source/Block/block_online.cpp:545-871), built from a CSR in device memory into device memory.
//
// Scope: canonical input (strictly increasing columns in every row) and windows of at most 16 rows.
// There every (row, column) is counted once, so a column's row vector holds 0/1 per 2-bit field,
// the 2:4 compatibility test of block_online.cpp:83-88 always passes, and the window's whole
// routing has a closed form (the one builder.cpp's match_all_compatible uses):
//   * TC columns: count >= density, ordered (count desc, column asc), chunks of 8, each chunk's
//     columns ascending (block_online.cpp:215-253);
//   * units: the other columns in the same order, consecutive pairs (:267-328); their nnz does not
//     increase with the unit index;
//   * order: std::sort of 0..n-1 by unit nnz descending (:358-363), whose ties fall where
//     libstdc++'s introsort puts them -- restated in csrc/introsort.hpp and run here with a wave per
//     partition step (isort::partition_batched is the step a wave takes, lane j holding pair j);
//   * matching: each unmatched unit in that order takes the lowest-index unmatched other unit (all
//     degrees are n - 1, and a lower index never has a smaller nnz) (:365-386);
//   * groups, 2:4 metadata, residual parts, TC parts and tiles follow from the pairs
//     (:629-733, :444-540, :736-776, :796-841).
// Other inputs go to the host builder.
//
// Stages (one pass each over device arrays, prefix sums between them):
//   A  every entry's position in its window sorted by (column, local row): ranks from binary
//      searches in the window's other rows, no sort; distinct columns with 16-bit row masks;
//   B  per window (a wave for windows of <= kSmallU distinct columns, a workgroup of 16 waves
//      otherwise): TC chunks, units, the introsort, the greedy matching, groups;
//   C  counts per window and per row, prefix sums;
//   D  the format arrays.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "dformat.hpp"
#include "format.hpp"
#include "half.hpp"
#include "introsort.hpp"
#include "trspmm.h"

namespace {

using u64 = unsigned long long;

constexpr int kSmallU = 8192;       // windows with more distinct columns take the workgroup kernel
constexpr int kBlockWaves = 8;      // waves of that kernel
constexpr int kLdsUnits = 65536;    // most units whose order it keeps in LDS (16-bit indices; the
                                    // device's LDS per workgroup may allow fewer)
constexpr int kMaxKey = 32;         // unit nnz <= 2 * window
constexpr int kGreedySpan = 1024;   // indices ahead of the matching's low end one round looks at

// ---- wave helpers --------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }
__device__ __forceinline__ int mbcnt(u64 m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
__device__ __forceinline__ u64 ballot(bool p) { return __ballot(p); }
__device__ __forceinline__ int rdlane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
// LDS written by some lanes of a wave and read by others: keep the compiler from reordering.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}
__device__ __forceinline__ int popc32(uint32_t x) { return __popc(x); }

// Errors a kernel reports (bit flags, or-ed into *err): the host refuses the build.
enum : uint32_t {
  kErrNonCanonical = 1u,   // a row's columns are not strictly increasing
  kErrNegativeColumn = 2u,
  kErrInternal = 4u,       // a partition step found no stop (cannot happen for a valid order)
};

// ---- prefix sums ---------------------------------------------------------------------------
constexpr int kScanItems = 16;
constexpr int kScanBlock = 256 * kScanItems;

__device__ int block_exclusive_sum_256(int v, int* sh /* >= 5 ints */, int& total) {
  const int l = lane_id(), w = threadIdx.x >> 6;
  int x = v;
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d);
    if (l >= d) x += y;
  }
  if (l == 63) sh[w] = x;
  __syncthreads();
  int base = 0;
  for (int i = 0; i < w; ++i) base += sh[i];
  total = sh[0] + sh[1] + sh[2] + sh[3];
  __syncthreads();
  return base + x - v;
}

template <class T>
__global__ __launch_bounds__(256) void k_scan_reduce(const T* __restrict__ in, int64_t n, int32_t* __restrict__ bsum) {
  __shared__ int sh[8];
  const int64_t b0 = (int64_t)blockIdx.x * kScanBlock + (int64_t)threadIdx.x * kScanItems;
  int s = 0;
  for (int i = 0; i < kScanItems; ++i)
    if (b0 + i < n) s += (int)in[b0 + i];
  int total;
  (void)block_exclusive_sum_256(s, sh, total);
  if (threadIdx.x == 0) bsum[blockIdx.x] = total;
}

__global__ __launch_bounds__(256) void k_scan_bsums(int32_t* __restrict__ bsum, int32_t nb) {
  __shared__ int sh[8];
  int carry = 0;
  for (int32_t b0 = 0; b0 < nb; b0 += 256) {
    const int32_t i = b0 + (int32_t)threadIdx.x;
    const int v = i < nb ? bsum[i] : 0;
    int total;
    const int ex = block_exclusive_sum_256(v, sh, total);
    if (i < nb) bsum[i] = carry + ex;
    carry += total;
  }
  if (threadIdx.x == 0) bsum[nb] = carry;
}

template <class T>
__global__ __launch_bounds__(256) void k_scan_apply(const T* __restrict__ in, int64_t n, const int32_t* __restrict__ bsum,
                                                    int32_t nb, int32_t* __restrict__ out) {
  __shared__ int sh[8];
  const int64_t b0 = (int64_t)blockIdx.x * kScanBlock + (int64_t)threadIdx.x * kScanItems;
  int v[kScanItems];
  int s = 0;
  for (int i = 0; i < kScanItems; ++i) {
    v[i] = b0 + i < n ? (int)in[b0 + i] : 0;
    s += v[i];
  }
  int total;
  int run = bsum[blockIdx.x] + block_exclusive_sum_256(s, sh, total);
  for (int i = 0; i < kScanItems; ++i)
    if (b0 + i < n) {
      out[b0 + i] = run;
      run += v[i];
    }
  if (blockIdx.x == 0 && threadIdx.x == 0) out[n] = bsum[nb];
}

// out[0..n) = exclusive prefix sums of in[0..n), out[n] = total (int32; the caller keeps totals
// within int32).  bsum: ceil(n / kScanBlock) + 1 ints of scratch.
template <class T>
hipError_t scan(const T* in, int64_t n, int32_t* out, int32_t* bsum, hipStream_t s) {
  const int32_t nb = (int32_t)((n + kScanBlock - 1) / kScanBlock);
  if (nb == 0) {
    hipLaunchKernelGGL(k_scan_bsums, dim3(1), dim3(256), 0, s, bsum, 0);
    return hipMemcpyAsync(out, bsum, sizeof(int32_t), hipMemcpyDeviceToDevice, s);
  }
  hipLaunchKernelGGL((k_scan_reduce<T>), dim3(nb), dim3(256), 0, s, in, n, bsum);
  hipLaunchKernelGGL(k_scan_bsums, dim3(1), dim3(256), 0, s, bsum, nb);
  hipLaunchKernelGGL((k_scan_apply<T>), dim3(nb), dim3(256), 0, s, in, n, bsum, nb, out);
  return hipGetLastError();
}
int64_t scan_scratch_ints(int64_t n) { return (n + kScanBlock - 1) / kScanBlock + 1; }

// ---- build description ---------------------------------------------------------------------
struct WinOut {
  int32_t nsub, ngroups, tvals, nres;
  int32_t res[2];   // residual columns (window-local distinct ids, ascending), nres <= 2
  int32_t pad[2];
};

struct Build {
  // input
  int32_t rows = 0, ws = 16, nwin = 0;
  int32_t lds_units = 0;      // windows of at most this many units keep their order in LDS
  int64_t nnz = 0;
  const int32_t* rowptr = nullptr;
  const int32_t* col = nullptr;
  const float* val = nullptr;
  // parameters (block_online.cpp:545-567)
  int32_t part_t = 32, part_c = 32, short_size = 3, density = 8, skip_tc = 0, unit_min = 2;
  float tc_min_util = 0.f;
  uint32_t* err = nullptr;
  // stage A: per sorted position p (window by window, (column, local row) ascending)
  int32_t* s_col = nullptr;
  int32_t* s_e = nullptr;
  uint8_t* s_lr = nullptr;
  uint8_t* s_new = nullptr;   // 1 where a new distinct column starts
  int32_t* s_u = nullptr;     // [nnz + 1] distinct column of each position (exclusive scan of s_new)
  // distinct columns u (window by window, ascending column): U of them
  int32_t U = 0;
  int32_t* ubase = nullptr;   // [nwin + 1]
  int32_t* ucol = nullptr;
  uint32_t* umask = nullptr;  // bit lr: row lr of the window holds the column
  int32_t* ufirst = nullptr;  // [U + 1] first sorted position
  // stage B (window-local arrays at the window's offset ubase[w], or ubase[w] + k * w)
  int32_t* ustat = nullptr;   // >= 0: TC slot (sub-block * 8 + k); -2: in a 2:4 group; -1: residual
  int32_t* ord = nullptr;     // the columns in (count desc, column asc) order (TC candidates, then units)
  int32_t* tcl = nullptr;     // at ubase + 8 w: sub-block s, slot k -> distinct id (-1 pad)
  int32_t* gl = nullptr;      // at ubase + 4 w: group g, member q -> distinct id (-1 pad), ascending
  uint8_t* unnz = nullptr;    // unit nnz
  int32_t* gperm = nullptr;   // unit order of windows beyond kLdsUnits units
  int32_t* gpos = nullptr;    // its inverse (large windows)
  uint8_t* leaf = nullptr;    // leaf length at a leaf's first position (large windows)
  int32_t* pairs = nullptr;   // matched pairs (x, y) (large windows)
  int32_t* ranges = nullptr;  // introsort range lists (large windows)
  WinOut* win = nullptr;
  // stage C
  int32_t* wparts = nullptr;  // per window counts, scanned in place into bases (nwin + 1 each)
  int32_t* wsubs = nullptr;
  int32_t* wtvals = nullptr;
  int32_t* wgroups = nullptr;
  int32_t* wtiles = nullptr;
  int32_t* rlp = nullptr;     // per row: long parts, long entries, short parts, short entries
  int32_t* rle = nullptr;
  int32_t* rsp = nullptr;
  int32_t* rse = nullptr;
  uint8_t* spill = nullptr;   // per entry: 1 if no array carries it
  int32_t* spill_at = nullptr;
};

// Format arrays being filled (device).
struct Out {
  int32_t *t_rowoff, *t_blockoff, *t_col, *t_winrow, *t_atomic;
  float* t_val;
  int64_t* t_bin;
  int32_t *c_off, *c_row, *c_atomic, *c_col;
  float* c_val;
  int32_t *cs_off, *cs_row, *cs_atomic, *cs_col;
  float* cs_val;
  int32_t *s_col, *s_win, *s_offsets;
  uint8_t* s_mask;
  float* s_val;
  int8_t* s_pos;
  int32_t *tile_win, *tile_group, *tile_cols, *packed_a, *packed_meta, *win_tile_off;
  int32_t *spill_row, *spill_col;
  float* spill_val;
};

__device__ __forceinline__ int32_t row_of(const int32_t* rowptr, int32_t rows, int64_t e) {
  int32_t lo = 0, hi = rows;   // rowptr[lo] <= e < rowptr[hi]
  while (hi - lo > 1) {
    const int32_t mid = (int32_t)(((uint32_t)lo + (uint32_t)hi) >> 1);
    if ((int64_t)rowptr[mid] <= e) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Entries of a[0, n) below c (inclusive: at most c); a ascending.
__device__ __forceinline__ int32_t count_below(const int32_t* a, int32_t n, int32_t c, bool inclusive) {
  int32_t lo = 0, hi = n;
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    const bool below = inclusive ? a[mid] <= c : a[mid] < c;
    if (below) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// The entry of distinct column u in local row lr (the column's positions are in row order).
__device__ __forceinline__ int32_t entry_of(const Build& B, int32_t u, int lr) {
  const uint32_t m = B.umask[u];
  return B.s_e[B.ufirst[u] + popc32(m & ((1u << lr) - 1u))];
}

// ---- stage A -------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_check_rows(const int32_t* __restrict__ rowptr, int32_t rows,
                                                    uint32_t* __restrict__ bad) {
  const int32_t r = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (r < rows && rowptr[r + 1] < rowptr[r]) atomicOr(bad, 1u);
}

// Position of entry e in its window ordered by (column, local row): its index in its row plus, for
// each other row of the window, the entries below its column (at most its column for earlier rows).
__global__ __launch_bounds__(256) void k_rank(Build B) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= B.nnz) return;
  const int32_t r = row_of(B.rowptr, B.rows, e);
  const int32_t w = r / B.ws, lr = r - w * B.ws;
  const int32_t r0 = w * B.ws, r1 = min(r0 + B.ws, B.rows);
  const int32_t c = B.col[e];
  const int32_t rb = B.rowptr[r];
  if (c < 0) atomicOr(B.err, kErrNegativeColumn);
  if (e > rb && B.col[e - 1] >= c) atomicOr(B.err, kErrNonCanonical);
  int32_t rank = (int32_t)(e - rb);
  for (int32_t q = r0; q < r1; ++q) {
    if (q == r) continue;
    const int32_t b = B.rowptr[q], n = B.rowptr[q + 1] - b;
    if (n > 0) rank += count_below(B.col + b, n, c, q < r);
  }
  const int64_t p = (int64_t)B.rowptr[r0] + rank;
  B.s_col[p] = c;
  B.s_e[p] = (int32_t)e;
  B.s_lr[p] = (uint8_t)lr;
  B.s_new[p] = rank == 0 ? 1 : 0;
}

__global__ __launch_bounds__(256) void k_new_columns(Build B) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= B.nnz || p == 0) return;
  if (!B.s_new[p] && B.s_col[p] != B.s_col[p - 1]) B.s_new[p] = 1;
}

__global__ __launch_bounds__(256) void k_window_bases(Build B) {
  const int32_t w = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (w > B.nwin) return;
  const int32_t r = min(w * B.ws, B.rows);
  B.ubase[w] = B.s_u[B.rowptr[r]];
}

__global__ __launch_bounds__(256) void k_distinct(Build B) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (p >= B.nnz || !B.s_new[p]) return;
  const int32_t u = B.s_u[p];
  B.ucol[u] = B.s_col[p];
  B.ufirst[u] = (int32_t)p;
  uint32_t m = 0;
  int64_t j = p;
  do {
    m |= 1u << B.s_lr[j];
    ++j;
  } while (j < B.nnz && !B.s_new[j]);
  B.umask[u] = m;
  if (p == 0) B.ufirst[B.U] = (int32_t)B.nnz;
}

// ---- stage B: per-window ordering ----------------------------------------------------------
// Shared memory of one window's wave(s).
struct WinShared {
  int start_of[kMaxKey + 1];   // first unit index of each nnz value (-1: none)
  int end_of[kMaxKey + 1];     // one past its last
  int hist[kBlockWaves][17];   // per wave count histograms
  int cnt[2];                  // range list sizes (workgroup kernel)
  int misc[8];
};

// Counting sort of the window's columns u in [0, U) that `sel` picks, by (count desc, u asc),
// into out[0, selected) (window-local ids); NW waves, wave w taking a contiguous run of chunks.
// Returns the number selected (all threads).
template <int NW, class Sel>
__device__ int count_sort(const uint32_t* umask, int U, Sel sel, int32_t* out, WinShared& sh) {
  const int l = lane_id(), w = (int)(threadIdx.x >> 6);
  const int chunks = (U + 63) >> 6;
  const int c0 = (int)((int64_t)chunks * w / NW), c1 = (int)((int64_t)chunks * (w + 1) / NW);
  // the count of this lane's column in chunk ch (0: not selected); four chunks' loads in flight
  auto count_of = [&](int ch) {
    const int u = ch * 64 + l;
    return ch < c1 && u < U && sel(u) ? popc32(umask[u]) : 0;
  };
  int myhist = 0;   // lane v: this wave's columns of count v
  for (int ch0 = c0; ch0 < c1; ch0 += 4) {
    int cs[4];
    for (int i = 0; i < 4; ++i) cs[i] = count_of(ch0 + i);
    for (int i = 0; i < 4; ++i) {
      const int c = cs[i];
      u64 rem = ballot(c != 0);
      while (rem) {
        const int v = rdlane(c, __builtin_ctzll(rem));
        const u64 b = ballot(c == v);
        if (l == v) myhist += __popcll(b);
        rem &= ~b;
      }
    }
  }
  if (l <= 16) sh.hist[w][l] = myhist;
  __syncthreads();
  // start of value v for this wave: all columns of larger counts, then this value's columns of
  // earlier waves
  int run = 0, total = 0;
  if (l >= 1 && l <= 16) {
    for (int v = 16; v > l; --v)
      for (int q = 0; q < NW; ++q) run += sh.hist[q][v];
    for (int q = 0; q < w; ++q) run += sh.hist[q][l];
  }
  for (int v = 1; v <= 16; ++v)
    for (int q = 0; q < NW; ++q) total += sh.hist[q][v];
  for (int ch0 = c0; ch0 < c1; ch0 += 4) {
    int cs[4];
    for (int i = 0; i < 4; ++i) cs[i] = count_of(ch0 + i);
    for (int i = 0; i < 4; ++i) {
      const int c = cs[i];
      const int u = (ch0 + i) * 64 + l;
      u64 rem = ballot(c != 0);
      while (rem) {
        const int v = rdlane(c, __builtin_ctzll(rem));
        const u64 b = ballot(c == v);
        const int base = rdlane(run, v);
        if (c == v) out[base + mbcnt(b)] = u;
        if (l == v) run += __popcll(b);
        rem &= ~b;
      }
    }
  }
  __syncthreads();
  return total;
}

// The batched partition step (isort::partition_batched with 64 lanes) of perm[s, e) by unit nnz,
// descending.  Keys do not increase with the unit index, so "key(x) <= pivot key" is x >=
// start_of[key] and "key(x) >= pivot key" is x < end_of[key].  Returns the cut.
template <class P>
__device__ int wave_partition(P* perm, int s, int e, const uint8_t* unnz, const WinShared& sh, int* Lbuf, int* Rbuf,
                              uint32_t* err, int* pivot_key) {
  const int l = lane_id();
  const int mid = s + (e - s) / 2;
  const int ia = s + 1, ib = mid, ic = e - 1;
  const int ka = unnz[perm[ia]], kb = unnz[perm[ib]], kc = unnz[perm[ic]];
  int t;   // std::__move_median_to_first(s, s + 1, mid, e - 1) with comp = key greater
  if (ka > kb) t = kb > kc ? ib : ka > kc ? ic : ia;
  else t = ka > kc ? ia : kb > kc ? ic : ib;
  const int vs = perm[s], vt = perm[t];
  wave_sync();
  if (l == 0) {
    perm[s] = (P)vt;
    perm[t] = (P)vs;
  }
  wave_sync();
  const int pk = unnz[vt];
  *pivot_key = pk;
  const int lo = sh.start_of[pk], hi = sh.end_of[pk];
  int aL = s + 1, aR = e - 1, nL = 0, nR = 0, rprev = e;
  for (int guard = 0; guard <= (e - s) / 64 + 2; ++guard) {
    while (nL < 64 && aL < e) {
      const int i = aL + l;
      const bool f = i < e && (int)perm[i] >= lo;
      const u64 m = ballot(f);
      if (f) Lbuf[nL + mbcnt(m)] = i;
      nL += __popcll(m);
      aL += 64;
    }
    while (nR < 64 && aR >= s) {
      const int i = aR - l;
      const bool f = i >= s && (int)perm[i] < hi;
      const u64 m = ballot(f);
      if (f) Rbuf[nR + mbcnt(m)] = i;
      nR += __popcll(m);
      aR -= 64;
    }
    wave_sync();
    const int Lj = l < nL ? Lbuf[l] : e;
    const int Rj = l < nR ? Rbuf[l] : -1;
    const u64 sm = ballot(Rj <= Lj);
    const int kk = sm ? (int)__builtin_ctzll(sm) : 64;
    int vL = 0, vR = 0;
    if (l < kk) {
      vL = perm[Lj];
      vR = perm[Rj];
    }
    wave_sync();
    if (l < kk) {
      perm[Lj] = (P)vR;
      perm[Rj] = (P)vL;
    }
    wave_sync();
    if (kk < 64) {
      const int Lk = rdlane(Lj, kk);
      const int rp = kk == 0 ? rprev : rdlane(Rj, kk - 1);
      const int cut = rp < Lk ? rp : Lk;
      if (cut <= s || cut >= e) {
        atomicOr(err, kErrInternal);
        return s + 1;
      }
      return cut;
    }
    rprev = rdlane(Rj, 63);
    const int Ln = l + 64 < nL ? Lbuf[l + 64] : 0, Rn = l + 64 < nR ? Rbuf[l + 64] : 0;
    wave_sync();
    if (l + 64 < nL) Lbuf[l] = Ln;
    if (l + 64 < nR) Rbuf[l] = Rn;
    wave_sync();
    nL -= 64;
    nR -= 64;
  }
  atomicOr(err, kErrInternal);
  return s + 1;
}

// A range whose depth limit ran out: std::__partial_sort(first, last, last) on one lane.
template <class P>
__device__ void lane0_heap_sort(P* perm, int s, int e, const uint8_t* unnz) {
  if (lane_id() == 0) {
    auto cmp = [unnz](P a, P b) { return unnz[a] > unnz[b]; };
    trs::isort::heap_sort(perm + s, perm + e, cmp);
  }
  wave_sync();
}

// A range whose units all have one nnz, finished by one wave: every unit goes to the offset
// isort::tied_final_offset gives (the loop's steps on equal elements), through tmp.
template <class P>
__device__ void wave_tied(P* perm, int s, int L, int32_t* tmp) {
  const int l = lane_id();
  for (int o = l; o < L; o += 64) tmp[s + (int)trs::isort::tied_final_offset(L, o)] = (int32_t)perm[s + o];
  __threadfence_block();
  wave_sync();
  for (int o = l; o < L; o += 64) perm[s + o] = (P)tmp[s + o];
  __threadfence_block();
  wave_sync();
}

// Depth limit and the range's key bounds in one int: keys are at most kMaxKey (6 bits).
__device__ __forceinline__ int pack_range(int d, int kmin, int kmax) { return d | (kmin << 8) | (kmax << 16); }

// Leaves (ranges the loop left at <= 16 elements) each get the stable sort the final insertion
// sort amounts to there (isort::final_insertion_sort never moves an element across a partition
// cut): a leaf's units and keys are loaded into registers at once and sorted by odd-even
// transposition, which swaps only strictly inverted neighbours (so equal keys keep their order).
// Threads [t0, t0 + nt) of the window share the positions.
template <class P>
__device__ void sort_leaves(P* perm, int n, const uint8_t* leaf, const uint8_t* unnz, int t0, int nt) {
  for (int i = (int)threadIdx.x - t0; i < n; i += nt) {
    const int len = leaf[i];
    if (len < 2) continue;
    int v[16], k[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = j < len ? (int)perm[i + j] : 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) k[j] = j < len ? (int)unnz[v[j]] : -1;   // -1: past the leaf, stays last
#pragma unroll
    for (int round = 0; round < 16; ++round) {
#pragma unroll
      for (int j = round & 1; j + 1 < 16; j += 2) {
        if (k[j + 1] > k[j]) {   // descending keys
          const int tv = v[j], tk = k[j];
          v[j] = v[j + 1];
          k[j] = k[j + 1];
          v[j + 1] = tv;
          k[j + 1] = tk;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < len) perm[i + j] = (P)v[j];
  }
}

// std::sort's loop over perm[0, n) by one wave, ranges on a stack held one per lane.  Each range
// carries bounds on its keys (the left part of a partition holds keys >= the pivot's, the right
// part keys <= it); a range whose bounds meet is finished by the closed form for equal keys.
template <class P>
__device__ void wave_introsort(P* perm, int n, const uint8_t* unnz, uint8_t* leaf, const WinShared& sh, int* Lbuf,
                               int* Rbuf, int32_t* tmp, uint32_t* err) {
  const int l = lane_id();
  int sf = 0, sl = 0, sd = 0, top = 0;
  if (l == 0) {
    sf = 0;
    sl = n;
    sd = pack_range(2 * trs::isort::lg(n), unnz[n - 1], unnz[0]);
  }
  top = 1;
  while (top > 0) {
    --top;
    const int f = rdlane(sf, top);
    int last = rdlane(sl, top);
    const int packed = rdlane(sd, top);
    int d = packed & 0xff, kmin = (packed >> 8) & 0xff, kmax = packed >> 16;
    bool done = false;
    while (last - f > 16) {
      if (kmin == kmax && trs::isort::tied_depth_ok(last - f, d)) {
        wave_tied(perm, f, last - f, tmp);
        done = true;
        break;
      }
      if (d == 0) {
        lane0_heap_sort(perm, f, last, unnz);
        done = true;
        break;
      }
      --d;
      int pk = 0;
      const int cut = wave_partition(perm, f, last, unnz, sh, Lbuf, Rbuf, err, &pk);
      if (top >= 63) {   // the stack never holds more than the depth limit (<= 2 log2 n) ranges
        atomicOr(err, kErrInternal);
        return;
      }
      if (l == top) {
        sf = cut;
        sl = last;
        sd = pack_range(d, kmin, pk);
      }
      ++top;
      last = cut;
      kmin = pk;
    }
    if (!done && l == 0) leaf[f] = (uint8_t)(last - f);
    wave_sync();
  }
}

// Greedy matching over the sorted order (one wave): the next unit of the order not yet taken
// pairs with the lowest-index unit not yet taken.  Two walks: the order's (a position in perm) and
// the low end's (an index b); `taken` (n bits, zeroed by the caller) records the units the order's
// walk took, which the low end skips, and the order skips units below b (the low end took them).
//
// 64 steps at a time: the order's next 64 candidates (positions >= a whose unit is >= b) and the
// low end's next 64 (untaken indices in [b, b + kGreedySpan)) are paired lane by lane, as if neither
// walk took a candidate of the other.  Step j is exact until one of them did: the order's
// candidate x_j is not above the low end's previous pick y_{j-1} (the low end took it first), or
// the low end's y_j is some x_i, i <= j (the order took it first).  Steps before the first such j
// are committed together; a first step that fails is taken on its own, exactly.  Pairs go to
// px[k], py[k]; returns their number, *left = the unit left unmatched (-1: none).  buf: 512 ints
// of LDS for this wave.
template <class P>
__device__ int wave_greedy(const P* perm, uint32_t* taken, int n, int32_t* px, int32_t* py, int* left, int* buf) {
  const int l = lane_id();
  int* Ab = buf;          // order candidates: positions
  int* Bb = buf + 128;    // low-end candidates: indices
  // for index b + d (d < kGreedySpan): the step whose order candidate it is (64: none)
  uint8_t* stepA = reinterpret_cast<uint8_t*>(buf + 256);
  int a = 0, b = 0, np = 0, lf = -1;
  for (int guard = 0; guard <= 2 * n + 2; ++guard) {
    int nA = 0, aEnd = a;
    for (; nA < 64 && aEnd < n; aEnd += 64) {
      const int p = aEnd + l;
      const bool f = p < n && (int)perm[p] >= b;
      const u64 m = ballot(f);
      const int r = nA + mbcnt(m);
      if (f && r < 64) Ab[r] = p;
      nA += __popcll(m);
    }
    if (nA == 0) break;   // no unit left for the order
    // positions the scan passed without a candidate stay passed (b only grows): after the
    // committed steps the walk resumes at the next collected candidate, or where the scan ended
    const bool scan_whole = nA <= 64;
    if (nA > 64) nA = 64;
    // the low end's candidates: the next 64 untaken indices from b, below b + kGreedySpan
    const int lim = min(n, b + kGreedySpan);
    int nB = 0, bEnd = b;
    for (; nB < 64 && bEnd < lim; bEnd += 64) {
      const int q = bEnd + l;
      const bool f = q < lim && !((taken[q >> 5] >> (q & 31)) & 1u);
      const u64 m = ballot(f);
      const int r = nB + mbcnt(m);
      if (f && r < 64) Bb[r] = q;
      nB += __popcll(m);
    }
    if (nB > 64) nB = 64;
    for (int i = l; i < kGreedySpan / 4; i += 64) reinterpret_cast<uint32_t*>(stepA)[i] = 0x40404040u;
    wave_sync();
    const int pj = l < nA ? Ab[l] : 0;
    const int xj = l < nA ? (int)perm[pj] : 0x7fffffff;
    const int yj = l < nB ? Bb[l] : 0x7fffffff;
    if (l < nA && xj - b < kGreedySpan) stepA[xj - b] = (uint8_t)l;
    wave_sync();
    // y_j taken by the order at step i <= j
    const bool hit = l < nB && (int)stepA[yj - b] <= l;
    int yprev = __shfl_up(yj, 1);
    if (l == 0) yprev = b - 1;
    const bool stop = l >= nA || l >= nB || xj <= yprev || hit;
    const u64 sm = ballot(stop);
    const int js = sm ? (int)__builtin_ctzll(sm) : 64;
    if (js > 0) {
      if (l < js) {
        px[np + l] = xj;
        py[np + l] = yj;
        atomicOr(&taken[xj >> 5], 1u << (xj & 31));
      }
      np += js;
      a = js < nA ? rdlane(pj, js) : scan_whole ? min(aEnd, n) : rdlane(pj, js - 1) + 1;
      // indices the low end's scan passed were taken: it resumes at its next candidate
      b = js < nB ? rdlane(yj, js) : rdlane(yj, js - 1) + 1;
      wave_sync();
      continue;
    }
    if (nB == 0 && lim < n) {   // every index in [b, lim) is taken: the low end passes them
      b = lim;
      continue;
    }
    // one exact step: the order takes x_0; the low end takes the first untaken index after it
    const int x0 = rdlane(xj, 0);
    a = rdlane(pj, 0) + 1;
    if (l == 0) atomicOr(&taken[x0 >> 5], 1u << (x0 & 31));
    wave_sync();
    int y = -1;
    for (int q0 = b; q0 < n; q0 += 64) {
      const int q = q0 + l;
      const bool f = q < n && !((taken[q >> 5] >> (q & 31)) & 1u);
      const u64 m = ballot(f);
      if (m) {
        y = q0 + (int)__builtin_ctzll(m);
        break;
      }
    }
    if (y < 0) {
      lf = x0;
      break;
    }
    if (l == 0) {
      px[np] = x0;
      py[np] = y;
    }
    ++np;
    b = y + 1;
    wave_sync();
  }
  *left = lf;
  return np;
}

__device__ __forceinline__ void sort4(int32_t* m) {   // ascending, -1 entries last
  auto key = [](int32_t v) { return v < 0 ? 0x7fffffff : v; };
  for (int i = 1; i < 4; ++i) {
    const int32_t v = m[i];
    int j = i;
    while (j > 0 && key(m[j - 1]) > key(v)) {
      m[j] = m[j - 1];
      --j;
    }
    m[j] = v;
  }
}

// Stage B for window w with NW waves.  Small windows keep the unit order in LDS (P = uint16_t,
// arrays given), large ones in LDS too up to kLdsUnits units, else in global memory.
template <int NW, class P>
__device__ void plan_window(const Build& B, int32_t w, P* perm, uint32_t* taken, uint8_t* unnz_w, uint8_t* leaf_w,
                            int32_t* px, int32_t* py, WinShared& sh, int* LRbuf, int* gbuf, int32_t* tmp) {
  const int tid = threadIdx.x, l = lane_id(), wv = tid >> 6;
  constexpr int NT = NW * 64;
  const int32_t ub = B.ubase[w], U = B.ubase[w + 1] - ub;
  const uint32_t* umask = B.umask + ub;
  int32_t* ustat = B.ustat + ub;
  int32_t* ord = B.ord + ub;
  int32_t* tcl = B.tcl + ub + 8 * w;
  int32_t* gl = B.gl + ub + 4 * w;
  for (int i = tid; i < U; i += NT) ustat[i] = -1;
  __syncthreads();

  // TC chunks (block_online.cpp:215-253)
  int nsub = 0, tvals = 0;
  if (!B.skip_tc) {
    const int density = B.density;
    const int ntc = count_sort<NW>(umask, U, [&](int u) { return popc32(umask[u]) >= density; }, ord, sh);
    if (wv == 0) {
      for (int i = l; i < ((ntc + 7) & ~7); i += 64) tcl[i] = -1;
      wave_sync();
      int acc = 0, tv = 0;
      for (int c0 = 0; c0 < ntc; c0 += 64) {
        const int j = c0 + l;
        const bool valid = j < ntc;
        const int u = valid ? ord[j] : 0x7fffffff;
        const int cnt = valid ? popc32(umask[u]) : 0;
        int sum = cnt;   // nnz of this lane's chunk of 8
        sum += __shfl_xor(sum, 1);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 4);
        const float util = (float)sum / (float)(B.ws * 8);
        const bool chunk_exists = ((c0 + (l & ~7)) < ntc);
        const bool accept = chunk_exists && !(util < B.tc_min_util);
        const u64 lead = ballot(accept && (l & 7) == 0);
        const int sub = acc + mbcnt(lead & ((1ull << (l & ~7)) - 1) & lead) ;
        int k = 0;
        for (int i = 0; i < 8; ++i) {
          const int v = __shfl(u, (l & ~7) + i);
          if (v < u) ++k;
        }
        if (valid && accept) {
          ustat[u] = sub * 8 + k;
          tcl[sub * 8 + k] = u;
          tv += cnt;
        }
        acc += __popcll(lead);
      }
      for (int d = 1; d < 64; d <<= 1) tv += __shfl_xor(tv, d);
      nsub = acc;
      tvals = tv;
      if (l == 0) {
        sh.misc[0] = nsub;
        sh.misc[1] = tvals;
      }
    }
    __syncthreads();
    nsub = sh.misc[0];
    tvals = sh.misc[1];
  }

  // units (block_online.cpp:267-328): the remaining columns in (count desc, column asc) order
  const int n2 = count_sort<NW>(umask, U, [&](int u) { return ustat[u] < 0; }, ord, sh);
  const int n = (n2 + 1) >> 1;
  for (int i = tid; i < n; i += NT) {
    const int a = popc32(umask[ord[2 * i]]);
    const int b = 2 * i + 1 < n2 ? popc32(umask[ord[2 * i + 1]]) : 0;
    unnz_w[i] = (uint8_t)(a + b);
  }
  if (tid <= kMaxKey) {
    sh.start_of[tid] = -1;
    sh.end_of[tid] = 0;
  }
  __syncthreads();
  for (int i = tid; i < n; i += NT) {
    const int k = unnz_w[i];
    if (i == 0 || unnz_w[i - 1] != k) sh.start_of[k] = i;
    if (i == n - 1 || unnz_w[i + 1] != k) sh.end_of[k] = i + 1;
    perm[i] = (P)i;
    leaf_w[i] = 0;
  }
  __syncthreads();

  // the order: std::sort(0..n-1, nnz desc) (block_online.cpp:358-363)
  int* Lbuf = LRbuf + wv * 256;
  int* Rbuf = Lbuf + 128;
  if (n > 16) {
    if constexpr (NW == 1) {
      wave_introsort(perm, n, unnz_w, leaf_w, sh, Lbuf, Rbuf, tmp, B.err);
    } else {
      // level by level: each wave takes ranges of the current list, children go to the next
      int* lists = B.ranges + ub;   // two lists of (first, last, depth), (U / 2) ints each
      const int cap = (U / 2) / 3;
      int cur = 0;
      if (tid == 0) {
        lists[0] = 0;
        lists[1] = n;
        lists[2] = pack_range(2 * trs::isort::lg(n), unnz_w[n - 1], unnz_w[0]);
        sh.cnt[0] = 1;
        sh.cnt[1] = 0;
      }
      __syncthreads();
      for (int level = 0; level < 64; ++level) {
        const int ncur = sh.cnt[cur];
        if (ncur == 0) break;
        int* lc = lists + cur * (U / 2);
        int* ln = lists + (cur ^ 1) * (U / 2);
        for (int r = wv; r < ncur; r += NW) {
          const int f = lc[3 * r], last = lc[3 * r + 1], packed = lc[3 * r + 2];
          const int d = packed & 0xff, kmin = (packed >> 8) & 0xff, kmax = packed >> 16;
          if (kmin == kmax && trs::isort::tied_depth_ok(last - f, d)) {
            wave_tied(perm, f, last - f, tmp);
            continue;
          }
          if (d == 0) {
            lane0_heap_sort(perm, f, last, unnz_w);
            continue;
          }
          int pk = 0;
          const int cut = wave_partition(perm, f, last, unnz_w, sh, Lbuf, Rbuf, B.err, &pk);
          if (l == 0) {
            const int cf[2] = {f, cut}, cl[2] = {cut, last};
            const int cp[2] = {pack_range(d - 1, pk, kmax), pack_range(d - 1, kmin, pk)};
            for (int h = 0; h < 2; ++h) {
              const int len = cl[h] - cf[h];
              if (len > 16) {
                const int at = atomicAdd(&sh.cnt[cur ^ 1], 1);
                if (at < cap) {
                  ln[3 * at] = cf[h];
                  ln[3 * at + 1] = cl[h];
                  ln[3 * at + 2] = cp[h];
                } else {
                  atomicOr(B.err, kErrInternal);
                }
              } else {
                leaf_w[cf[h]] = (uint8_t)len;
              }
            }
          }
        }
        __syncthreads();
        if (tid == 0) {
          sh.cnt[cur] = 0;
          if (sh.cnt[cur ^ 1] > cap) sh.cnt[cur ^ 1] = cap;
        }
        cur ^= 1;
        __syncthreads();
      }
    }
    __syncthreads();
    sort_leaves(perm, n, leaf_w, unnz_w, 0, NT);
    __syncthreads();
  }
  for (int i = tid; i < n / 32 + 2; i += NT) taken[i] = 0u;
  __syncthreads();

  // greedy matching (block_online.cpp:365-391)
  if (wv == 0) {
    int left = -1;
    const int np = wave_greedy(perm, taken, n, px, py, &left, gbuf);
    if (l == 0) {
      sh.misc[2] = np;
      sh.misc[3] = left;
    }
  }
  __syncthreads();
  const int np = sh.misc[2], left = sh.misc[3];
  // groups (block_online.cpp:629-666): pairs in order, then the unmatched unit if big enough
  for (int k = tid; k < np; k += NT) {
    const int x = px[k], y = py[k];
    int32_t m[4] = {ord[2 * x], 2 * x + 1 < n2 ? ord[2 * x + 1] : -1, ord[2 * y], 2 * y + 1 < n2 ? ord[2 * y + 1] : -1};
    sort4(m);
    for (int q = 0; q < 4; ++q) {
      gl[4 * k + q] = m[q];
      if (m[q] >= 0) ustat[m[q]] = -2;
    }
  }
  int ngroups = np, nres = 0, r0 = -1, r1 = -1;
  if (left >= 0) {
    int32_t m[4] = {ord[2 * left], 2 * left + 1 < n2 ? ord[2 * left + 1] : -1, -1, -1};
    sort4(m);
    if ((int)unnz_w[left] >= B.unit_min) {
      if (tid < 4) {
        gl[4 * np + tid] = m[tid];
        if (m[tid] >= 0) ustat[m[tid]] = -2;
      }
      ngroups = np + 1;
    } else {
      r0 = m[0];
      r1 = m[1];
      nres = r1 >= 0 ? 2 : 1;
    }
  }
  if (tid == 0) {
    WinOut o;
    o.nsub = nsub;
    o.ngroups = ngroups;
    o.tvals = tvals;
    o.nres = nres;
    o.res[0] = r0;
    o.res[1] = r1;
    o.pad[0] = o.pad[1] = 0;
    B.win[w] = o;
  }
}

// Windows of at most kSmallU distinct columns, one wave each (workgroups of one wave); matched
// pairs go to the window's part of B.pairs.
__global__ __launch_bounds__(64) void k_plan_small(Build B) {
  const int32_t w = blockIdx.x;
  const int32_t ub = B.ubase[w], U = B.ubase[w + 1] - ub;
  if (U > kSmallU) return;
  __shared__ uint16_t perm[kSmallU / 2 + 1];
  __shared__ uint8_t unnz[kSmallU / 2 + 1];
  __shared__ uint8_t leaf[kSmallU / 2 + 1];
  __shared__ uint32_t taken[kSmallU / 64 + 2];
  __shared__ int LR[256];
  __shared__ int GB[512];
  __shared__ WinShared sh;
  int32_t* px = B.pairs + ub;
  int32_t* py = px + (U + 3) / 4 + 1;
  plan_window<1>(B, w, perm, taken, unnz, leaf, px, py, sh, LR, GB, B.gperm + ub);
}

// The other windows, a workgroup of kBlockWaves waves each, largest first (window list `big`):
// unit order (16-bit indices) and taken bits in LDS for windows of at most B.lds_units units ...
__global__ __launch_bounds__(kBlockWaves * 64) void k_plan_large(Build B, const int32_t* big, int32_t nbig) {
  extern __shared__ uint16_t lds_perm[];   // B.lds_units entries, then the taken bits
  __shared__ int LR[kBlockWaves * 256];
  __shared__ int GB[512];
  __shared__ WinShared sh;
  uint32_t* taken = reinterpret_cast<uint32_t*>(lds_perm + ((B.lds_units + 1) & ~1));
  for (int32_t i = blockIdx.x; i < nbig; i += gridDim.x) {
    const int32_t w = big[i];
    const int32_t ub = B.ubase[w];
    const int32_t U = B.ubase[w + 1] - ub;
    // units <= ceil(U / 2); the global arrays are sized by U at the window's offset
    int32_t* px = B.pairs + ub;
    int32_t* py = px + (U + 3) / 4 + 1;
    plan_window<kBlockWaves>(B, w, lds_perm, taken, B.unnz + ub, B.leaf + ub, px, py, sh, LR, GB, B.gperm + ub);
    __syncthreads();
  }
}

// ... and in global memory for larger ones.
__global__ __launch_bounds__(kBlockWaves * 64) void k_plan_huge(Build B, const int32_t* big, int32_t nbig) {
  __shared__ int LR[kBlockWaves * 256];
  __shared__ int GB[512];
  __shared__ WinShared sh;
  for (int32_t i = blockIdx.x; i < nbig; i += gridDim.x) {
    const int32_t w = big[i];
    const int32_t ub = B.ubase[w];
    const int32_t U = B.ubase[w + 1] - ub;
    int32_t* px = B.pairs + ub;
    int32_t* py = px + (U + 3) / 4 + 1;
    plan_window<kBlockWaves>(B, w, B.gperm + ub, reinterpret_cast<uint32_t*>(B.gpos + ub), B.unnz + ub,
                             B.leaf + ub, px, py, sh, LR, GB, B.gpos + ub);
    __syncthreads();
  }
}

// Windows for the workgroup kernels: (distinct columns, window) of each, big[0, nbig) (the host
// orders them, largest first, and splits them between the two kernels).
__global__ __launch_bounds__(256) void k_list_large(Build B, int32_t* big, int32_t* nbig) {
  const int32_t w = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (w >= B.nwin) return;
  const int32_t U = B.ubase[w + 1] - B.ubase[w];
  if (U <= kSmallU) return;
  const int32_t i = atomicAdd(nbig, 1);
  big[2 * i] = U;
  big[2 * i + 1] = w;
}

// ---- stage C: counts -----------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_window_counts(Build B) {
  const int32_t w = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (w >= B.nwin) return;
  const WinOut o = B.win[w];
  const int32_t parts = o.nsub == 0 ? 0 : o.nsub <= B.part_t ? 1 : o.nsub / B.part_t + (o.nsub % B.part_t ? 1 : 0);
  B.wparts[w] = parts;
  B.wsubs[w] = o.nsub;
  B.wtvals[w] = o.tvals;
  B.wgroups[w] = o.ngroups;
  B.wtiles[w] = (o.ngroups + 3) / 4;
}

// Residual entries of row r (block_online.cpp:705-733, split as :397-439).
__device__ __forceinline__ int residual_count(const Build& B, int32_t r, const WinOut& o, int32_t ub) {
  const int lr = r % B.ws;
  int n = 0;
  for (int j = 0; j < o.nres; ++j) n += (B.umask[ub + o.res[j]] >> lr) & 1u;
  return n;
}

__global__ __launch_bounds__(256) void k_row_counts(Build B) {
  const int32_t r = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (r >= B.rows) return;
  const int32_t w = r / B.ws;
  const WinOut o = B.win[w];
  const int n = residual_count(B, r, o, B.ubase[w]);
  int lp = 0, le = 0, sp = 0, se = 0;
  if (n > 0) {
    if (n <= B.short_size) {
      sp = 1;
      se = n;
    } else if (n <= B.part_c) {
      lp = 1;
      le = n;
    } else {
      lp = n / B.part_c;
      le = lp * B.part_c;
      const int rem = n % B.part_c;
      if (rem > 0) {
        if (rem <= B.short_size) {
          sp = 1;
          se = rem;
        } else {
          lp += 1;
          le += rem;
        }
      }
    }
  }
  B.rlp[r] = lp;
  B.rle[r] = le;
  B.rsp[r] = sp;
  B.rse[r] = se;
}

// ---- stage D: the arrays -------------------------------------------------------------------
// The window holding item i of a per-window numbering with exclusive bases base[0..nwin]
// (base[nwin] = the total; i below it).
__device__ __forceinline__ int32_t window_of(const int32_t* base, int32_t nwin, int32_t i) {
  int32_t lo = 0, hi = nwin;   // base[lo] <= i < base[hi]
  while (hi - lo > 1) {
    const int32_t mid = (lo + hi) >> 1;
    if (base[mid] <= i) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Per window: TC parts (block_online.cpp:502-537), group and tile offsets (:736-776, :840).
__global__ __launch_bounds__(256) void k_fill_windows(Build B, Out O) {
  const int32_t w = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (w == 0) {
    O.t_rowoff[0] = 0;
    O.s_offsets[B.nwin] = B.wgroups[B.nwin];
    O.win_tile_off[B.nwin] = B.wtiles[B.nwin];
  }
  if (w >= B.nwin) return;
  O.s_offsets[w] = B.wgroups[w];
  O.win_tile_off[w] = B.wtiles[w];
  const WinOut o = B.win[w];
  if (o.nsub == 0) return;
  const int32_t pb = B.wparts[w], sb = B.wsubs[w];
  const int32_t nparts = B.wparts[w + 1] - pb;
  for (int q = 0; q < nparts; ++q) {
    O.t_rowoff[pb + q + 1] = sb + min((q + 1) * B.part_t, o.nsub);
    O.t_winrow[pb + q] = w * 16;   // block_online.cpp:494 (window id * 16 for every window size)
    O.t_atomic[pb + q] = nparts == 1 ? (o.nres > 0 ? 1 : 0) : 1;
  }
}

// Values per TC sub-block (their prefix sums are t_blockNew_offset).
__global__ __launch_bounds__(256) void k_tc_counts(Build B, int32_t nsubs, int32_t* __restrict__ cnt) {
  const int32_t s = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (s >= nsubs) return;
  const int32_t w = window_of(B.wsubs, B.nwin, s);
  const int32_t ub = B.ubase[w];
  const int32_t* tcl = B.tcl + ub + 8 * w + (int64_t)(s - B.wsubs[w]) * 8;
  int c = 0;
  for (int k = 0; k < 8; ++k)
    if (tcl[k] >= 0) c += popc32(B.umask[ub + tcl[k]]);
  cnt[s] = c;
}

// TC sub-block s: columns, row bits and values (block_online.cpp:444-540): bit (row % 8) * 8 + k
// of t_binary[2s] (rows 0-7) or [2s + 1] (rows 8-15); values in ascending bit order, which is the
// rows' CSR order.
__global__ __launch_bounds__(256) void k_fill_tc(Build B, Out O, int32_t nsubs) {
  const int32_t s = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (s >= nsubs) return;
  const int32_t w = window_of(B.wsubs, B.nwin, s);
  const int32_t ub = B.ubase[w];
  const int32_t* tcl = B.tcl + ub + 8 * w + (int64_t)(s - B.wsubs[w]) * 8;
  uint64_t lo = 0, hi = 0;
  int32_t u[8];
  for (int k = 0; k < 8; ++k) {
    u[k] = tcl[k];
    O.t_col[(int64_t)s * 8 + k] = u[k] >= 0 ? B.ucol[ub + u[k]] : -1;
    if (u[k] < 0) continue;
    uint32_t m = B.umask[ub + u[k]];
    while (m) {
      const int lr = __builtin_ctz(m);
      m &= m - 1;
      if (lr < 8) lo |= 1ull << (lr * 8 + k);
      else hi |= 1ull << ((lr - 8) * 8 + k);
    }
  }
  O.t_bin[2 * (int64_t)s] = (int64_t)lo;
  O.t_bin[2 * (int64_t)s + 1] = (int64_t)hi;
  int32_t vi = O.t_blockoff[s];
  for (int half = 0; half < 2; ++half) {
    uint64_t bits = half ? hi : lo;
    while (bits) {
      const int b = __builtin_ctzll(bits);
      bits &= bits - 1;
      const int lr = half * 8 + b / 8, k = b % 8;
      O.t_val[vi++] = B.val[entry_of(B, ub + u[k], lr)];
    }
  }
}

// Window of each 2:4 group (s_window, block_online.cpp:664).
__global__ __launch_bounds__(256) void k_group_windows(Build B, Out O, int32_t ngroups) {
  const int32_t g = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (g < ngroups) O.s_win[g] = window_of(B.wgroups, B.nwin, g);
}

// Group g, local row lr: columns (lr = 0), the row's mask, its first two values and their
// positions; the row's further values are spilled (block_online.cpp:629-703).
__global__ __launch_bounds__(256) void k_fill_groups(Build B, Out O, int64_t items) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= items) return;
  const int ws = B.ws;
  const int32_t g = (int32_t)(t / ws);
  const int lr = (int)(t - (int64_t)g * ws);
  const int32_t w = O.s_win[g];
  const int32_t ub = B.ubase[w];
  const int32_t* gl = B.gl + ub + 4 * w + (int64_t)(g - B.wgroups[w]) * 4;
  uint32_t present = 0;
  int kept = 0;
  float v[2] = {0.f, 0.f};
  int p[2] = {-1, -1};
  for (int q = 0; q < 4; ++q) {
    const int32_t m = gl[q];
    if (lr == 0) O.s_col[(int64_t)g * 4 + q] = m >= 0 ? B.ucol[ub + m] : -1;
    if (m < 0 || !((B.umask[ub + m] >> lr) & 1u)) continue;
    present |= 1u << q;
    const int32_t e = entry_of(B, ub + m, lr);
    if (kept < 2) {
      v[kept] = B.val[e];
      p[kept] = q;
    } else {
      B.spill[e] = 1;
    }
    ++kept;
  }
  O.s_mask[t] = (uint8_t)present;
  O.s_val[2 * t] = v[0];
  O.s_val[2 * t + 1] = v[1];
  O.s_pos[2 * t] = (int8_t)p[0];
  O.s_pos[2 * t + 1] = (int8_t)p[1];
}

// block_online.cpp:190-210 (g window-local, gend the window's group count)
__device__ __forceinline__ void load_chunk(const Out& O, int64_t gb, int g, int gend, int lr, int ws, float& v0,
                                           float& v1, int& p0, int& p1) {
  v0 = v1 = 0.f;
  p0 = 0;
  p1 = 1;
  if (g >= gend || lr >= ws) return;
  const int64_t b = ((gb + g) * ws + lr) * 2;
  const int q0 = O.s_pos[b], q1 = O.s_pos[b + 1];
  const float a0 = O.s_val[b], a1 = O.s_val[b + 1];
  if (q0 < 0 && q1 < 0) return;
  if (q0 >= 0 && q1 >= 0) {
    if (q0 <= q1) {
      p0 = q0; p1 = q1; v0 = a0; v1 = a1;
    } else {
      p0 = q1; p1 = q0; v0 = a1; v1 = a0;
    }
    return;
  }
  const int rp = q0 >= 0 ? q0 : q1;
  const float rv = q0 >= 0 ? a0 : a1;
  const int dummy = rp == 0 ? 1 : 0;
  if (dummy < rp) {
    p0 = dummy; p1 = rp; v0 = 0.f; v1 = rv;
  } else {
    p0 = rp; p1 = dummy; v0 = rv; v1 = 0.f;
  }
}

__device__ __forceinline__ uint16_t f16_bits(float f) { return trs::half_bits_of(__float_as_uint(f)); }

// Tile t: 4 groups of its window (block_online.cpp:796-841).
__global__ __launch_bounds__(256) void k_fill_tiles(Build B, Out O, int32_t ntiles) {
  const int32_t t = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (t >= ntiles) return;
  const int ws = B.ws;
  const int32_t w = window_of(B.wtiles, B.nwin, t);
  const int32_t gb = B.wgroups[w], G = B.wgroups[w + 1] - gb;
  const int base = (t - B.wtiles[w]) * 4;
  O.tile_win[t] = w;
  O.tile_group[t] = gb + base;
  for (int k = 0; k < 16; ++k) {
    const int g = base + k / 4;
    O.tile_cols[(int64_t)t * 16 + k] = g < G ? O.s_col[((int64_t)gb + g) * 4 + k % 4] : -1;
  }
  for (int rg = 0; rg < 8; ++rg) {
    float a[16];
    uint32_t meta = 0;
    for (int c = 0; c < 4; ++c) {
      int p0, p1;
      load_chunk(O, gb, base + c, G, rg, ws, a[4 * c], a[4 * c + 1], p0, p1);
      meta |= ((uint32_t)(p0 & 3) | ((uint32_t)(p1 & 3) << 2)) << (4 * c);
      load_chunk(O, gb, base + c, G, rg + 8, ws, a[4 * c + 2], a[4 * c + 3], p0, p1);
      meta |= ((uint32_t)(p0 & 3) | ((uint32_t)(p1 & 3) << 2)) << (16 + 4 * c);
    }
    O.packed_meta[(int64_t)t * 8 + rg] = (int32_t)meta;
    for (int j = 0; j < 8; ++j)
      O.packed_a[((int64_t)t * 8 + rg) * 8 + j] =
          (int32_t)((uint32_t)f16_bits(a[2 * j]) | ((uint32_t)f16_bits(a[2 * j + 1]) << 16));
  }
}

// Residual parts of row r (block_online.cpp:397-439, :705-733): entries of the window's residual
// columns in the row, ascending column (CSR) order.
__global__ __launch_bounds__(256) void k_fill_residual(Build B, Out O) {
  const int32_t r = (int32_t)(blockIdx.x * 256 + threadIdx.x);
  if (r == 0) {
    O.c_off[0] = 0;
    O.cs_off[0] = 0;
  }
  if (r >= B.rows) return;
  const int32_t w = r / B.ws;
  const int lr = r - w * B.ws;
  const WinOut o = B.win[w];
  if (o.nres == 0) return;
  const int32_t ub = B.ubase[w];
  int32_t ent[2];
  int n = 0;
  for (int j = 0; j < o.nres; ++j)
    if ((B.umask[ub + o.res[j]] >> lr) & 1u) ent[n++] = entry_of(B, ub + o.res[j], lr);
  if (n == 0) return;
  const int base_atomic = o.nsub > 0 ? 1 : 0;
  int32_t lp = B.rlp[r], le = B.rle[r], sp = B.rsp[r], se = B.rse[r];
  auto emit = [&](bool shrt, int atomic, int off, int cnt) {
    if (shrt) {
      O.cs_row[sp] = r;
      O.cs_atomic[sp] = atomic;
      for (int i = 0; i < cnt; ++i) {
        O.cs_col[se + i] = B.col[ent[off + i]];
        O.cs_val[se + i] = B.val[ent[off + i]];
      }
      se += cnt;
      O.cs_off[++sp] = se;
    } else {
      O.c_row[lp] = r;
      O.c_atomic[lp] = atomic;
      for (int i = 0; i < cnt; ++i) {
        O.c_col[le + i] = B.col[ent[off + i]];
        O.c_val[le + i] = B.val[ent[off + i]];
      }
      le += cnt;
      O.c_off[++lp] = le;
    }
  };
  if (n <= B.short_size) {
    emit(true, base_atomic, 0, n);
  } else if (n <= B.part_c) {
    emit(false, base_atomic, 0, n);
  } else {
    const int full = n / B.part_c;
    int off = 0;
    for (int i = 0; i < full; ++i, off += B.part_c) emit(false, 1, off, B.part_c);
    const int rem = n % B.part_c;
    if (rem > 0) emit(rem <= B.short_size, 1, off, rem);
  }
}

// Spill entries in CSR order (block_online.cpp drops them; slots 29-31).
__global__ __launch_bounds__(256) void k_fill_spill(Build B, Out O) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= B.nnz || !B.spill[e]) return;
  const int32_t i = B.spill_at[e];
  O.spill_row[i] = row_of(B.rowptr, B.rows, e);
  O.spill_col[i] = B.col[e];
  O.spill_val[i] = B.val[e];
}

// ---- host ----------------------------------------------------------------------------------
unsigned grid_of(int64_t n, int per = 256) { return (unsigned)std::max<int64_t>(1, (n + per - 1) / per); }

struct Arena {   // bump allocation inside one hipMalloc
  char* base = nullptr;
  size_t used = 0, cap = 0;
  template <class T>
  T* take(int64_t n) {
    used = (used + 255) & ~size_t(255);
    T* p = reinterpret_cast<T*>(base + used);
    used += (size_t)std::max<int64_t>(n, 1) * sizeof(T);
    return p;
  }
};
template <class T>
size_t bytes_of(int64_t n) { return (((size_t)std::max<int64_t>(n, 1) * sizeof(T)) + 255) & ~size_t(255); }

int fail(int code, const std::string& msg) {
  trs::set_error(msg);
  return code;
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

struct DevBuf {
  void* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
};

}  // namespace

extern "C" {

int trs_build_online_device(const int32_t* rowptr, const int32_t* col, const float* val, int32_t rows, int64_t nnz,
                            const trs_build_params* prm, void* stream, trs_dformat** out) {
  if (!out) return fail(TRS_EINVAL, "trs_build_online_device: out is NULL");
  *out = nullptr;
  if (!prm) return fail(TRS_EINVAL, "trs_build_online_device: params is NULL");
  if (prm->struct_size != (int32_t)sizeof(trs_build_params))
    return fail(TRS_EINVAL, "trs_build_online_device: trs_build_params.struct_size is " +
                                std::to_string(prm->struct_size) + ", this library's is " +
                                std::to_string(sizeof(trs_build_params)));
  if (!(prm->window > 0 && prm->window <= 32 && prm->wide > 0 && prm->wide <= 32))
    return fail(TRS_EINVAL, "trs_build_online_device: requires 0 < window <= 32 and 0 < wide <= 32");
  if (prm->window > 16)
    return fail(TRS_EINVAL, "trs_build_online_device: windows of more than 16 rows are built on the host "
                            "(trs_build_online)");
  if (rows < 0 || nnz < 0 || !rowptr || (nnz > 0 && (!col || !val)) || nnz > INT32_MAX)
    return fail(TRS_EINVAL, "trs_build_online_device: bad CSR arguments");
  if (prm->part_size_t <= 0 || prm->part_size_c <= 0)
    return fail(TRS_EINVAL, "trs_build_online_device: partSize_t and partSize_c must be positive");
  const auto t0 = std::chrono::high_resolution_clock::now();
  hipStream_t s = static_cast<hipStream_t>(stream);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(TRS_EDEVICE, "trs_build_online_device: no HIP device");
  }

  // LDS of the workgroup window kernel: its static arrays, then the unit order (16-bit)
  int max_lds = 0;
  hipFuncAttributes fa{};
  if (hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
      hipFuncGetAttributes(&fa, (const void*)k_plan_large) != hipSuccess) {
    (void)hipGetLastError();
    return fail(TRS_EDEVICE, "trs_build_online_device: device attributes unavailable");
  }
  Build B;
  // 2 bytes of order and 1 taken bit per unit
  B.lds_units = (int32_t)std::min<int64_t>(
      kLdsUnits, std::max<int64_t>(0, ((int64_t)max_lds - (int64_t)fa.sharedSizeBytes - 1024) * 8 / 17));
  B.rows = rows;
  B.ws = prm->window;
  B.nwin = (rows + B.ws - 1) / B.ws;
  B.nnz = nnz;
  B.rowptr = rowptr;
  B.col = col;
  B.val = val;
  B.part_t = prm->part_size_t;
  B.part_c = prm->part_size_c;
  B.short_size = prm->short_size;
  B.density = prm->density;
  B.tc_min_util = prm->tc_min_util;
  B.skip_tc = prm->skip_tc >= 0 ? (prm->skip_tc != 0) : env_flag("LIBRA_SKIP_TC", false);
  B.unit_min = prm->sptc_unit_min_nnz >= 0 ? prm->sptc_unit_min_nnz : env_int("LIBRA_SPTC_UNIT_MIN_NNZ", 2);
  const int32_t W = B.nwin;

  // phase 1: validation and stage A
  DevBuf s1;
  const size_t need1 = bytes_of<uint32_t>(4) + bytes_of<int32_t>(nnz) * 2 + bytes_of<uint8_t>(nnz) * 2 +
                       bytes_of<int32_t>(nnz + 1) + bytes_of<int32_t>(W + 1) + bytes_of<int32_t>(scan_scratch_ints(nnz) + 64);
  if (hipMalloc(&s1.p, need1) != hipSuccess) {
    (void)hipGetLastError();
    return fail(TRS_ENOMEM, "trs_build_online_device: hipMalloc of " + std::to_string(need1) + " bytes failed");
  }
  Arena A1{static_cast<char*>(s1.p), 0, need1};
  B.err = A1.take<uint32_t>(4);
  B.s_col = A1.take<int32_t>(nnz);
  B.s_e = A1.take<int32_t>(nnz);
  B.s_lr = A1.take<uint8_t>(nnz);
  B.s_new = A1.take<uint8_t>(nnz);
  B.s_u = A1.take<int32_t>(nnz + 1);
  B.ubase = A1.take<int32_t>(W + 1);
  int32_t* bsum = A1.take<int32_t>(scan_scratch_ints(nnz) + 64);
  uint32_t herr[4] = {0, 0, 0, 0};
  int32_t ends[2] = {-1, -1};
  if (hipMemsetAsync(B.err, 0, 16, s) != hipSuccess) return fail(TRS_EDEVICE, "hipMemsetAsync failed");
  hipLaunchKernelGGL(k_check_rows, dim3(grid_of(rows)), dim3(256), 0, s, rowptr, rows, B.err);
  if (hipMemcpyAsync(&ends[0], rowptr, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipMemcpyAsync(&ends[1], rowptr + rows, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipMemcpyAsync(herr, B.err, 16, hipMemcpyDeviceToHost, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
    return fail(TRS_EDEVICE, std::string("trs_build_online_device: ") + hipGetErrorString(hipGetLastError()));
  if (ends[0] != 0 || (int64_t)ends[1] != nnz)
    return fail(TRS_EINVAL, "trs_build_online_device: rowptr must start at 0 and end at nnz");
  if (herr[0]) return fail(TRS_EINVAL, "trs_build_online_device: rowptr must be non-decreasing");
  if (nnz > 0) {
    hipLaunchKernelGGL(k_rank, dim3(grid_of(nnz)), dim3(256), 0, s, B);
    hipLaunchKernelGGL(k_new_columns, dim3(grid_of(nnz)), dim3(256), 0, s, B);
  }
  if (scan(B.s_new, nnz, B.s_u, bsum, s) != hipSuccess) return fail(TRS_EDEVICE, "scan failed");
  hipLaunchKernelGGL(k_window_bases, dim3(grid_of(W + 1)), dim3(256), 0, s, B);
  int32_t U = 0;
  if (hipMemcpyAsync(&U, B.s_u + nnz, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipMemcpyAsync(herr, B.err, 16, hipMemcpyDeviceToHost, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
    return fail(TRS_EDEVICE, std::string("trs_build_online_device: ") + hipGetErrorString(hipGetLastError()));
  if (herr[0] & kErrNegativeColumn) return fail(TRS_EINVAL, "trs_build_online_device: negative column index");
  if (herr[0] & kErrNonCanonical)
    return fail(TRS_ENOTCANON, "trs_build_online_device: a row's columns are not strictly increasing (build such "
                               "input with trs_build_online)");
  B.U = U;

  // phase 2: stages B and C
  DevBuf s2;
  const int64_t Ue = (int64_t)U + 8 * (int64_t)W + 64;
  const size_t need2 = bytes_of<int32_t>(U) * 3 + bytes_of<uint32_t>(U) + bytes_of<int32_t>(U + 1) +
                       bytes_of<int32_t>(Ue) * 2 + bytes_of<uint8_t>(U) * 2 + bytes_of<int32_t>(U) * 4 +
                       bytes_of<WinOut>(W) + bytes_of<int32_t>(W + 1) * 5 + bytes_of<int32_t>(rows + 1) * 4 +
                       bytes_of<uint8_t>(nnz) + bytes_of<int32_t>(nnz + 1) + bytes_of<int32_t>(2 * (int64_t)W + 2) +
                       bytes_of<int32_t>(scan_scratch_ints(std::max<int64_t>(nnz, rows)) + 64);
  if (hipMalloc(&s2.p, need2) != hipSuccess) {
    (void)hipGetLastError();
    return fail(TRS_ENOMEM, "trs_build_online_device: hipMalloc of " + std::to_string(need2) + " bytes failed");
  }
  Arena A2{static_cast<char*>(s2.p), 0, need2};
  B.ucol = A2.take<int32_t>(U);
  B.umask = A2.take<uint32_t>(U);
  B.ufirst = A2.take<int32_t>(U + 1);
  B.ustat = A2.take<int32_t>(U);
  B.ord = A2.take<int32_t>(U);
  B.tcl = A2.take<int32_t>(Ue);
  B.gl = A2.take<int32_t>(Ue);
  B.unnz = A2.take<uint8_t>(U);
  B.leaf = A2.take<uint8_t>(U);
  B.gperm = A2.take<int32_t>(U);
  B.gpos = A2.take<int32_t>(U);
  B.pairs = A2.take<int32_t>(U);
  B.ranges = A2.take<int32_t>(U);
  B.win = A2.take<WinOut>(W);
  B.wparts = A2.take<int32_t>(W + 1);
  B.wsubs = A2.take<int32_t>(W + 1);
  B.wtvals = A2.take<int32_t>(W + 1);
  B.wgroups = A2.take<int32_t>(W + 1);
  B.wtiles = A2.take<int32_t>(W + 1);
  B.rlp = A2.take<int32_t>(rows + 1);
  B.rle = A2.take<int32_t>(rows + 1);
  B.rsp = A2.take<int32_t>(rows + 1);
  B.rse = A2.take<int32_t>(rows + 1);
  B.spill = A2.take<uint8_t>(nnz);
  B.spill_at = A2.take<int32_t>(nnz + 1);
  int32_t* big = A2.take<int32_t>(2 * (int64_t)W + 2);
  int32_t* bsum2 = A2.take<int32_t>(scan_scratch_ints(std::max<int64_t>(nnz, rows)) + 64);
  int32_t* nbig_d = bsum2 + scan_scratch_ints(std::max<int64_t>(nnz, rows)) + 32;
  if (nnz > 0) hipLaunchKernelGGL(k_distinct, dim3(grid_of(nnz)), dim3(256), 0, s, B);
  if (hipMemsetAsync(nbig_d, 0, 8, s) != hipSuccess || hipMemsetAsync(B.spill, 0, (size_t)std::max<int64_t>(nnz, 1), s) != hipSuccess)
    return fail(TRS_EDEVICE, "hipMemsetAsync failed");
  if (W > 0) {
    hipLaunchKernelGGL(k_list_large, dim3(grid_of(W)), dim3(256), 0, s, B, big, nbig_d);
    hipLaunchKernelGGL(k_plan_small, dim3(W), dim3(64), 0, s, B);
    int32_t nbig = 0;
    if (hipMemcpyAsync(&nbig, nbig_d, 4, hipMemcpyDeviceToHost, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
      return fail(TRS_EDEVICE, std::string("trs_build_online_device: ") + hipGetErrorString(hipGetLastError()));
    if (nbig > 0) {
      // largest windows first (they take longest), split between the LDS and the global-memory
      // kernel by unit count
      std::vector<int32_t> lst(2 * (size_t)nbig);
      if (hipMemcpy(lst.data(), big, lst.size() * 4, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(TRS_EDEVICE, "trs_build_online_device: window list copy failed");
      std::vector<std::pair<int32_t, int32_t>> order((size_t)nbig);
      for (int32_t i = 0; i < nbig; ++i) order[i] = {lst[2 * i], lst[2 * i + 1]};
      std::sort(order.begin(), order.end(), [](const auto& x, const auto& y) {
        return x.first != y.first ? x.first > y.first : x.second < y.second;
      });
      std::vector<int32_t> in_lds, in_global;
      for (const auto& o : order) ((o.first + 1) / 2 <= B.lds_units ? in_lds : in_global).push_back(o.second);
      std::vector<int32_t> ids(in_lds);
      ids.insert(ids.end(), in_global.begin(), in_global.end());
      if (hipMemcpy(big, ids.data(), ids.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
        return fail(TRS_EDEVICE, "trs_build_online_device: window list copy failed");
      if (!in_lds.empty()) {
        const size_t lds = (size_t)((B.lds_units + 1) & ~1) * sizeof(uint16_t) + ((size_t)B.lds_units / 32 + 2) * 4;
        if (hipFuncSetAttribute((const void*)k_plan_large, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess)
          return fail(TRS_EDEVICE, "trs_build_online_device: the window kernel cannot get its LDS");
        hipLaunchKernelGGL(k_plan_large, dim3((unsigned)std::min<size_t>(in_lds.size(), 1024)), dim3(kBlockWaves * 64),
                           lds, s, B, big, (int32_t)in_lds.size());
      }
      if (!in_global.empty())
        hipLaunchKernelGGL(k_plan_huge, dim3((unsigned)std::min<size_t>(in_global.size(), 1024)),
                           dim3(kBlockWaves * 64), 0, s, B, big + in_lds.size(), (int32_t)in_global.size());
    }
    hipLaunchKernelGGL(k_window_counts, dim3(grid_of(W)), dim3(256), 0, s, B);
  }
  if (rows > 0) hipLaunchKernelGGL(k_row_counts, dim3(grid_of(rows)), dim3(256), 0, s, B);
  if (scan(B.wparts, W, B.wparts, bsum2, s) != hipSuccess || scan(B.wsubs, W, B.wsubs, bsum2, s) != hipSuccess ||
      scan(B.wtvals, W, B.wtvals, bsum2, s) != hipSuccess || scan(B.wgroups, W, B.wgroups, bsum2, s) != hipSuccess ||
      scan(B.wtiles, W, B.wtiles, bsum2, s) != hipSuccess || scan(B.rlp, rows, B.rlp, bsum2, s) != hipSuccess ||
      scan(B.rle, rows, B.rle, bsum2, s) != hipSuccess || scan(B.rsp, rows, B.rsp, bsum2, s) != hipSuccess ||
      scan(B.rse, rows, B.rse, bsum2, s) != hipSuccess)
    return fail(TRS_EDEVICE, "scan failed");
  int32_t tot[9];
  int32_t* srcs[9] = {B.wparts + W, B.wsubs + W, B.wtvals + W, B.wgroups + W, B.wtiles + W,
                      B.rlp + rows, B.rle + rows, B.rsp + rows, B.rse + rows};
  for (int i = 0; i < 9; ++i)
    if (hipMemcpyAsync(&tot[i], srcs[i], 4, hipMemcpyDeviceToHost, s) != hipSuccess)
      return fail(TRS_EDEVICE, "hipMemcpyAsync failed");
  if (hipMemcpyAsync(herr, B.err, 16, hipMemcpyDeviceToHost, s) != hipSuccess || hipStreamSynchronize(s) != hipSuccess)
    return fail(TRS_EDEVICE, std::string("trs_build_online_device: ") + hipGetErrorString(hipGetLastError()));
  if (herr[0] & kErrInternal)
    return fail(TRS_EDEVICE, "trs_build_online_device: internal error in the unit order (please report)");
  const int64_t P_t = tot[0], S_t = tot[1], TV = tot[2], G = tot[3], T = tot[4], Pc = tot[5], Ec = tot[6],
                Ps = tot[7], Es = tot[8];
  if (G > INT32_MAX / 32 || T > INT32_MAX / 64)
    return fail(TRS_ERANGE, "trs_build_online_device: output exceeds int32 index range");

  // phase 3: the format arrays (one allocation, kept by the result) and stage D
  auto* F = new trs_dformat();
  F->rows = rows;
  F->window = B.ws;
  F->device = dev;
  F->nnz = nnz;
  const int ws = B.ws;
  const int64_t numel[32] = {P_t + 1, S_t + 1, S_t * 8, TV, P_t, P_t, S_t * 2, Pc + 1, Pc, Pc, Ec, Ec,
                             Ps + 1, Ps, Ps, Es, Es, G * 4, G * ws, G * ws * 2, G * ws * 2, G, (int64_t)W + 1,
                             T, T, T * 16, T * 64, T * 8, (int64_t)W + 1, 0, 0, 0};
  const size_t esz[32] = {4, 4, 4, 4, 4, 4, 8, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 1, 4, 1, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4, 4};
  // (the spill count is known after the group pass: the spill list gets an allocation of its own)
  size_t need3 = 0;
  for (int i = 0; i < 29; ++i) need3 += (((size_t)std::max<int64_t>(numel[i], 1) * esz[i]) + 255) & ~size_t(255);
  need3 += bytes_of<int32_t>(rows + 1) + bytes_of<int32_t>(nnz) + bytes_of<float>(nnz);
  if (hipMalloc(&F->mem, need3) != hipSuccess) {
    (void)hipGetLastError();
    delete F;
    return fail(TRS_ENOMEM, "trs_build_online_device: hipMalloc of " + std::to_string(need3) + " bytes failed");
  }
  Arena A3{static_cast<char*>(F->mem), 0, need3};
  for (int i = 0; i < 29; ++i) {
    A3.used = (A3.used + 255) & ~size_t(255);
    F->slot[i].ptr = A3.base + A3.used;
    F->slot[i].numel = numel[i];
    A3.used += (size_t)std::max<int64_t>(numel[i], 1) * esz[i];
  }
  F->csr_rowptr = A3.take<int32_t>(rows + 1);
  F->csr_col = A3.take<int32_t>(nnz);
  F->csr_val = A3.take<float>(nnz);
  Out O;
  O.t_rowoff = (int32_t*)F->slot[0].ptr;
  O.t_blockoff = (int32_t*)F->slot[1].ptr;
  O.t_col = (int32_t*)F->slot[2].ptr;
  O.t_val = (float*)F->slot[3].ptr;
  O.t_winrow = (int32_t*)F->slot[4].ptr;
  O.t_atomic = (int32_t*)F->slot[5].ptr;
  O.t_bin = (int64_t*)F->slot[6].ptr;
  O.c_off = (int32_t*)F->slot[7].ptr;
  O.c_row = (int32_t*)F->slot[8].ptr;
  O.c_atomic = (int32_t*)F->slot[9].ptr;
  O.c_col = (int32_t*)F->slot[10].ptr;
  O.c_val = (float*)F->slot[11].ptr;
  O.cs_off = (int32_t*)F->slot[12].ptr;
  O.cs_row = (int32_t*)F->slot[13].ptr;
  O.cs_atomic = (int32_t*)F->slot[14].ptr;
  O.cs_col = (int32_t*)F->slot[15].ptr;
  O.cs_val = (float*)F->slot[16].ptr;
  O.s_col = (int32_t*)F->slot[17].ptr;
  O.s_mask = (uint8_t*)F->slot[18].ptr;
  O.s_val = (float*)F->slot[19].ptr;
  O.s_pos = (int8_t*)F->slot[20].ptr;
  O.s_win = (int32_t*)F->slot[21].ptr;
  O.s_offsets = (int32_t*)F->slot[22].ptr;
  O.tile_win = (int32_t*)F->slot[23].ptr;
  O.tile_group = (int32_t*)F->slot[24].ptr;
  O.tile_cols = (int32_t*)F->slot[25].ptr;
  O.packed_a = (int32_t*)F->slot[26].ptr;
  O.packed_meta = (int32_t*)F->slot[27].ptr;
  O.win_tile_off = (int32_t*)F->slot[28].ptr;
  auto fail_f = [&](int code, const std::string& m) {
    delete F;
    return fail(code, m);
  };
  if (hipMemcpyAsync(F->csr_rowptr, rowptr, (size_t)(rows + 1) * 4, hipMemcpyDeviceToDevice, s) != hipSuccess ||
      (nnz > 0 && (hipMemcpyAsync(F->csr_col, col, (size_t)nnz * 4, hipMemcpyDeviceToDevice, s) != hipSuccess ||
                   hipMemcpyAsync(F->csr_val, val, (size_t)nnz * 4, hipMemcpyDeviceToDevice, s) != hipSuccess)))
    return fail_f(TRS_EDEVICE, "trs_build_online_device: copy of the input CSR failed");
  hipLaunchKernelGGL(k_fill_windows, dim3(grid_of((int64_t)W + 1)), dim3(256), 0, s, B, O);
  // t_blockNew_offset: prefix sums of the sub-blocks' value counts (B.ord is free after stage B
  // and holds U >= S_t ints)
  if (S_t > 0) hipLaunchKernelGGL(k_tc_counts, dim3(grid_of(S_t)), dim3(256), 0, s, B, (int32_t)S_t, B.ord);
  if (scan(B.ord, S_t, O.t_blockoff, bsum2, s) != hipSuccess) return fail_f(TRS_EDEVICE, "scan failed");
  if (S_t > 0) hipLaunchKernelGGL(k_fill_tc, dim3(grid_of(S_t)), dim3(256), 0, s, B, O, (int32_t)S_t);
  if (G > 0) {
    hipLaunchKernelGGL(k_group_windows, dim3(grid_of(G)), dim3(256), 0, s, B, O, (int32_t)G);
    hipLaunchKernelGGL(k_fill_groups, dim3(grid_of(G * ws)), dim3(256), 0, s, B, O, G * ws);
  }
  if (T > 0) hipLaunchKernelGGL(k_fill_tiles, dim3(grid_of(T)), dim3(256), 0, s, B, O, (int32_t)T);
  hipLaunchKernelGGL(k_fill_residual, dim3(grid_of(std::max(rows, 1))), dim3(256), 0, s, B, O);
  if (scan(B.spill, nnz, B.spill_at, bsum2, s) != hipSuccess) return fail_f(TRS_EDEVICE, "scan failed");
  int32_t nsp = 0;
  if (hipMemcpyAsync(&nsp, B.spill_at + nnz, 4, hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return fail_f(TRS_EDEVICE, std::string("trs_build_online_device: ") + hipGetErrorString(hipGetLastError()));
  DevBuf sp;
  const size_t need4 = bytes_of<int32_t>(nsp) * 2 + bytes_of<float>(nsp);
  if (hipMalloc(&sp.p, need4) != hipSuccess) {
    (void)hipGetLastError();
    return fail_f(TRS_ENOMEM, "trs_build_online_device: hipMalloc of the spill list failed");
  }
  Arena A4{static_cast<char*>(sp.p), 0, need4};
  O.spill_row = A4.take<int32_t>(nsp);
  O.spill_col = A4.take<int32_t>(nsp);
  O.spill_val = A4.take<float>(nsp);
  if (nnz > 0) hipLaunchKernelGGL(k_fill_spill, dim3(grid_of(nnz)), dim3(256), 0, s, B, O);
  if (hipStreamSynchronize(s) != hipSuccess || hipGetLastError() != hipSuccess)
    return fail_f(TRS_EDEVICE, "trs_build_online_device: kernel failed");
  // the spill list lives in its own allocation, owned through slot pointers kept below
  F->slot[29] = {O.spill_row, nsp};
  F->slot[30] = {O.spill_col, nsp};
  F->slot[31] = {O.spill_val, nsp};
  F->spill_mem = sp.p;
  sp.p = nullptr;
  F->elapsed = std::chrono::duration<double>(std::chrono::high_resolution_clock::now() - t0).count();
  *out = F;
  return TRS_OK;
}


int trs_dformat_slot(const trs_dformat* f, int32_t slot, const void** data, int64_t* numel) {
  if (!f || !data || !numel) return fail(TRS_EINVAL, "trs_dformat_slot: NULL argument");
  if (slot < 0 || slot > 31) return fail(TRS_EINVAL, "trs_dformat_slot: slot out of range 0..31");
  *data = f->slot[slot].ptr;
  *numel = f->slot[slot].numel;
  return TRS_OK;
}

double trs_dformat_elapsed(const trs_dformat* f) { return f ? f->elapsed : 0.0; }
int32_t trs_dformat_rows(const trs_dformat* f) { return f ? f->rows : 0; }
int32_t trs_dformat_window(const trs_dformat* f) { return f ? f->window : 0; }
void trs_dformat_free(trs_dformat* f) { delete f; }

int trs_dformat_download(const trs_dformat* f, trs_format** out) {
  if (!f || !out) return fail(TRS_EINVAL, "trs_dformat_download: NULL argument");
  *out = nullptr;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess || cur != f->device)
    return fail(TRS_EINVAL, "trs_dformat_download: the format lives on device " + std::to_string(f->device) +
                                ", the current device is " + std::to_string(cur));
  auto* H = new trs_format();
  H->rows = f->rows;
  H->window = f->window;
  H->canonical = true;
  H->elapsed = f->elapsed;
  bool ok = true;
  auto get = [&](auto& vec, int slot) {
    using T = typename std::decay_t<decltype(vec)>::value_type;
    vec.resize((size_t)f->slot[slot].numel);
    if (!vec.empty() && hipMemcpy(vec.data(), f->slot[slot].ptr, vec.size() * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
      ok = false;
  };
  try {
    get(H->t_rowoff, 0); get(H->t_blockoff, 1); get(H->t_col, 2); get(H->t_val, 3); get(H->t_winrow, 4);
    get(H->t_atomic, 5); get(H->t_bin, 6); get(H->c_off, 7); get(H->c_row, 8); get(H->c_atomic, 9);
    get(H->c_col, 10); get(H->c_val, 11); get(H->cs_off, 12); get(H->cs_row, 13); get(H->cs_atomic, 14);
    get(H->cs_col, 15); get(H->cs_val, 16); get(H->s_col, 17); get(H->s_mask, 18); get(H->s_val, 19);
    get(H->s_pos, 20); get(H->s_win, 21); get(H->s_offsets, 22); get(H->tile_win, 23); get(H->tile_group, 24);
    get(H->tile_cols, 25); get(H->packed_a, 26); get(H->packed_meta, 27); get(H->win_tile_off, 28);
    get(H->spill_row, 29); get(H->spill_col, 30); get(H->spill_val, 31);
    H->csr_rowptr.resize((size_t)f->rows + 1);
    H->csr_col.resize((size_t)f->nnz);
    H->csr_val.resize((size_t)f->nnz);
    if (hipMemcpy(H->csr_rowptr.data(), f->csr_rowptr, H->csr_rowptr.size() * 4, hipMemcpyDeviceToHost) != hipSuccess ||
        (f->nnz > 0 && (hipMemcpy(H->csr_col.data(), f->csr_col, (size_t)f->nnz * 4, hipMemcpyDeviceToHost) != hipSuccess ||
                        hipMemcpy(H->csr_val.data(), f->csr_val, (size_t)f->nnz * 4, hipMemcpyDeviceToHost) != hipSuccess)))
      ok = false;
  } catch (const std::bad_alloc&) {
    delete H;
    return fail(TRS_ENOMEM, "trs_dformat_download: out of host memory");
  }
  if (!ok) {
    delete H;
    (void)hipGetLastError();
    return fail(TRS_EDEVICE, "trs_dformat_download: device-to-host copy failed");
  }
  *out = H;
  return TRS_OK;
}

}  // extern "C"
