// Device kernels of the hybrid SpMM / SDDMM path (gfx950) and their launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace trs {

// Residual task: rows [row_begin, row_end) with their entries [nz_begin, nz_end), or, when
// row_end < 0, a piece [nz_begin, nz_end) of row `row_begin` whose sum goes to partial slot
// ~row_end (a split row, finished by the fixup kernel).
struct Task { int32_t row_begin, row_end, nz_begin, nz_end; };

// A split row: C[row] = sum of partial slots slot_list[slot_begin .. slot_begin + slots) in order.
struct Fixup { int32_t row, slot_begin, slots, pad; };

// Rows per multi-row residual task (the task kernel preloads their row pointers into LDS).
constexpr int kTaskRows = 32;
// Split rows with more slots than this are summed by one workgroup each.
// (A Fixup's slot_begin indexes DevicePlan::slot_list, which names the row's partial slots in
// summation order.)
constexpr int kWideFixupSlots = 16;

// XCDs of an MI355X: workgroup i of a launch runs on XCD i mod kXcds (each XCD has its own L2).
constexpr int kXcds = 8;
// XCD whose L2 serves column c's B row in the SpMM column split: a multiplicative hash spreads hot
// and cold columns evenly over the XCDs.
__host__ __device__ inline int xcd_of_column(int32_t c) { return (int)(((uint32_t)c * 2654435761u) >> 29); }

// SDDMM split rows, merged: out[e] = xbuf[x_src[k_begin + e - e_begin]] for e in [e_begin, e_end),
// at most kMergeTaskEntries indices per task (a multiple of 256).
struct MergeTask { int32_t e_begin, e_end, k_begin, pad; };
constexpr int32_t kMergeTaskEntries = 4096;

// A window handled by the MFMA window kernel: 16 output rows starting at row0 (rows >= m are
// dropped), dense 16x16 fp16 tiles [tile_begin, tile_end), plus that window's residual rows.
struct MfmaWindow { int32_t row0, tile_begin, tile_end, pad; };

struct DevicePlan {
  int32_t m = 0, n = 0;
  int64_t nnz_csr = 0;
  const int32_t* rowptr = nullptr;   // [m + 1] residual CSR (fp16 values)
  const int32_t* col = nullptr;
  const uint16_t* val = nullptr;
  const Task* tasks = nullptr;
  int32_t ntasks = 0;
  const Fixup* fixups = nullptr;      // split rows with <= kWideFixupSlots slots
  int32_t nfixups = 0;
  const Fixup* wfixups = nullptr;     // split rows with more slots
  int32_t nwfixups = 0;
  int32_t partial_slots = 0;
  const MfmaWindow* mwin = nullptr;
  int32_t nmwin = 0;
  const int32_t* tile_cols = nullptr;  // [tiles][16]
  const uint16_t* tile_a = nullptr;    // [tiles][16 rows][16 cols] fp16 (SpMM)
  int32_t ntiles = 0;
  // SpMM 2:4 quads (sptc_sparse): window i owns quads [win_quad[i], win_quad[i + 1]); quad q covers
  // four 16-column tiles, tile b as columns 16 b .. 16 b + 15 (quad_cols[q][64], -1 = none); lane l
  // of v_smfmac_f32_16x16x64_f16 holds row l % 16 of tile l / 16: quad_a[q][l][8] fp16, two values
  // per group of 4 columns, at the 2-bit column positions packed in quad_idx[q][l] (value j at
  // bits 2j .. 2j + 1).
  const int32_t* win_quad = nullptr;
  const int32_t* quad_cols = nullptr;
  const uint16_t* quad_a = nullptr;
  const uint16_t* quad_idx = nullptr;
  int32_t nquads = 0;
  // SDDMM plans: output index of each residual entry (null = identity; see res_off) and, per tile, its first
  // row and the output index of each of its 256 (row, column) slots (-1 = not stored)
  const int32_t* res_pos = nullptr;
  const int32_t* tile_row0 = nullptr;
  const int32_t* tile_pos = nullptr;
  int32_t feature_lanes = 0;   // lanes per residual lane group (0 = automatic)
  int32_t streaming = 0;       // bit 0: non-temporal A-stream loads, bit 1: non-temporal C stores
  int32_t xcd_run = 1;         // consecutive workgroups per XCD run (1 = hardware round robin)
  int32_t stage = 0;           // staged task streams: 0 automatic, -1 never
  int32_t occupancy = 0;       // waves per SIMD for the residual task kernel: 2..8, 0 automatic, -1 uncapped
  int32_t sddmm_unroll = 0;    // SDDMM residual entries in flight per lane group (4, 8; 0 automatic)
  int32_t split_dispatch = 0;  // 1: main part and XCD split part as two launches (profiling)
  int32_t task_nnz = 0;        // entries per packed residual task
  int32_t task_max = 0;        // most entries of any residual task (packed rows or a piece)
  const int32_t* slot_list = nullptr;   // partial slots of the split rows, in summation order
  // XCD column split: sub-rows (pieces of long rows by column range, laid out range-major in
  // col / val after the main part) with their own tasks, queue x = x_tasks [xq[x], xq[x + 1]) for
  // XCD x; SpMM sub-row j sums into partial slot j
  const Task* x_tasks = nullptr;
  int32_t x_ntasks = 0;
  int32_t x_task_max = 0;
  const int32_t* x_rowptr = nullptr;
  const int32_t* x_pos = nullptr;       // SDDMM: output index of the split part's entries
  const int32_t* x_sub_row = nullptr;   // SDDMM: the row of sub-row j
  // SDDMM plans with a split part also keep the unsplit task list of all rows, used below
  // kSddmmSplitMinK
  const Task* full_tasks = nullptr;
  int32_t nfull_tasks = 0;
  const Task* narrow_tasks = nullptr;  // SDDMM: the unsplit layout in pieces of S entries, for lane
  int32_t nnarrow_tasks = 0;           // groups of <= 8 lanes (none where no row is longer than S)
  int32_t xq[kXcds + 1] = {};
  // set in the view the launcher builds for the split part (see split_view): tasks come from the
  // per-XCD queues, workgroup i taking queue i mod kXcds; rows are sub-rows
  int32_t xcd_queues = 0;
  const int32_t* sub_row = nullptr;
  int32_t res_off = 0;   // res_pos[q - res_off] is entry q's output index
  // Staged hot rows: hot_col is col with every entry of the nhot most used columns renumbered
  // ~rank (rank 0 = most used), hot_rows[rank] that column.  A call copies those B (Y) rows into a
  // dense buffer and the task kernels then read hot_col, gathering a negative id ~rank from the
  // buffer (hot_b, leading dimension hot_ld: set in the launch view only).
  const int32_t* hot_col = nullptr;
  const int32_t* hot_rows = nullptr;
  int32_t nhot = 0;
  const uint16_t* hot_b = nullptr;
  int32_t hot_ld = 0;
  // SDDMM split part written in its own order: with a buffer from the workspace, sub-row entry q
  // (of the x_entries after the main part) writes xbuf[q - nnz_csr], and a merge pass puts the
  // split rows' outputs in place: merge task i covers output indices [e_begin, e_end), whose
  // values sit at xbuf[x_src[k]] (k counts the split rows' entries in output order)
  const int32_t* x_src = nullptr;
  const MergeTask* merge = nullptr;
  int32_t nmerge = 0;
  int64_t x_entries = 0;
  int32_t out_off = 0;   // set in the view that writes xbuf: entry q writes out[q - out_off]
};

// Hot-row staging applies to 16-byte gathers of at least this many features (one 16-lane group,
// 256-byte rows: R-MAT 2^20 K = 128 -6%, K = 256 -5%; K = 32 and 64 unchanged or slower).
constexpr int kHotMinK = 128;
// The SDDMM split part writes its own buffer (then merged) from this width on.
constexpr int kSddmmMergeMinK = 128;
// Bytes of that buffer for plan p at width K (0: the plan has no split part, or K is narrower).
inline int64_t merge_buffer_bytes(const DevicePlan& p, int K) {
  return p.nmerge > 0 && K >= kSddmmMergeMinK ? p.x_entries * 4 : 0;
}
// Bytes of the staged-row buffer of plan p at width K (0 when the plan or K does not stage).
inline int64_t hot_buffer_bytes(const DevicePlan& p, int K) {
  if (p.nhot <= 0 || K < kHotMinK || K % 8 != 0) return 0;
  return (int64_t)p.nhot * K * 2;
}
// Column histogram of col[0, total) into counts[n] (ids outside [0, n) are skipped), counted in
// `copies` histograms counts[k * n .. (k + 1) * n) (all zeroed by the caller) and summed into the
// first; and the renumbering hot_col[e] = rank[col[e]] >= 0 ? ~rank[col[e]] : col[e].
hipError_t launch_count_columns(const int32_t* col, int64_t total, int32_t n, int32_t* counts, int copies,
                                hipStream_t stream);
hipError_t launch_renumber_hot(const int32_t* col, int64_t total, int32_t n, const int32_t* rank, int32_t* hot_col,
                               hipStream_t stream);
// counts[col[e]] -= 1 for the residual entries e of the nmwin MFMA windows' rows (rowptr [m + 1]):
// the window kernel reads those through the plain ids, so they do not count towards staging.
hipError_t launch_uncount_windows(const MfmaWindow* mwin, int32_t nmwin, int32_t m, const int32_t* rowptr,
                                  const int32_t* col, int32_t n, int32_t* counts, hipStream_t stream);

// SDDMM runs a plan's split part from this feature width on (narrower rows measured faster
// unsplit).
constexpr int kSddmmSplitMinK = 128;

// Device-side plan lowering (the residual of a plan built from the input CSR the format keeps).
// A dense tile's stored entries: rows row0 + r (r < 16), columns cols[k]; bit (r % 4) * 16 + k of
// present[r / 4] marks entry (r, k).
struct TileEntries { int32_t row0; int32_t cols[16]; int32_t pad[3]; uint64_t present[4]; };
// Byte e of the flag words (little-endian) = 1 for every CSR entry e (rows < m, columns ascending)
// that a tile stores; *marked (zeroed by the caller) counts the entries flagged, each once.
// tile_pos (optional, SDDMM): tile_pos[t * 256 + r * 16 + k] = CSR index of stored entry (r, k).
hipError_t launch_mark_tile_entries(const TileEntries* tiles, int32_t ntiles, int32_t m, const int32_t* rowptr,
                                    const int32_t* col, uint32_t* flag_words, uint32_t* marked, int32_t* tile_pos,
                                    hipStream_t stream);
// Entries of CSR rows [0, m) into the plan's entry arrays.  Row r with split_index[r] = i >= 0 is
// scattered by the XCD of each column to cursor[i * kXcds + x] onward (column order kept), with
// x_pos[position - x_base] = CSR index when x_pos is set; compact (SpMM) plans store such a row
// only there.  Every other row -- and in a non-compact (SDDMM) plan every row -- goes, without its
// flagged entries (flag may be null), to main_rowptr[r] onward, with res_pos[position] = CSR index
// when res_pos is set.  Values (val_out set) are rounded to fp16.
struct PlaceEntries {
  int32_t m = 0;
  const int32_t* rowptr = nullptr;
  const int32_t* col = nullptr;
  const float* val = nullptr;
  const uint8_t* flag = nullptr;
  const int32_t* main_rowptr = nullptr;
  const int32_t* split_index = nullptr;
  const int32_t* cursor = nullptr;
  int32_t* col_out = nullptr;
  uint16_t* val_out = nullptr;
  int32_t* res_pos = nullptr;
  int32_t* x_pos = nullptr;
  int64_t x_base = 0;
  int32_t compact = 1;
  // SDDMM: x_src[merge_off[split_index] + offset in the row] = position - x_base (when x_src set)
  const int32_t* merge_off = nullptr;
  int32_t* x_src = nullptr;
};
hipError_t launch_place_entries(const PlaceEntries& a, hipStream_t stream);

// Plans from a device-resident format (trs_dformat): what the host lowering reads of the input
// CSR's columns, computed where they are.
// *first_bad (the caller sets it to ~0ull) = the lowest index e with col[e] outside [0, n).
hipError_t launch_check_columns(const int32_t* col, int64_t total, int32_t n, unsigned long long* first_bad,
                                hipStream_t stream);
// Chunk i of the split-row candidates, entries col[start[i] .. start[i] + len[i]) of candidate
// row[i]: cnt[row[i] * kXcds + x] += its entries of XCD class x (xcd_of_column; cnt zeroed by the
// caller); with seen (n bytes, zeroed by the caller, 4-byte padded) seen[c] = 1 for its columns.
hipError_t launch_split_stats(const int32_t* col, const int32_t* start, const int32_t* len, const int32_t* row,
                              int32_t chunks, int32_t* cnt, uint8_t* seen, hipStream_t stream);
// *out += the nonzero bytes of flags[0, n) (values 0 or 1, n padded to 4 bytes; *out zeroed by
// the caller).
hipError_t launch_count_flags(const uint8_t* flags, int64_t n, unsigned long long* out, hipStream_t stream);
// 2:4 group tiles of a window-16 format (tiles of four groups per window, block_online.cpp:796-841):
// pass[t] = 1 when the stored values of tile t's groups (s_pos >= 0, 32 per group) are at least
// min_fill * 256, the fill rule of the host lowering.
hipError_t launch_group_tile_fill(const int32_t* tile_win, const int32_t* tile_group, const int32_t* s_offsets,
                                  const int8_t* s_pos, int32_t ntiles, float min_fill, uint8_t* pass,
                                  hipStream_t stream);
// The groups of the listed tiles, packed: GroupTile i holds tile ids[i]'s window row, group count,
// s_columns, s_values and s_pos (window 16).
struct GroupTile { int32_t row0, ngroups; int32_t cols[16]; float val[4][32]; int8_t pos[4][32]; };
hipError_t launch_gather_group_tiles(const int32_t* ids, int32_t nids, const int32_t* tile_win,
                                     const int32_t* tile_group, const int32_t* s_offsets, const int32_t* s_col,
                                     const float* s_val, const int8_t* s_pos, GroupTile* out, hipStream_t stream);

// hot: the staged-row buffer (hot_buffer_bytes(p, K) bytes; null = gather every row from B).
// ev (optional): 4 events recorded before the task kernel (and the hot-row copy) and after each of
// the three kernels.
hipError_t launch_spmm(const DevicePlan& p, const uint16_t* B, int64_t ldb, int K, float* C, int64_t ldc,
                       float* partial, uint16_t* hot, hipStream_t stream, hipEvent_t* ev = nullptr);
// out[0, n) = 0 with a kernel (not a memset node: callers may capture the stream in a graph).
hipError_t launch_zero_fill(float* out, int64_t n, hipStream_t stream);
// hot: as for launch_spmm, Y rows.  xbuf: the split part's own output buffer
// (merge_buffer_bytes(p, K) bytes; null = the split part writes its outputs in place).  ev
// (optional): 3 events recorded before the residual kernels (and the hot-row copy) and after them
// (and the merge), and after the tile kernel.
hipError_t launch_sddmm(const DevicePlan& p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy,
                        int K, float* out, uint16_t* hot, float* xbuf, hipStream_t stream,
                        hipEvent_t* ev = nullptr);

}  // namespace trs
