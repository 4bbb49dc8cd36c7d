/* trspmm.h -- C ABI of the MI355X (gfx950) hybrid fp16 SpMM / SDDMM library (libtrspmm.so).
 *
 * Plain pointers and sizes only; no exceptions cross this boundary.  Every function returns a
 * trs_status; on failure trs_last_error() describes the problem (thread-local).
 *
 * Object model
 *   trs_format  host-side output of the format builder (the reference's 29-array tuple + spill).
 *   trs_plan    device-resident, immutable execution plan.  Plans may be shared between threads;
 *               calls on the same plan may run concurrently on different streams as long as each
 *               call gets its own output buffer and workspace.
 * Device pointers (B, C, X, Y, out, workspace) are caller-owned HIP device memory; `stream` is a
 * hipStream_t (NULL = the default stream).  fp16 data is passed as uint16_t bit patterns.
 *
 * Versioning
 *   Parameter structs (trs_build_params, trs_reorder_params, trs_plan_options) start with
 *   `struct_size`, which their *_default initialiser sets to sizeof the struct of this header.
 *   Every entry point that reads such a struct refuses a struct_size other than the library's
 *   with TRS_EINVAL, before it reads anything past that first field, so a caller compiled against
 *   another version of this header (whose struct may be shorter) gets an error, never a read past
 *   its struct.  Always fill these structs with the *_default function of the header you compile
 *   against, then change fields.  trs_plan_stats_get takes the size of the caller's stats struct
 *   and refuses other sizes the same way.  TRSPMM_ABI_VERSION is the version of this header;
 *   trs_abi_version() returns the library's.
 */
#ifndef TRSPMM_H
#define TRSPMM_H

#include <stdint.h>

/* 1: first release; 2: plan options xcd_split .. hot_rows, reorder minhash, wider plan stats;
 * 3: struct_size fields and the stats size argument; 4: the GPU format builder
 * (trs_build_online_device, trs_dformat_*) and plans from its output (trs_plan_create_dformat,
 * trs_plan_create_sddmm_dformat); struct layouts as in 3. */
#define TRSPMM_ABI_VERSION 4

#ifdef __cplusplus
extern "C" {
#endif

typedef enum trs_status {
  TRS_OK = 0,
  TRS_EINVAL = 1,     /* bad argument: shape, dtype-size, range (reference: TORCH_CHECK -> RuntimeError) */
  TRS_ENOMEM = 2,     /* host or device allocation failed */
  TRS_EDEVICE = 3,    /* HIP runtime error (no GPU, launch failure, ...) */
  TRS_ENOTCANON = 4,  /* CSR rows not strictly increasing: a plan cannot be built from it */
  TRS_ERANGE = 5,     /* index outside [0, rows) / [0, cols), or size beyond int32 addressing */
  TRS_EIO = 6         /* format file cannot be opened / written, or is not a valid format file */
} trs_status;

/* ---------------------------------------------------------------------------------------------
 * Format builder.
 * Replaces Libra5BlockOnline.block_sptc_2to4_online
 * (TR-source/Block/block_online.cpp:545-549 signature, :844-870 return list).
 * ------------------------------------------------------------------------------------------- */
typedef struct trs_build_params {
  int32_t struct_size;       /* sizeof(trs_build_params), set by trs_build_params_default */
  int32_t part_size_t;       /* partSize_t: TC sub-blocks per part (32) */
  int32_t part_size_c;       /* partSize_c: residual nnz per long part (32) */
  int32_t short_size;        /* shortSize: residual rows with <= this nnz form short parts (3) */
  int32_t density;           /* TC column threshold: nnz of a column inside a window (8) */
  int32_t window;            /* rows per window, 1..32 (16) */
  int32_t wide;              /* accepted and range-checked (1..32) only, as in the reference (16) */
  float tc_min_util;         /* minimum fill of a 16x8 TC chunk (0.0) */
  float sptc_min_util;       /* accepted, unused -- as in the reference (0.5) */
  int32_t sptc_threshold;    /* accepted, unused -- as in the reference (12) */
  int32_t skip_tc;           /* -1: read env LIBRA_SKIP_TC like the reference; 0 / 1 explicit */
  int32_t sptc_unit_min_nnz; /* -1: read env LIBRA_SPTC_UNIT_MIN_NNZ (default 2); >= 0 explicit */
  int32_t num_threads;       /* host threads; 0 = OpenMP default */
} trs_build_params;

void trs_build_params_default(trs_build_params* p);

typedef struct trs_format trs_format;

/* rowptr[rows+1], col[nnz], val[nnz] (float32) on the host.  Output arrays are bit-exact with the
 * reference builder for any input; the spill list (slots 29-31) holds the entries the reference
 * drops, so that tuple + spill reproduces the input exactly. */
int trs_build_online(const int32_t* rowptr, const int32_t* col, const float* val, int32_t rows,
                     int64_t nnz, const trs_build_params* params, trs_format** out);

/* Slot 0..28: reference tuple order (t_rowkNew_offset ... s_window_tile_offset);
 * slot 29/30/31: spill rows (int32) / columns (int32) / values (float32).
 * Element types per slot: int32 except 3, 11, 16, 19, 31 (float32), 6 (int64), 18 (uint8),
 * 20 (int8).  The data pointer stays valid until trs_format_free. */
int trs_format_slot(const trs_format* f, int32_t slot, const void** data, int64_t* numel);
double trs_format_elapsed(const trs_format* f);  /* reference slot 29: build wall time, s */
int32_t trs_format_window(const trs_format* f);
int32_t trs_format_rows(const trs_format* f);
int32_t trs_format_canonical(const trs_format* f); /* 1 if every row had increasing columns */
void trs_format_free(trs_format* f);

/* Format builder on the GPU.  No reference counterpart: it builds what
 * Libra5BlockOnline.block_sptc_2to4_online returns (the reference builds on one CPU thread,
 * TR-source/Block/block_online.cpp:545-871) from a CSR in device memory (rowptr[rows + 1], col[nnz],
 * val[nnz] float32, on the current device) into device memory, on `stream` (NULL: the default
 * stream); the call returns when the format is complete.  The 32 slots are bit-exact with
 * trs_build_online's on the same input and parameters.  Canonical input only (strictly increasing
 * columns in every row: TRS_ENOTCANON otherwise) and windows of at most 16 rows (TRS_EINVAL
 * otherwise); trs_build_online builds every other input.  The result keeps its own copy of the
 * input CSR, so the caller's buffers may be freed after the call. */
typedef struct trs_dformat trs_dformat;
int trs_build_online_device(const int32_t* rowptr, const int32_t* col, const float* val, int32_t rows,
                            int64_t nnz, const trs_build_params* params, void* stream, trs_dformat** out);
/* Device pointer and element count of slot 0..31 (element types as for trs_format_slot). */
int trs_dformat_slot(const trs_dformat* f, int32_t slot, const void** data, int64_t* numel);
/* A host trs_format with the same 32 slots (and the input CSR, for device plan lowering). */
int trs_dformat_download(const trs_dformat* f, trs_format** out);
double trs_dformat_elapsed(const trs_dformat* f);   /* build wall time, s */
int32_t trs_dformat_rows(const trs_dformat* f);
int32_t trs_dformat_window(const trs_dformat* f);
void trs_dformat_free(trs_dformat* f);

/* Format cache.  No counterpart in the reference, which rebuilds the format on every run
 * (spmm/tr_csr_fp16/mdataset2_online.py:100-113); for callers that reuse a graph across runs.
 * One versioned little-endian file holds all 32 slots, rows, window, the canonical flag and the
 * build time, with a 64-bit checksum.  trs_format_write writes to "<path>.tmp" and renames, so a
 * reader never sees a partial file; trs_format_read refuses truncated, corrupted or other-version
 * files with TRS_EIO.  A read format is used exactly like a built one. */
int trs_format_write(const trs_format* f, const char* path);
int trs_format_read(const char* path, trs_format** out);

/* ---------------------------------------------------------------------------------------------
 * Row reorder.
 * Replaces apply_tca_reorder (spmm/tr_csr_fp16/tr_tca_reorder.py:44-357), which the reference
 * dataset layer runs before the builder when LIBRA_TCA_REORDER=1 (mdataset2_online.py:72-95):
 * rows with similar column sets are clustered (MinHash-LSH candidate pairs scored by exact
 * Jaccard, greedy union-find merging in order of similarity, clusters closing at `thres` rows;
 * then the clusters' column unions clustered the same way up to `cluster_thres` clusters) and
 * laid out cluster by cluster.  Deterministic for given parameters and thread-count independent.
 * ------------------------------------------------------------------------------------------- */
typedef struct trs_reorder_params {
  int32_t struct_size;    /* sizeof(trs_reorder_params), set by trs_reorder_params_default */
  int32_t thres;          /* rows at which a level-1 cluster closes (16) */
  int32_t cluster_thres;  /* level-1 clusters at which a level-2 group closes (128) */
  int32_t num_perm;       /* MinHash permutations (128); LSH bands x rows per band are chosen
                             for lsh_threshold like the reference's LSH library does */
  float lsh_threshold;    /* Jaccard similarity the LSH banding targets (0.2) */
  int32_t bucket_span;    /* LSH buckets larger than bucket_span + 1 pair each member with the
                             next bucket_span members only (64); <= 0: every pair, as the
                             reference */
  int32_t num_threads;    /* host threads; 0 = OpenMP default */
  int32_t exhaustive;     /* 1: every pair of non-empty sets is a candidate (small inputs, tests) */
  int32_t align_window;   /* 0: the reference's layout.  W > 0 (no reference counterpart): level-1
                             clusters never exceed W rows (thres is ignored) and are packed
                             first-fit decreasing into whole W-row windows per level-2 group, so
                             clusters do not straddle windows */
  uint64_t seed;          /* MinHash permutation seed (1, the reference LSH library's default) */
  int32_t minhash;        /* MinHash family: 1 = the reference's LSH library (datasketch: SHA-1 of
                             the decimal string, permutations (a x + b) mod 2^61 - 1 drawn by
                             numpy's legacy RandomState(seed)) (default); 0 = a 64-bit mixing hash */
} trs_reorder_params;

void trs_reorder_params_default(trs_reorder_params* p);

/* rowptr[rows+1], col[nnz] on the host, columns in [0, ncols).  order[new_row] = old_row, a
 * permutation of [0, rows). */
int trs_tca_reorder(const int32_t* rowptr, const int32_t* col, int32_t rows, int64_t nnz, int32_t ncols,
                    const trs_reorder_params* params, int32_t* order);

/* The reorder's LSH pieces, for tests and diagnostics (no reference counterpart; they expose what
 * the reference's LSH library computes inside tr_tca_reorder.py:84-90, :121-123).
 * trs_lsh_bands: the (bands, rows per band) minimising the equally weighted false-positive and
 * false-negative areas for `threshold` at num_perm permutations.
 * trs_minhash_signatures: sig[i * count + k] = the k-th MinHash value of set i (elements
 * elems[off[i] .. off[i + 1]), non-negative; empty sets 0xffffffff) in params' family and seed. */
int trs_lsh_bands(float threshold, int32_t num_perm, int32_t* bands, int32_t* rows);
int trs_minhash_signatures(const int64_t* off, const int32_t* elems, int32_t nsets,
                           const trs_reorder_params* params, int32_t count, uint32_t* sig);

/* ---------------------------------------------------------------------------------------------
 * Statistics-only 2:4 matching ("dual routing").
 * Replaces matching_utils.match_2to4 (TR-source/Block/block_matching_window_para_dr.cpp:361-451,
 * built by TR-source/setup_24matching.py:8-12): per window of window_size rows, columns carry a
 * 16-bit row mask; a sliding 1:2 pairing (32 positions, overlap <= t_max) and a 2:4 grouping of the
 * pairs (1024 positions, conflict-free masks) are counted, and the unmatched columns are routed to
 * dense TC blocks of dense_threshold columns or to padded 2:4 groups.  No format arrays: counts only.
 * Counters are 64-bit (the reference's 32-bit ones wrap on very large inputs); otherwise the totals
 * equal the reference's, including its mask of local rows >= 16 (a shift of 1 by local_row mod 32,
 * kept to 16 bits).
 * ------------------------------------------------------------------------------------------- */
typedef struct trs_match_stats {
  int64_t total_rows, total_cols, total_nnz;
  double sparsity;                 /* 1 - total_nnz / (total_rows * total_cols) */
  int64_t num_row_panels;          /* windows */
  int64_t num_sptc_groups;         /* 2:4 groups (matched and fallback) */
  int64_t num_tc_blocks;           /* dense blocks of dense_threshold columns */
  int64_t num_16x16_blocks;        /* groups rounded up to 4 per window */
  int64_t block_padding_groups;
  int64_t fine_fallback;           /* columns without a 1:2 partner */
  int64_t coarse_fallback;         /* columns of pairs without a 2:4 partner */
  int64_t fake_zeros;              /* padding slots of all groups */
  int64_t tc_total_nnz, tc_block_count, tc_block_max_nnz;
  int64_t tc_block_min_nnz;        /* 999999 when there is no TC block, as in the reference */
} trs_match_stats;

/* rowptr[rows+1], col[nnz] on the host (rows need not be sorted; duplicates count once);
 * total_cols = max(col) + 1.  TRS_EINVAL for window_size outside [1, 64], dense_threshold < 1,
 * rows <= 0 or no column (the reference's "invalid matrix dimensions"), or a rowptr that is not
 * monotone within [0, nnz]; TRS_ERANGE for a negative column.  num_threads 0 = OpenMP default;
 * the result does not depend on it. */
int trs_match_2to4(const int32_t* rowptr, const int32_t* col, int32_t rows, int64_t nnz, int32_t window_size,
                   int32_t dense_threshold, int32_t t_max, int32_t num_threads, trs_match_stats* out);

/* ---------------------------------------------------------------------------------------------
 * Plans.  A plan lowers format arrays to the device layout the kernels read (dense 16x16 fp16
 * MFMA tiles + an fp16 CSR residual with load-balanced row tasks), validates every index on the
 * host, and uploads once.  m = output rows (mOri), n = rows of the dense operand (kOri).
 * ------------------------------------------------------------------------------------------- */
typedef struct trs_plan trs_plan;

typedef struct trs_plan_options {
  int32_t struct_size;    /* sizeof(trs_plan_options), set by trs_plan_options_default */
  int32_t mfma_tc;        /* 1: TC sub-blocks run on MFMA tiles; 0: lowered to the CSR residual */
  int32_t mfma_sptc;      /* 1: 2:4 group tiles whose fill >= sptc_min_fill run on MFMA */
  float sptc_min_fill;    /* fill threshold (nnz / 256 slots of a 16x16 tile) for mfma_sptc */
  int32_t task_nnz;       /* residual nnz per lane-group task packing short rows (0 = automatic:
                             about four mean rows, 32..128, and smaller -- down to 16 -- where
                             that leaves fewer than 16,384 tasks) */
  int32_t piece_nnz;      /* longest residual run one lane group walks; longer rows are split
                             into pieces summed by the fixup kernel (0 = automatic: 256, or 64
                             where the automatic task size leaves fewer than 16,384 tasks) */
  int32_t feature_lanes;  /* lanes per lane group (power of two <= 64; each lane holds 8 features):
                             fewer lanes = several feature passes with a smaller B working set
                             per pass (0 = automatic) */
  int32_t streaming;      /* non-temporal hints, bit 0: A-stream loads, bit 1: C stores and
                             residual SDDMM outputs (keeps them from evicting gathered B / Y
                             rows); 0 plain; -1 automatic (bit 1) */
  int32_t window_row_cap; /* longest residual row an MFMA window may carry before its tiles go
                             back to the residual path, when that row is also more than twice
                             its window's mean residual row (0 = automatic: 128) */
  int32_t xcd_run;        /* workgroups are remapped so each of the 8 XCDs (own L2) runs this many
                             consecutive work items in a row; 1 = hardware round robin,
                             0 = automatic */
  int32_t sddmm_unroll;   /* SDDMM residual entries in flight per lane group: 4 or 8; 0 = automatic
                             (4 for passes of exactly 128 features with 16-byte loads, else 8) */
  int32_t stage;          /* a residual task's column ids (and values) are copied into LDS once
                             before its gathers: 0 = automatic (16-lane groups, i.e. K = 65..128,
                             and tasks of <= 256 entries), -1 = never */
  int32_t occupancy;      /* waves per SIMD the residual task kernels may hold (2..8; values
                             outside are clamped): fewer concurrent tasks keep fewer gathered rows
                             in flight.  0 = automatic (SpMM: 2 for K <= 64, uncapped above;
                             SDDMM: uncapped), -1 = uncapped (as many as registers and LDS allow) */
  int32_t xcd_split;      /* XCD column split: the columns are divided among the 8 XCDs by a hash
                             and residual rows with at least this many entries are cut into one
                             sub-row per XCD, run by that XCD's workgroups (workgroup i runs on XCD
                             i mod 8), so each XCD's L2 holds B (or Y) rows of an eighth of the
                             columns; an SpMM sub-row costs a partial slot, an SDDMM sub-row entry
                             an output index (SDDMM uses the split from K = 128 on).
                             0 = automatic (SpMM 256, SDDMM 512, and only when those rows read
                             their columns at least 4 times each on average: no L2 reuse to gain
                             otherwise), -1 = off */
  int32_t host_lowering;  /* trs_plan_create only.  0: when the format holds its input CSR (a format
                             built in this process from canonical input), the MFMA tiles are cut
                             from the format on the host and the residual (the input CSR minus the
                             kept tiles' entries, XCD sub-rows included) is built on the device;
                             the plan is the same as the host lowering's.  1: always on the host */
  int32_t sptc_sparse;    /* SpMM plans: 1 = MFMA tiles whose every row has at most 2 entries in
                             each group of 4 columns (the 2:4 group tiles, and TC tiles that happen
                             to be 2:4) run on gfx950's sparse v_smfmac_f32_16x16x64_f16, four tiles
                             (64 columns) per instruction, their values stored compressed with
                             2-bit column indices, as the reference runs its packed 2:4 tiles on
                             mma.sp (mGCNkernel_online.cu:812-933) (default); 0 = every tile on
                             the dense v_mfma_f32_16x16x16_f16 with zero fill */
  int32_t hot_rows;       /* staged hot rows: the B (Y) rows of the columns the residual task
                             kernels gather most are copied into a dense buffer at the start of a
                             call (workspace), and the task kernels read them there; the plan keeps
                             a second copy of its column ids with those columns renumbered.  Used
                             for K >= 128 (K % 8 == 0) on 16-byte aligned operands.  0 = automatic
                             (32768 rows, at most n / 16, and only when they take >= 30% of the
                             gathers), > 0 = that many rows, -1 = off.  Never for plans with more
                             than 4 columns per entry (n > 4 nnz) */
  int32_t split_dispatch; /* 0: the residual task kernels run the main part and the XCD split part
                             in one launch (default, faster); 1: as two launches, main part first,
                             so that a profiler attributes time and counters to each part */
} trs_plan_options;

void trs_plan_options_default(trs_plan_options* o);

/* Full-accuracy plan from the builder output: TC + 2:4 groups + residual + spill == input.
 * Replaces the device half of Libra6SpMMOnline.forward_fp16_tcu_cuda_sptc_mma_parallel_online
 * (TR-source/SpMM/mGCN_online.cpp:760-1138) for callers that keep the trs_format.  A format built
 * in this process from canonical input keeps its input CSR, and then the residual is built on the
 * device (opt->host_lowering; the plan is the same either way).  Synchronous: returns when the
 * plan is on the device. */
int trs_plan_create(const trs_format* f, int32_t m, int32_t n, const trs_plan_options* opt,
                    trs_plan** out);

/* Plan from the host arrays the reference parallel operator receives
 * (mGCN_online.cpp:760-800; t_value / c_value are fp16 bits, s_value float32, t_binary int64).
 * The result is the SpMM of exactly what those arrays carry (no spill).  spill_* may be NULL
 * (spill_count 0); when given, the plan also carries those entries. */
typedef struct trs_parallel_arrays {
  const int32_t* t_row_offset; int64_t n_t_row_offset;
  const int32_t* t_block_offset; int64_t n_t_block_offset;
  const int32_t* t_column; int64_t n_t_column;
  const uint16_t* t_value; int64_t n_t_value;
  const int32_t* t_window_row; int64_t n_t_window_row;
  const int32_t* t_atomic; int64_t n_t_atomic;
  const int64_t* t_binary; int64_t n_t_binary;
  const int32_t* c_row_offsets; int64_t n_c_row_offsets;
  const int32_t* c_row; int64_t n_c_row;
  const int32_t* c_atomic; int64_t n_c_atomic;
  const int32_t* c_column; int64_t n_c_column;
  const uint16_t* c_value; int64_t n_c_value;
  const int32_t* cs_row_offsets; int64_t n_cs_row_offsets;
  const int32_t* cs_row; int64_t n_cs_row;
  const int32_t* cs_atomic; int64_t n_cs_atomic;
  const int32_t* cs_column; int64_t n_cs_column;
  const uint16_t* cs_value; int64_t n_cs_value;
  const int32_t* s_column; const float* s_value; const int8_t* s_pos; int64_t groups;
  const int32_t* s_offsets; int64_t n_s_offsets;          /* windows + 1 */
  const int32_t* s_tile_column; const int32_t* s_packed_a; const int32_t* s_packed_meta;
  const int32_t* s_window_tile_offset; int64_t tiles; int64_t n_s_window_tile_offset;
  int32_t use_packed_tiles;  /* 1: 2:4 share from packed tiles (as the reference parallel kernel);
                                0: from s_column/s_value/s_pos */
  const int32_t* spill_row; const int32_t* spill_col; const float* spill_val; int64_t spill_count;
  int32_t parts_t, parts_c, partsize_c, parts_c_short, window, m, n;
} trs_parallel_arrays;

int trs_plan_create_parallel(const trs_parallel_arrays* a, const trs_plan_options* opt, trs_plan** out);

/* 2:4-group-only plans.
 * Replaces forward_fp16_sptc_online (s_window rows, mGCN_online.cpp:202-400) when s_window != NULL,
 * and forward_fp16_sptc_mma_online (window from s_offsets, mGCN_online.cpp:404-650) otherwise. */
int trs_plan_create_sptc(const int32_t* s_column, const float* s_value, const int8_t* s_pos,
                         int64_t groups, const int32_t* s_window, const int32_t* s_offsets,
                         int64_t n_s_offsets, int32_t window, int32_t m, int32_t n,
                         const trs_plan_options* opt, trs_plan** out);

/* Replaces forward_fp16_sptc_mma_packed_online (mGCN_online.cpp:654-757). */
int trs_plan_create_sptc_packed(const int32_t* s_tile_column, const int32_t* s_packed_a,
                                const int32_t* s_packed_meta, const int32_t* s_window_tile_offset,
                                int64_t tiles, int64_t n_s_window_tile_offset, int32_t window,
                                int32_t m, int32_t n, const trs_plan_options* opt, trs_plan** out);

/* SDDMM plan over the builder output, on the SpMM tiling: dense 16x16 tiles (TC blocks, 2:4 group
 * tiles with fill >= sptc_min_fill) run as MFMA dot products sampled at the stored entries, the
 * rest as wave64 CSR dot products.  Outputs follow the input's CSR order (the format must come
 * from canonical CSR).  Lowered on the device like trs_plan_create's plans.  No reference
 * counterpart (the reference has no SDDMM). */
int trs_plan_create_sddmm(const trs_format* f, int32_t m, int32_t n, const trs_plan_options* opt,
                          trs_plan** out);

/* trs_plan_create / trs_plan_create_sddmm from a device-resident format (trs_build_online_device),
 * on the device that holds it (TRS_EINVAL when another device is current).  No reference
 * counterpart (the reference hands its 29 arrays from the host, spmm/tr_csr_fp16/
 * mdataset2_online.py:100-113).  The format does not come to the host: its row pointers, the TC
 * arrays (slots 0-4, 6) and the 2:4 group tiles that pass the fill rule do; the residual is
 * placed from the format's device copy of the input CSR.  The plan equals the one
 * trs_plan_create(_sddmm) makes from trs_dformat_download's format, with the same options. */
int trs_plan_create_dformat(const trs_dformat* f, int32_t m, int32_t n, const trs_plan_options* opt,
                            trs_plan** out);
int trs_plan_create_sddmm_dformat(const trs_dformat* f, int32_t m, int32_t n, const trs_plan_options* opt,
                                  trs_plan** out);

/* Plain CSR SDDMM plan (fp16 values kept for the caller's reference only; SDDMM does not scale by
 * them): outputs in the given entry order.  No reference counterpart. */
int trs_plan_create_csr(const int32_t* rowptr, const int32_t* col, const uint16_t* val,
                        int32_t m, int32_t n, const trs_plan_options* opt, trs_plan** out);

typedef struct trs_plan_stats {
  int64_t m, n, nnz;                 /* nnz carried by the plan (all shares) */
  int64_t mfma_tiles, mfma_nnz;      /* 16x16 tiles on MFMA and the nonzeros inside them */
  int64_t csr_nnz;                   /* residual nonzeros */
  int64_t tasks, split_rows, partial_slots;
  int64_t device_bytes;              /* plan footprint in HBM */
  int64_t mfma_windows;              /* 16-row windows owned by the MFMA window kernel */
  int64_t window_csr_nnz;            /* residual nonzeros inside those windows */
  int64_t device_lowered;            /* 1: the residual was built on the device (host_lowering) */
  int64_t sparse_tiles;              /* of mfma_tiles, those run on the sparse MFMA (sptc_sparse) */
  int64_t hot_rows;                  /* staged hot rows (option hot_rows; 0 = none) */
  int64_t hot_entries;               /* entries whose B (Y) rows are staged */
} trs_plan_stats;

/* stats_bytes = sizeof(trs_plan_stats) of the caller's header; any other size: TRS_EINVAL, nothing
 * written. */
int trs_plan_stats_get(const trs_plan* p, trs_plan_stats* s, int64_t stats_bytes);
void trs_plan_free(trs_plan* p);

/* ---------------------------------------------------------------------------------------------
 * Execution.
 * ------------------------------------------------------------------------------------------- */
/* Bytes of device workspace trs_spmm_f16 needs for feature width K (0 when none): the partial
 * slots of split rows and, for K >= 128, the plan's staged hot B rows (option hot_rows). */
int64_t trs_spmm_workspace_bytes(const trs_plan* p, int32_t K);

/* C[m, K] (float32, row stride ldc) = A_plan (m x n) * B[n, K] (fp16, row stride ldb).
 * Every element of C is written exactly once per call (no prior zeroing needed, no atomics).
 * fp16 products, fp32 accumulation.  ldb < 2^31 (TRS_ERANGE otherwise). */
int trs_spmm_f16(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C, int64_t ldc,
                 void* workspace, int64_t workspace_bytes, void* stream);

/* trs_spmm_f16 without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  The workspace (partial slots, staged hot rows) comes from a static device array of
 * TRS_NOALLOC_SCRATCH_BYTES,
 * which every GPU the library runs on holds until the process ends; the call allocates nothing.
 * Plans whose trs_spmm_workspace_bytes(p, K) exceeds that size are refused with TRS_EINVAL.  All
 * calls on one GPU share its array: calls that overlap on one GPU race (serialise them).  Same
 * kernels and arguments as trs_spmm_f16, so the output is bitwise equal to it.  The first call on
 * each device looks the array's address up (hipGetSymbolAddress): make that call outside stream
 * capture.  Later calls only launch kernels and can be captured into a HIP graph; each replay
 * rewrites the array's contents before reading them. */
#define TRS_NOALLOC_SCRATCH_BYTES ((int64_t)128 << 20)
int trs_spmm_f16_noalloc(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C, int64_t ldc,
                         void* stream);

/* out[e] = sum_k X[row_e, k] * Y[col_e, k] for every stored entry e of the plan (order: see the
 * plan constructor).  X [m, K], Y [n, K] fp16; out float32 [nnz].  Only SDDMM plans
 * (trs_plan_create_sddmm, trs_plan_create_csr) are accepted.  ldy < 2^31 (TRS_ERANGE otherwise).
 * Kernels only (no memset nodes), so the call can be captured in a HIP graph. */
int trs_sddmm_f16(const trs_plan* p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy,
                  int32_t K, float* out, void* stream);

/* Bytes of device workspace trs_sddmm_f16_ws uses at feature width K: from K = 128, an output
 * buffer for the plan's split part (XCD sub-rows of its long rows, merged into place at the end of
 * the call) and the plan's staged hot Y rows (plan option hot_rows); 0 when the plan or K uses
 * neither.  No reference counterpart. */
int64_t trs_sddmm_workspace_bytes(const trs_plan* p, int32_t K);

/* trs_sddmm_f16 with a workspace of trs_sddmm_workspace_bytes(p, K) bytes (fewer: TRS_EINVAL):
 * the call copies the plan's hot Y rows there before the dot products gather them, and its split
 * part writes its outputs there in its own order before a merge puts them in place.  The same
 * outputs, bitwise (only where rows are read from and sums written to changes); trs_sddmm_f16
 * runs without either.  A workspace is the call's own: calls that overlap need separate
 * workspaces.  No reference counterpart. */
int trs_sddmm_f16_ws(const trs_plan* p, const uint16_t* X, int64_t ldx, const uint16_t* Y, int64_t ldy,
                     int32_t K, float* out, void* workspace, int64_t workspace_bytes, void* stream);

/* Launch-by-launch timing helper for the reference operators' `epoches` semantics
 * (mGCNkernel_online.cu:1604-1712): `warmup` untimed calls, then `iters` timed calls bracketed by
 * HIP events on `stream`; *ms_avg = mean time per call.  C holds the result of the last call. */
int trs_spmm_f16_timed(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C,
                       int64_t ldc, void* workspace, int64_t workspace_bytes, void* stream,
                       int32_t warmup, int32_t iters, float* ms_avg);

/* Per-kernel durations for profiling: `iters` calls, each of the (up to) three kernels of a call
 * bracketed by HIP events on `stream`.  ms[0] = residual task kernel, ms[1] = MFMA window kernel,
 * ms[2] = split-row fixup kernel; averages per call, 0 for a kernel the plan does not launch.
 * No reference counterpart (the reference reports per-stream completion times instead,
 * mGCNkernel_online.cu:1676-1687). */
int trs_spmm_f16_kernel_ms(const trs_plan* p, const uint16_t* B, int64_t ldb, int32_t K, float* C,
                           int64_t ldc, void* workspace, int64_t workspace_bytes, void* stream,
                           int32_t iters, float* ms);

/* SDDMM counterpart of trs_spmm_f16_kernel_ms (calls as trs_sddmm_f16_ws; workspace may be NULL
 * for unstaged calls): ms[0] = CSR dot-product kernel (with the hot-row copy), ms[1] = MFMA tile
 * kernel (averages over `iters` calls).  No reference counterpart. */
int trs_sddmm_f16_kernel_ms(const trs_plan* p, const uint16_t* X, int64_t ldx, const uint16_t* Y,
                            int64_t ldy, int32_t K, float* out, void* workspace, int64_t workspace_bytes,
                            void* stream, int32_t iters, float* ms);

const char* trs_last_error(void);

/* TRSPMM_ABI_VERSION of the header the library was built from. */
int32_t trs_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* TRSPMM_H */
