// PyTorch extension with the reference operator signatures, over the C ABI of libtrspmm.so.
//
//   block_sptc_2to4_online          TR-source/Block/block_online.cpp:545-549, 873-876
//   forward_fp16_tcu_cuda_sptc_mma_parallel_online
//                                   TR-source/SpMM/mGCN_online.cpp:760-1138, 1151
//   forward_fp16_sptc_online        mGCN_online.cpp:202-400, 1145
//   forward_fp16_sptc_mma_online    mGCN_online.cpp:404-650, 1147
//   forward_fp16_sptc_mma_packed_online
//                                   mGCN_online.cpp:654-757, 1149
// Same positional arguments, dtype/shape checks (TORCH_CHECK -> RuntimeError) and return lists.
// The operators take CPU tensors and return CPU tensors, and time `epoches` launches after 10
// warm-up launches like the reference; the returned output comes from the last launch, which is
// complete on its own because every launch writes every output element once.
// Extras beyond the reference: the builder's spill list (`block_sptc_2to4_online_with_spill`) and
// optional spill arguments of the parallel operator, so the hybrid result equals the CSR SpMM.
#include <torch/cuda.h>
#include <torch/extension.h>

#include <cstdlib>
#include <cstring>
#include <vector>

#include "trspmm.h"

#define CHECK_CPU(x) TORCH_CHECK(!(x).is_cuda(), #x " must be a CPU tensor")
#define CHECK_DTYPE(x, dt) TORCH_CHECK((x).dtype() == (dt), #x " has an unexpected dtype")

namespace {

void ok(int rc, const char* what) { TORCH_CHECK(rc == TRS_OK, what, ": ", trs_last_error()); }

struct FormatGuard {
  trs_format* f = nullptr;
  ~FormatGuard() { trs_format_free(f); }
};
struct PlanGuard {
  trs_plan* p = nullptr;
  ~PlanGuard() { trs_plan_free(p); }
};

torch::Tensor slot_tensor(const trs_format* f, int slot, torch::ScalarType dt) {
  const void* data = nullptr;
  int64_t n = 0;
  ok(trs_format_slot(f, slot, &data, &n), "trs_format_slot");
  auto t = torch::empty({n}, torch::TensorOptions().dtype(dt));
  if (n) std::memcpy(t.data_ptr(), data, (size_t)n * t.element_size());
  return t;
}

std::vector<torch::Tensor> build_impl(torch::Tensor row1, torch::Tensor column1, torch::Tensor values1,
                                      int partSize_t, int partSize_c, int shortSize, int density, int window,
                                      int wide, float tc_min_util, float sptc_min_util, int sptc_threshold,
                                      bool with_spill) {
  // block_online.cpp:551-553
  TORCH_CHECK(row1.dtype() == torch::kInt32 && column1.dtype() == torch::kInt32);
  TORCH_CHECK(values1.dtype() == torch::kFloat32);
  TORCH_CHECK(window > 0 && window <= 32 && wide > 0 && wide <= 32);
  CHECK_CPU(row1);
  CHECK_CPU(column1);
  CHECK_CPU(values1);
  row1 = row1.contiguous();
  column1 = column1.contiguous();
  values1 = values1.contiguous();
  TORCH_CHECK(row1.dim() == 1 && row1.size(0) >= 1, "row1 must be 1-D with at least one element");
  TORCH_CHECK(column1.numel() == values1.numel(), "column1 and values1 must have the same length");
  trs_build_params p;
  trs_build_params_default(&p);
  p.part_size_t = partSize_t;
  p.part_size_c = partSize_c;
  p.short_size = shortSize;
  p.density = density;
  p.window = window;
  p.wide = wide;
  p.tc_min_util = tc_min_util;
  p.sptc_min_util = sptc_min_util;
  p.sptc_threshold = sptc_threshold;
  FormatGuard g;
  {
    pybind11::gil_scoped_release nogil;
    ok(trs_build_online(row1.data_ptr<int32_t>(), column1.data_ptr<int32_t>(), values1.data_ptr<float>(),
                        (int32_t)(row1.size(0) - 1), column1.numel(), &p, &g.f),
       "block_sptc_2to4_online");
  }
  const torch::ScalarType dt[32] = {
      torch::kInt32, torch::kInt32, torch::kInt32, torch::kFloat32, torch::kInt32, torch::kInt32, torch::kInt64,
      torch::kInt32, torch::kInt32, torch::kInt32, torch::kInt32, torch::kFloat32,
      torch::kInt32, torch::kInt32, torch::kInt32, torch::kInt32, torch::kFloat32,
      torch::kInt32, torch::kUInt8, torch::kFloat32, torch::kInt8, torch::kInt32, torch::kInt32,
      torch::kInt32, torch::kInt32, torch::kInt32, torch::kInt32, torch::kInt32, torch::kInt32,
      torch::kInt32, torch::kInt32, torch::kFloat32};
  std::vector<torch::Tensor> out;
  for (int s = 0; s < 29; ++s) out.push_back(slot_tensor(g.f, s, dt[s]));
  const int64_t G = out[21].size(0), T = out[23].size(0);
  out[17] = out[17].view({G, 4});
  out[18] = out[18].view({G, window});
  out[19] = out[19].view({G, window, 2});
  out[20] = out[20].view({G, window, 2});
  out[25] = out[25].view({T, 16});
  out[26] = out[26].view({T, 8, 4, 2});
  out[27] = out[27].view({T, 8});
  out.push_back(torch::tensor(trs_format_elapsed(g.f)));
  if (with_spill)
    for (int s = 29; s < 32; ++s) out.push_back(slot_tensor(g.f, s, dt[s]));
  return out;
}

std::vector<torch::Tensor> block_sptc_2to4_online(torch::Tensor row1, torch::Tensor column1, torch::Tensor values1,
                                                  int partSize_t, int partSize_c, int shortSize, int density,
                                                  int window, int wide, float tc_min_util, float sptc_min_util,
                                                  int sptc_threshold) {
  return build_impl(row1, column1, values1, partSize_t, partSize_c, shortSize, density, window, wide, tc_min_util,
                    sptc_min_util, sptc_threshold, false);
}

std::vector<torch::Tensor> block_sptc_2to4_online_with_spill(torch::Tensor row1, torch::Tensor column1,
                                                             torch::Tensor values1, int partSize_t, int partSize_c,
                                                             int shortSize, int density, int window, int wide,
                                                             float tc_min_util, float sptc_min_util,
                                                             int sptc_threshold) {
  return build_impl(row1, column1, values1, partSize_t, partSize_c, shortSize, density, window, wide, tc_min_util,
                    sptc_min_util, sptc_threshold, true);
}

// Plan options of the operators whose reference kernels run 2:4 tiles on sparse tensor cores
// (mma.sp, mGCNkernel_online.cu:570-786, 812-933): 2:4 tiles on gfx950's sparse MFMA.
trs_plan_options sparse_tile_options() {
  trs_plan_options o;
  trs_plan_options_default(&o);
  o.sptc_sparse = 1;
  return o;
}

struct RunResult {
  torch::Tensor out;
  float ms = 0.f;
  float kernel_ms[3] = {0.f, 0.f, 0.f};   // residual tasks, MFMA windows, split-row fixups
};

// Run a plan on a CPU rhs with the reference's timing semantics: 10 warm-up launches, `epoches`
// timed launches (mGCNkernel_online.cu:1604-1674); the result of the last launch is returned.
RunResult run_plan(trs_plan* plan, torch::Tensor rhs, int dimN, int mOri, int kOri, int epoches) {
  auto dev = torch::TensorOptions().device(torch::kCUDA);
  torch::Tensor B = rhs.reshape({kOri, dimN}).to(dev.dtype(torch::kFloat16));
  torch::Tensor C = torch::empty({mOri, dimN}, dev.dtype(torch::kFloat32));
  const int64_t wsb = trs_spmm_workspace_bytes(plan, dimN);
  torch::Tensor ws = torch::empty({std::max<int64_t>(wsb, 1)}, dev.dtype(torch::kUInt8));
  torch::cuda::synchronize();
  RunResult r;
  const uint16_t* b = reinterpret_cast<const uint16_t*>(B.data_ptr());
  ok(trs_spmm_f16_timed(plan, b, dimN, dimN, C.data_ptr<float>(), dimN, ws.data_ptr(), wsb, nullptr, 10, epoches, &r.ms),
     "spmm");
  ok(trs_spmm_f16_kernel_ms(plan, b, dimN, dimN, C.data_ptr<float>(), dimN, ws.data_ptr(), wsb, nullptr, epoches,
                            r.kernel_ms),
     "spmm kernel timing");
  torch::cuda::synchronize();
  r.out = C.cpu();
  return r;
}

void common_checks(int window, int dimN, int mOri, int kOri, int epoches, const torch::Tensor& rhs,
                   const char* window_msg, int max_window) {
  if (max_window > 0) {
    TORCH_CHECK(window > 0 && window <= max_window, window_msg);
  } else {
    TORCH_CHECK(window > 0, window_msg);
  }
  TORCH_CHECK(dimN > 0, "dimN must be positive");
  TORCH_CHECK(mOri > 0, "mOri must be positive");
  TORCH_CHECK(kOri > 0, "kOri must be positive");
  TORCH_CHECK(epoches > 0, "epoches must be positive");
  TORCH_CHECK(rhs.numel() == (int64_t)kOri * dimN, "rhs_matrix must have kOri * dimN elements");
}

const uint16_t* h16(const torch::Tensor& t) { return reinterpret_cast<const uint16_t*>(t.data_ptr()); }

// The reference's on/off environment switches: "1", "true" or "TRUE" enable
// (TR-source/SpMM/mGCNkernel_online.cu:27-32).
bool env_enabled(const char* name) {
  const char* v = std::getenv(name);
  return v && (std::strcmp(v, "1") == 0 || std::strcmp(v, "true") == 0 || std::strcmp(v, "TRUE") == 0);
}

std::vector<torch::Tensor> parallel_online(
    torch::Tensor t_row_offset, torch::Tensor t_blockNew_offset, torch::Tensor t_column, torch::Tensor t_value,
    torch::Tensor t_window_row, torch::Tensor t_atomic, torch::Tensor t_binary, torch::Tensor c_row_offsets,
    torch::Tensor c_row, torch::Tensor c_atomic, torch::Tensor c_column, torch::Tensor c_value,
    torch::Tensor c_row_offsets_short, torch::Tensor c_row_short, torch::Tensor c_atomic_short,
    torch::Tensor c_column_short, torch::Tensor c_value_short, torch::Tensor s_column, torch::Tensor s_value,
    torch::Tensor s_pos, torch::Tensor s_offsets, torch::Tensor s_tile_window, torch::Tensor s_tile_column,
    torch::Tensor s_packed_a, torch::Tensor s_packed_meta, torch::Tensor s_window_tile_offset,
    torch::Tensor rhs_matrix, int parts_t, int parts_c, int partsize_c, int parts_c_short, int window, int dimN,
    int mOri, int kOri, int epoches, c10::optional<torch::Tensor> spill_row, c10::optional<torch::Tensor> spill_col,
    c10::optional<torch::Tensor> spill_val) {
  std::vector<torch::Tensor*> all = {&t_row_offset, &t_blockNew_offset, &t_column, &t_value, &t_window_row,
                                     &t_atomic, &t_binary, &c_row_offsets, &c_row, &c_atomic, &c_column, &c_value,
                                     &c_row_offsets_short, &c_row_short, &c_atomic_short, &c_column_short,
                                     &c_value_short, &s_column, &s_value, &s_pos, &s_offsets, &s_tile_window,
                                     &s_tile_column, &s_packed_a, &s_packed_meta, &s_window_tile_offset, &rhs_matrix};
  static const char* names[] = {"t_row_offset", "t_blockNew_offset", "t_column", "t_value", "t_window_row",
                                "t_atomic", "t_binary", "c_row_offsets", "c_row", "c_atomic", "c_column", "c_value",
                                "c_row_offsets_short", "c_row_short", "c_atomic_short", "c_column_short",
                                "c_value_short", "s_column", "s_value", "s_pos", "s_offsets", "s_tile_window",
                                "s_tile_column", "s_packed_a", "s_packed_meta", "s_window_tile_offset", "rhs_matrix"};
  for (size_t i = 0; i < all.size(); ++i) TORCH_CHECK(!all[i]->is_cuda(), names[i], " must be a CPU tensor");
  for (auto* t : all) *t = t->contiguous();
  CHECK_DTYPE(t_row_offset, torch::kInt32);
  CHECK_DTYPE(t_blockNew_offset, torch::kInt32);
  CHECK_DTYPE(t_column, torch::kInt32);
  CHECK_DTYPE(t_value, torch::kFloat16);
  CHECK_DTYPE(t_window_row, torch::kInt32);
  CHECK_DTYPE(t_atomic, torch::kInt32);
  CHECK_DTYPE(t_binary, torch::kInt64);
  CHECK_DTYPE(c_row_offsets, torch::kInt32);
  CHECK_DTYPE(c_row, torch::kInt32);
  CHECK_DTYPE(c_atomic, torch::kInt32);
  CHECK_DTYPE(c_column, torch::kInt32);
  CHECK_DTYPE(c_value, torch::kFloat16);
  CHECK_DTYPE(c_row_offsets_short, torch::kInt32);
  CHECK_DTYPE(c_row_short, torch::kInt32);
  CHECK_DTYPE(c_atomic_short, torch::kInt32);
  CHECK_DTYPE(c_column_short, torch::kInt32);
  CHECK_DTYPE(c_value_short, torch::kFloat16);
  CHECK_DTYPE(s_column, torch::kInt32);
  CHECK_DTYPE(s_value, torch::kFloat32);
  CHECK_DTYPE(s_pos, torch::kInt8);
  CHECK_DTYPE(s_offsets, torch::kInt32);
  CHECK_DTYPE(s_tile_window, torch::kInt32);
  CHECK_DTYPE(s_tile_column, torch::kInt32);
  CHECK_DTYPE(s_packed_a, torch::kInt32);
  CHECK_DTYPE(s_packed_meta, torch::kInt32);
  CHECK_DTYPE(rhs_matrix, torch::kFloat16);
  common_checks(window, dimN, mOri, kOri, epoches, rhs_matrix, "parallel mma path requires 0 < window <= 16", 16);
  TORCH_CHECK(s_column.dim() == 2 && s_column.size(1) == 4, "s_column must have shape [groups, 4]");
  TORCH_CHECK(s_value.dim() == 3 && s_value.size(1) == window && s_value.size(2) == 2,
              "s_value must have shape [groups, window, 2]");
  TORCH_CHECK(s_pos.dim() == 3 && s_pos.size(1) == window && s_pos.size(2) == 2,
              "s_pos must have shape [groups, window, 2]");
  TORCH_CHECK(s_offsets.dim() == 1 && s_offsets.size(0) >= 1, "s_offsets must be 1-D with at least one item");
  TORCH_CHECK(s_tile_window.dim() == 1, "s_tile_window must be 1-D");
  TORCH_CHECK(s_tile_column.dim() == 2 && s_tile_column.size(1) == 16, "s_tile_column must have shape [tiles, 16]");
  TORCH_CHECK(s_packed_a.dim() == 4 && s_packed_a.size(1) == 8 && s_packed_a.size(2) == 4 && s_packed_a.size(3) == 2,
              "s_packed_a must have shape [tiles, 8, 4, 2]");
  TORCH_CHECK(s_packed_meta.dim() == 2 && s_packed_meta.size(1) == 8, "s_packed_meta must have shape [tiles, 8]");
  const int64_t groups = s_column.size(0);
  TORCH_CHECK(s_value.size(0) == groups, "s_value group count mismatch");
  TORCH_CHECK(s_pos.size(0) == groups, "s_pos group count mismatch");
  const int32_t* so = s_offsets.data_ptr<int32_t>();
  const int64_t nwin = s_offsets.size(0) - 1;
  TORCH_CHECK(so[0] == 0, "s_offsets must start with 0");
  TORCH_CHECK(so[nwin] == groups, "s_offsets end must equal group count");
  int64_t tiles_from_offsets = 0;
  for (int64_t w = 0; w < nwin; ++w) {
    TORCH_CHECK(so[w + 1] - so[w] >= 0, "s_offsets must be non-decreasing");
    tiles_from_offsets += (so[w + 1] - so[w] + 3) / 4;
  }
  const int64_t tiles = s_tile_window.size(0);
  TORCH_CHECK(s_tile_column.size(0) == tiles, "s_tile_column tile count mismatch");
  TORCH_CHECK(s_packed_a.size(0) == tiles, "s_packed_a tile count mismatch");
  TORCH_CHECK(s_packed_meta.size(0) == tiles, "s_packed_meta tile count mismatch");
  TORCH_CHECK(tiles == tiles_from_offsets, "packed tile count must match offsets-derived tile count");
  TORCH_CHECK(s_window_tile_offset.dim() == 1 && s_window_tile_offset.size(0) == nwin + 1,
              "s_window_tile_offset must have one entry per window plus one");
  // part counts select how many parts run, as the reference grids do; they may not exceed the arrays
  TORCH_CHECK(parts_t >= 0 && parts_t <= t_atomic.size(0) && parts_t <= t_row_offset.size(0) - 1,
              "parts_t exceeds the TC part arrays");
  TORCH_CHECK(parts_c >= 0 && parts_c <= c_row.size(0) && parts_c <= c_row_offsets.size(0) - 1,
              "parts_c exceeds the residual part arrays");
  TORCH_CHECK(parts_c_short >= 0 && parts_c_short <= c_row_short.size(0) &&
                  parts_c_short <= c_row_offsets_short.size(0) - 1,
              "parts_c_short exceeds the short residual part arrays");
  (void)partsize_c;

  trs_parallel_arrays a;
  std::memset(&a, 0, sizeof(a));
  // LIBRA_SKIP_TC_KERNEL skips the TC share, as the reference's debug switch skips its TC kernel
  // (mGCNkernel_online.cu:1397-1410)
  const int tc_parts = env_enabled("LIBRA_SKIP_TC_KERNEL") ? 0 : parts_t;
  a.t_row_offset = t_row_offset.data_ptr<int32_t>(); a.n_t_row_offset = tc_parts + 1;
  a.t_block_offset = t_blockNew_offset.data_ptr<int32_t>(); a.n_t_block_offset = t_blockNew_offset.numel();
  a.t_column = t_column.data_ptr<int32_t>(); a.n_t_column = t_column.numel();
  a.t_value = h16(t_value); a.n_t_value = t_value.numel();
  a.t_window_row = t_window_row.data_ptr<int32_t>(); a.n_t_window_row = tc_parts;
  a.t_atomic = t_atomic.data_ptr<int32_t>(); a.n_t_atomic = tc_parts;
  a.t_binary = t_binary.data_ptr<int64_t>(); a.n_t_binary = t_binary.numel();
  a.c_row_offsets = c_row_offsets.data_ptr<int32_t>(); a.n_c_row_offsets = parts_c + 1;
  a.c_row = c_row.data_ptr<int32_t>(); a.n_c_row = parts_c;
  a.c_atomic = c_atomic.data_ptr<int32_t>(); a.n_c_atomic = parts_c;
  a.c_column = c_column.data_ptr<int32_t>(); a.n_c_column = c_column.numel();
  a.c_value = h16(c_value); a.n_c_value = c_value.numel();
  a.cs_row_offsets = c_row_offsets_short.data_ptr<int32_t>(); a.n_cs_row_offsets = parts_c_short + 1;
  a.cs_row = c_row_short.data_ptr<int32_t>(); a.n_cs_row = parts_c_short;
  a.cs_atomic = c_atomic_short.data_ptr<int32_t>(); a.n_cs_atomic = parts_c_short;
  a.cs_column = c_column_short.data_ptr<int32_t>(); a.n_cs_column = c_column_short.numel();
  a.cs_value = h16(c_value_short); a.n_cs_value = c_value_short.numel();
  TORCH_CHECK(c_value.numel() >= c_column.numel() && c_value_short.numel() >= c_column_short.numel(),
              "residual value arrays shorter than column arrays");
  a.s_column = s_column.data_ptr<int32_t>(); a.s_value = s_value.data_ptr<float>(); a.s_pos = s_pos.data_ptr<int8_t>();
  a.groups = groups;
  a.s_offsets = so; a.n_s_offsets = nwin + 1;
  a.s_tile_column = s_tile_column.data_ptr<int32_t>(); a.s_packed_a = s_packed_a.data_ptr<int32_t>();
  a.s_packed_meta = s_packed_meta.data_ptr<int32_t>();
  a.s_window_tile_offset = s_window_tile_offset.data_ptr<int32_t>(); a.tiles = tiles;
  a.n_s_window_tile_offset = s_window_tile_offset.numel();
  a.use_packed_tiles = 1;   // the reference parallel operator's 2:4 kernel reads the packed tiles
  torch::Tensor sr, sc, sv;
  if (spill_row.has_value() || spill_col.has_value() || spill_val.has_value()) {
    TORCH_CHECK(spill_row.has_value() && spill_col.has_value() && spill_val.has_value(),
                "spill_row, spill_col and spill_val go together");
    sr = spill_row->contiguous(); sc = spill_col->contiguous(); sv = spill_val->contiguous();
    CHECK_CPU(sr); CHECK_CPU(sc); CHECK_CPU(sv);
    CHECK_DTYPE(sr, torch::kInt32); CHECK_DTYPE(sc, torch::kInt32); CHECK_DTYPE(sv, torch::kFloat32);
    TORCH_CHECK(sr.numel() == sc.numel() && sc.numel() == sv.numel(), "spill arrays must have equal length");
    a.spill_row = sr.data_ptr<int32_t>(); a.spill_col = sc.data_ptr<int32_t>(); a.spill_val = sv.data_ptr<float>();
    a.spill_count = sr.numel();
  }
  a.parts_t = tc_parts; a.parts_c = parts_c; a.partsize_c = partsize_c; a.parts_c_short = parts_c_short;
  a.window = window; a.m = mOri; a.n = kOri;
  PlanGuard pg;
  const trs_plan_options po = sparse_tile_options();
  ok(trs_plan_create_parallel(&a, &po, &pg.p), "forward_fp16_tcu_cuda_sptc_mma_parallel_online");
  auto res = run_plan(pg.p, rhs_matrix, dimN, mOri, kOri, epoches);
  // Per-path times with the reference's meaning (mGCNkernel_online.cu:1676-1687): the time from
  // the common start of the `epoches` launches to the completion of that path, divided by
  // `epoches`.  Here the paths are kernels of one stream, run in the order residual tasks ->
  // MFMA windows -> split-row fixups in every launch: path X completes (epoches - 1) steps plus
  // its offset inside the last step after the start.  TC = the MFMA window kernel (dense TC and
  // 2:4 tiles), cuda_long = the residual task kernel, cuda_short = the fixups; the 2:4 groups
  // finish with the MFMA window kernel (dense tiles) and the residual kernel (the rest), so their
  // completion is the later of the two, the MFMA window kernel's.
  const float e = (float)epoches;
  auto completion = [&](float offset) { return ((e - 1.f) * res.ms + offset) / e; };
  const float t_long = completion(res.kernel_ms[0]);
  const float t_tc = completion(res.kernel_ms[0] + res.kernel_ms[1]);
  const float t_short = completion(res.kernel_ms[0] + res.kernel_ms[1] + res.kernel_ms[2]);
  return {res.out, torch::tensor(res.ms), torch::tensor(t_tc), torch::tensor(t_long), torch::tensor(t_short),
          torch::tensor(t_tc)};
}

std::vector<torch::Tensor> sptc_online(torch::Tensor s_column, torch::Tensor s_value, torch::Tensor s_pos,
                                       torch::Tensor s_window, torch::Tensor rhs_matrix, int window, int dimN,
                                       int mOri, int kOri, int epoches) {
  for (auto* t : {&s_column, &s_value, &s_pos, &s_window, &rhs_matrix}) {
    TORCH_CHECK(!t->is_cuda(), "inputs must be CPU tensors");
    *t = t->contiguous();
  }
  CHECK_DTYPE(s_column, torch::kInt32);
  CHECK_DTYPE(s_value, torch::kFloat32);
  CHECK_DTYPE(s_pos, torch::kInt8);
  CHECK_DTYPE(s_window, torch::kInt32);
  CHECK_DTYPE(rhs_matrix, torch::kFloat16);
  common_checks(window, dimN, mOri, kOri, epoches, rhs_matrix, "window must be positive", 0);
  TORCH_CHECK(s_column.dim() == 2 && s_column.size(1) == 4, "s_column must have shape [groups, 4]");
  TORCH_CHECK(s_value.dim() == 3 && s_value.size(1) == window && s_value.size(2) == 2,
              "s_value must have shape [groups, window, 2]");
  TORCH_CHECK(s_pos.dim() == 3 && s_pos.size(1) == window && s_pos.size(2) == 2,
              "s_pos must have shape [groups, window, 2]");
  TORCH_CHECK(s_window.dim() == 1, "s_window must be 1-D");
  const int64_t groups = s_window.size(0);
  TORCH_CHECK(s_column.size(0) == groups, "s_column group count mismatch");
  TORCH_CHECK(s_value.size(0) == groups, "s_value group count mismatch");
  TORCH_CHECK(s_pos.size(0) == groups, "s_pos group count mismatch");
  PlanGuard pg;
  ok(trs_plan_create_sptc(s_column.data_ptr<int32_t>(), s_value.data_ptr<float>(), s_pos.data_ptr<int8_t>(), groups,
                          s_window.data_ptr<int32_t>(), nullptr, 0, window, mOri, kOri, nullptr, &pg.p),
     "forward_fp16_sptc_online");
  auto res = run_plan(pg.p, rhs_matrix, dimN, mOri, kOri, epoches);
  return {res.out, torch::tensor(res.ms)};
}

std::vector<torch::Tensor> sptc_mma_online(torch::Tensor s_column, torch::Tensor s_value, torch::Tensor s_pos,
                                           torch::Tensor s_offsets, torch::Tensor rhs_matrix, int window, int dimN,
                                           int mOri, int kOri, int epoches) {
  for (auto* t : {&s_column, &s_value, &s_pos, &s_offsets, &rhs_matrix}) {
    TORCH_CHECK(!t->is_cuda(), "inputs must be CPU tensors");
    *t = t->contiguous();
  }
  CHECK_DTYPE(s_column, torch::kInt32);
  CHECK_DTYPE(s_value, torch::kFloat32);
  CHECK_DTYPE(s_pos, torch::kInt8);
  CHECK_DTYPE(s_offsets, torch::kInt32);
  CHECK_DTYPE(rhs_matrix, torch::kFloat16);
  common_checks(window, dimN, mOri, kOri, epoches, rhs_matrix, "mma path requires 0 < window <= 16", 16);
  TORCH_CHECK(s_column.dim() == 2 && s_column.size(1) == 4, "s_column must have shape [groups, 4]");
  TORCH_CHECK(s_value.dim() == 3 && s_value.size(1) == window && s_value.size(2) == 2,
              "s_value must have shape [groups, window, 2]");
  TORCH_CHECK(s_pos.dim() == 3 && s_pos.size(1) == window && s_pos.size(2) == 2,
              "s_pos must have shape [groups, window, 2]");
  TORCH_CHECK(s_offsets.dim() == 1 && s_offsets.size(0) >= 1, "s_offsets must be 1-D with at least one item");
  const int64_t groups = s_column.size(0);
  TORCH_CHECK(s_value.size(0) == groups, "s_value group count mismatch");
  TORCH_CHECK(s_pos.size(0) == groups, "s_pos group count mismatch");
  PlanGuard pg;
  const trs_plan_options po = sparse_tile_options();
  ok(trs_plan_create_sptc(s_column.data_ptr<int32_t>(), s_value.data_ptr<float>(), s_pos.data_ptr<int8_t>(), groups,
                          nullptr, s_offsets.data_ptr<int32_t>(), s_offsets.numel(), window, mOri, kOri, &po,
                          &pg.p),
     "forward_fp16_sptc_mma_online");
  auto res = run_plan(pg.p, rhs_matrix, dimN, mOri, kOri, epoches);
  return {res.out, torch::tensor(res.ms)};
}

std::vector<torch::Tensor> sptc_mma_packed_online(torch::Tensor s_tile_column, torch::Tensor s_packed_a,
                                                  torch::Tensor s_packed_meta, torch::Tensor s_window_tile_offset,
                                                  torch::Tensor rhs_matrix, int window, int dimN, int mOri, int kOri,
                                                  int epoches) {
  CHECK_CPU(s_tile_column);
  CHECK_CPU(s_packed_a);
  CHECK_CPU(s_packed_meta);
  CHECK_CPU(s_window_tile_offset);
  CHECK_CPU(rhs_matrix);
  for (auto* t : {&s_tile_column, &s_packed_a, &s_packed_meta, &s_window_tile_offset, &rhs_matrix})
    *t = t->contiguous();
  CHECK_DTYPE(s_tile_column, torch::kInt32);
  CHECK_DTYPE(s_packed_a, torch::kInt32);
  CHECK_DTYPE(s_packed_meta, torch::kInt32);
  CHECK_DTYPE(s_window_tile_offset, torch::kInt32);
  CHECK_DTYPE(rhs_matrix, torch::kFloat16);
  common_checks(window, dimN, mOri, kOri, epoches, rhs_matrix, "packed mma path requires 0 < window <= 16", 16);
  TORCH_CHECK(s_tile_column.dim() == 2 && s_tile_column.size(1) == 16, "s_tile_column must have shape [tiles, 16]");
  TORCH_CHECK(s_packed_a.dim() == 4 && s_packed_a.size(1) == 8 && s_packed_a.size(2) == 4 && s_packed_a.size(3) == 2,
              "s_packed_a must have shape [tiles, 8, 4, 2]");
  TORCH_CHECK(s_packed_meta.dim() == 2 && s_packed_meta.size(1) == 8, "s_packed_meta must have shape [tiles, 8]");
  TORCH_CHECK(s_window_tile_offset.dim() == 1 && s_window_tile_offset.size(0) >= 2,
              "s_window_tile_offset must be 1-D with at least 2 elements");
  const int64_t tiles = s_tile_column.size(0);
  TORCH_CHECK(s_packed_a.size(0) == tiles, "s_packed_a tile count mismatch");
  TORCH_CHECK(s_packed_meta.size(0) == tiles, "s_packed_meta tile count mismatch");
  PlanGuard pg;
  const trs_plan_options po = sparse_tile_options();
  ok(trs_plan_create_sptc_packed(s_tile_column.data_ptr<int32_t>(), s_packed_a.data_ptr<int32_t>(),
                                 s_packed_meta.data_ptr<int32_t>(), s_window_tile_offset.data_ptr<int32_t>(), tiles,
                                 s_window_tile_offset.numel(), window, mOri, kOri, &po, &pg.p),
     "forward_fp16_sptc_mma_packed_online");
  auto res = run_plan(pg.p, rhs_matrix, dimN, mOri, kOri, epoches);
  return {res.out, torch::tensor(res.ms)};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("block_sptc_2to4_online", &block_sptc_2to4_online,
        "Hybrid format builder: 16-row windows -> TC blocks, 2:4 groups, CSR residual (29 arrays + time)");
  m.def("block_sptc_2to4_online_with_spill", &block_sptc_2to4_online_with_spill,
        "block_sptc_2to4_online plus the spill list (rows, columns, values the 2:4 step drops)");
  m.def("forward_fp16_tcu_cuda_sptc_mma_parallel_online", &parallel_online,
        "Hybrid fp16 SpMM over the builder arrays (MFMA tiles + wave64 residual)", pybind11::arg("t_row_offset"),
        pybind11::arg("t_blockNew_offset"), pybind11::arg("t_column"), pybind11::arg("t_value"),
        pybind11::arg("t_window_row"), pybind11::arg("t_atomic"), pybind11::arg("t_binary"),
        pybind11::arg("c_row_offsets"), pybind11::arg("c_row"), pybind11::arg("c_atomic"), pybind11::arg("c_column"),
        pybind11::arg("c_value"), pybind11::arg("c_row_offsets_short"), pybind11::arg("c_row_short"),
        pybind11::arg("c_atomic_short"), pybind11::arg("c_column_short"), pybind11::arg("c_value_short"),
        pybind11::arg("s_column"), pybind11::arg("s_value"), pybind11::arg("s_pos"), pybind11::arg("s_offsets"),
        pybind11::arg("s_tile_window"), pybind11::arg("s_tile_column"), pybind11::arg("s_packed_a"),
        pybind11::arg("s_packed_meta"), pybind11::arg("s_window_tile_offset"), pybind11::arg("rhs_matrix"),
        pybind11::arg("parts_t"), pybind11::arg("parts_c"), pybind11::arg("partsize_c"),
        pybind11::arg("parts_c_short"), pybind11::arg("window"), pybind11::arg("dimN"), pybind11::arg("mOri"),
        pybind11::arg("kOri"), pybind11::arg("epoches"), pybind11::arg("spill_row") = pybind11::none(),
        pybind11::arg("spill_col") = pybind11::none(), pybind11::arg("spill_val") = pybind11::none());
  m.def("forward_fp16_sptc_online", &sptc_online, "2:4 group SpMM, rows from s_window");
  m.def("forward_fp16_sptc_mma_online", &sptc_mma_online, "2:4 group SpMM, windows from s_offsets");
  m.def("forward_fp16_sptc_mma_packed_online", &sptc_mma_packed_online, "2:4 group SpMM from packed tiles");
}
