// Internal (C++) form of the builder output.  The C ABI in include/trspmm.h exposes it as an
// opaque handle with per-slot accessors.
#pragma once
#include <cstdint>
#include <string>
#include <vector>

#include "trspmm.h"

struct trs_format {
  // Slots 0-28: the reference return list (TR-source/Block/block_online.cpp:844-870).
  std::vector<int32_t> t_rowoff, t_blockoff, t_col, t_winrow, t_atomic;
  std::vector<float> t_val;
  std::vector<int64_t> t_bin;
  std::vector<int32_t> c_off, c_row, c_atomic, c_col;
  std::vector<float> c_val;
  std::vector<int32_t> cs_off, cs_row, cs_atomic, cs_col;
  std::vector<float> cs_val;
  std::vector<int32_t> s_col, s_win, s_offsets;
  std::vector<uint8_t> s_mask;
  std::vector<float> s_val;
  std::vector<int8_t> s_pos;
  std::vector<int32_t> tile_win, tile_group, tile_cols, packed_a, packed_meta, win_tile_off;
  // Slots 29-31: input entries that no array above carries (CSR edge order).
  std::vector<int32_t> spill_row, spill_col;
  std::vector<float> spill_val;

  // The input CSR itself (rowptr, col, val), kept when it is canonical: plan lowering can then
  // build the residual on the device from it instead of expanding the arrays above on the host.
  // Not part of the format file: a format read back has none and lowers on the host.
  std::vector<int32_t> csr_rowptr, csr_col;
  std::vector<float> csr_val;

  double elapsed = 0.0;     // slot "29" of the reference list (wall time of the build)
  int32_t rows = 0;         // rows of the input CSR (row1.size(0) - 1)
  int32_t window = 16;
  bool canonical = true;    // every input row had strictly increasing column indices
};

namespace trs {
void set_error(const std::string& msg);
uint16_t half_bits(float f);   // IEEE binary16, round to nearest even (c10::Half semantics)
}  // namespace trs
