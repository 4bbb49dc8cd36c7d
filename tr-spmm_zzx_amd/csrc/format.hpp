// Internal (C++) form of the builder output.  The C ABI in include/trspmm.h exposes it as an
// opaque handle with per-slot accessors.
#pragma once
#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "trspmm.h"

namespace trs {
// Allocator whose value-initialising construct() leaves scalars uninitialised.  The builder sizes
// the format arrays and then writes every element in parallel, so the zero-fill of a plain
// resize() would only add a serial pass over the whole allocation (and take all its page faults on
// one thread: 0.35 s of a 0.73 s R-MAT build).
template <class T>
struct uninit_allocator : std::allocator<T> {
  uninit_allocator() noexcept = default;
  template <class U>
  uninit_allocator(const uninit_allocator<U>&) noexcept {}
  template <class U>
  struct rebind { using other = uninit_allocator<U>; };
  template <class U>
  void construct(U* p) noexcept { ::new (static_cast<void*>(p)) U; }
  template <class U, class... A>
  void construct(U* p, A&&... a) { ::new (static_cast<void*>(p)) U(std::forward<A>(a)...); }
};
template <class T>
using array = std::vector<T, uninit_allocator<T>>;
}  // namespace trs

struct trs_format {
  // Slots 0-28: the reference return list (TR-source/Block/block_online.cpp:844-870).
  trs::array<int32_t> t_rowoff, t_blockoff, t_col, t_winrow, t_atomic;
  trs::array<float> t_val;
  trs::array<int64_t> t_bin;
  trs::array<int32_t> c_off, c_row, c_atomic, c_col;
  trs::array<float> c_val;
  trs::array<int32_t> cs_off, cs_row, cs_atomic, cs_col;
  trs::array<float> cs_val;
  trs::array<int32_t> s_col, s_win, s_offsets;
  trs::array<uint8_t> s_mask;
  trs::array<float> s_val;
  trs::array<int8_t> s_pos;
  trs::array<int32_t> tile_win, tile_group, tile_cols, packed_a, packed_meta, win_tile_off;
  // Slots 29-31: input entries that no array above carries (CSR edge order).
  trs::array<int32_t> spill_row, spill_col;
  trs::array<float> spill_val;

  // The input CSR itself (rowptr, col, val), kept when it is canonical: plan lowering can then
  // build the residual on the device from it instead of expanding the arrays above on the host.
  // Not part of the format file: a format read back has none and lowers on the host.
  trs::array<int32_t> csr_rowptr, csr_col;
  trs::array<float> csr_val;

  double elapsed = 0.0;     // slot "29" of the reference list (wall time of the build)
  int32_t rows = 0;         // rows of the input CSR (row1.size(0) - 1)
  int32_t window = 16;
  bool canonical = true;    // every input row had strictly increasing column indices
};

namespace trs {
void set_error(const std::string& msg);
uint16_t half_bits(float f);   // IEEE binary16, round to nearest even (c10::Half semantics)
void half_bits_n(const float* src, uint16_t* dst, int64_t n);   // the same for n values
}  // namespace trs
