// Device-resident builder output (trs_dformat of include/trspmm.h): the 32 slots of trs_format in
// device memory, plus a copy of the input CSR, from which plans lower their residual.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "trspmm.h"

struct trs_dformat {
  void* mem = nullptr;         // slots 0-28 and the CSR copy
  void* spill_mem = nullptr;   // slots 29-31
  struct Slot { void* ptr; int64_t numel; };
  Slot slot[32] = {};
  int32_t* csr_rowptr = nullptr;
  int32_t* csr_col = nullptr;
  float* csr_val = nullptr;
  int64_t nnz = 0;
  int32_t rows = 0, window = 16, device = 0;
  double elapsed = 0.0;
  ~trs_dformat() {
    if (mem) (void)hipFree(mem);
    if (spill_mem) (void)hipFree(spill_mem);
  }
};
