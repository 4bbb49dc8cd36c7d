/* Test helper (compiled by tests/test_capi_c.py with gcc as C99 and linked against libtrspmm.so):
 * the C ABI used from plain C, as a C caller of the reference's builder path would use it.
 * Builds the format of a small CSR given on stdin ("rows nnz", then rowptr, then col, then val)
 * with trs_build_online and prints the element count of every slot, one per line; then checks the
 * error paths (NULL arguments, a params struct from another header version) and the ABI version.
 * No GPU is touched.  Exit status 0 on success. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "trspmm.h"

int main(void) {
  int32_t rows = 0;
  int64_t nnz = 0;
  if (scanf("%d %ld", &rows, &nnz) != 2) return 2;
  int32_t* rowptr = malloc(sizeof(int32_t) * (size_t)(rows + 1));
  int32_t* col = malloc(sizeof(int32_t) * (size_t)(nnz > 0 ? nnz : 1));
  float* val = malloc(sizeof(float) * (size_t)(nnz > 0 ? nnz : 1));
  for (int32_t i = 0; i <= rows; ++i)
    if (scanf("%d", &rowptr[i]) != 1) return 2;
  for (int64_t i = 0; i < nnz; ++i)
    if (scanf("%d", &col[i]) != 1) return 2;
  for (int64_t i = 0; i < nnz; ++i)
    if (scanf("%f", &val[i]) != 1) return 2;

  if (trs_abi_version() != TRSPMM_ABI_VERSION) {
    fprintf(stderr, "ABI version %d, header %d\n", trs_abi_version(), TRSPMM_ABI_VERSION);
    return 3;
  }
  trs_build_params p;
  trs_build_params_default(&p);
  if (p.struct_size != (int32_t)sizeof p) return 4;

  trs_format* f = NULL;
  int rc = trs_build_online(rowptr, col, val, rows, nnz, &p, &f);
  if (rc != TRS_OK) {
    fprintf(stderr, "trs_build_online: %s\n", trs_last_error());
    return 5;
  }
  for (int32_t s = 0; s < 32; ++s) {
    const void* data = NULL;
    int64_t n = -1;
    if (trs_format_slot(f, s, &data, &n) != TRS_OK) return 6;
    printf("%ld\n", (long)n);
  }
  if (trs_format_rows(f) != rows || trs_format_window(f) != 16 || trs_format_canonical(f) != 1) return 7;
  trs_format_free(f);

  /* errors are statuses with a message, never crashes */
  if (trs_build_online(rowptr, col, val, rows, nnz, &p, NULL) != TRS_EINVAL) return 8;
  if (strlen(trs_last_error()) == 0) return 9;
  trs_build_params q = p;
  q.struct_size = (int32_t)sizeof q - 4; /* a caller compiled against a shorter struct */
  f = NULL;
  if (trs_build_online(rowptr, col, val, rows, nnz, &q, &f) != TRS_EINVAL || f != NULL) return 10;
  free(rowptr);
  free(col);
  free(val);
  return 0;
}
