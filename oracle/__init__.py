"""CPU oracle for the hybrid SpMM / SDDMM path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
anything from this package, and only as the checker or the reported CPU baseline.  The product path
(``tr-spmm_zzx_amd``) never imports, links or calls it, and fails loudly when its own HIP library is
missing.

Contents
  builder_oracle.cpp / builder.py  literal restatement of the reference format builder
                                   (TR-source/Block/block_online.cpp:545-871) + spill tracking
  spmm.py                          CSR SpMM / SDDMM in float64, and the meaning of every format
                                   array (the semantic spec the GPU plan must honour)
  tca.py                           the TCA row reorder's clustering and ordering rules
                                   (spmm/tr_csr_fp16/tr_tca_reorder.py) over exhaustive candidates
  matching.py                      the statistics-only 2:4 matcher
                                   (TR-source/Block/block_matching_window_para_dr.cpp)
  Makefile                         builds _build/liboracle_builder.so and, where the reference
                                   sources exist, _ref/Libra5BlockOnline (the reference builder)
                                   and _ref/matching_utils (the reference matcher)

Parity status of each function is stated in its docstring ("pinned by ...").
"""
