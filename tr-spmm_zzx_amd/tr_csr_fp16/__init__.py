"""Dataset layer of the hybrid SpMM path under the reference's module names
(spmm/tr_csr_fp16/{tr_paths,mdataset2_online}.py), so the reference harness
(spmm/tr_csr_fp16/test_tr_csr_online.py) runs unchanged on top of this library."""
