"""Drop-in for the reference operator module ``Libra6SpMMOnline``
(TR-source/SpMM/setup_online.py:8-16, TR-source/SpMM/mGCN_online.cpp:1141-1152).

Same four functions, positional arguments and return lists; CPU tensors in and out, with the
reference's `epoches` timing (10 warm-up launches, then `epoches` timed launches).
"""
from trspmm._native import ext as _ext

forward_fp16_tcu_cuda_sptc_mma_parallel_online = _ext().forward_fp16_tcu_cuda_sptc_mma_parallel_online
forward_fp16_sptc_online = _ext().forward_fp16_sptc_online
forward_fp16_sptc_mma_online = _ext().forward_fp16_sptc_mma_online
forward_fp16_sptc_mma_packed_online = _ext().forward_fp16_sptc_mma_packed_online
