"""Drop-in for the reference's statistics-only 2:4 matcher module ``matching_utils``
(TR-source/setup_24matching.py:8-12, TR-source/Block/block_matching_window_para_dr.cpp:453-498).

``match_2to4(row_ptr, col_ind, values, window_size=16, dense_threshold=8, t_max=8)`` returns the
same statistics dict; the work runs in libtrspmm (trs_match_2to4).
"""
from trspmm.matching import match_2to4  # noqa: F401
