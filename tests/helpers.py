"""Shared test helpers: the BC struct view moe_ffn reads, and tolerances."""
import ctypes

import numpy as np  # noqa: F401

from mojollama_amd.workloads import BCView  # noqa: E402,F401  (the BC struct moe_ffn reads)


# Normalised max error bound (max|got - ref| / max|ref|) per semantic for the
# GPU library against the oracle.  Every GEMV accumulates in fp32 from exactly
# decoded weights, so the bound is set by fp32 summation order (~1e-7 for
# these row lengths); 2e-5 leaves two orders of margin while any decode
# mistake (a wrong nibble, scale or element order) costs > 3e-3, as
# tests/test_oracle.py::test_semantic_variants_are_distinguishable shows.
GEMV_TOL = 2e-5
# moe outputs chain three GEMVs and a SiLU; expf differs from glibc by <= 1 ulp.
MOE_TOL = 1e-4
# moe_forward_omp requantises the SiLU output h to Q8_0 before an MXFP4 down
# projection (QK:2166-2189, mxfp4_row_dot_q8).  Any fp32 summation-order
# difference in h (the reference's own AVX order vs ours) flips a few Q8 codes
# by one step, and one flip moves that token's output by about
# 3 / (127 * sqrt(M)) ~ 4e-4 of its max: the bound there is the north star's 1e-3.
MOE_Q8H_TOL = 1e-3


def moe_tol(qts):
    return MOE_Q8H_TOL if qts[2] == 39 else MOE_TOL


def fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def up(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))
