"""Shared test helpers: the BC struct view moe_ffn reads, and tolerances."""
import ctypes

import numpy as np

# moe_ffn reads these BC fields (x86-64 offsets of the engine's struct, CE:536-589).
BC_SIZE, BC_N, BC_NE, BC_NK, BC_M = 736, 4, 224, 228, 232
BC_ROUTER, BC_GATE, BC_UP, BC_DOWN, BC_QG, BC_QU, BC_QD = 240, 248, 256, 264, 272, 276, 280


class BCView:
    """A zeroed BC-sized buffer with the moe_ffn fields of layer 0 filled in."""

    def __init__(self, N, E, K, M, router, gate, upw, down, qts):
        self.buf = (ctypes.c_uint64 * (BC_SIZE // 8))()
        base = ctypes.addressof(self.buf)
        self.keep = [router, gate, upw, down]
        self.pr = (ctypes.c_void_p * 1)(router.ctypes.data)
        self.pg = (ctypes.c_void_p * 1)(gate.ctypes.data)
        self.pu = (ctypes.c_void_p * 1)(upw.ctypes.data)
        self.pd = (ctypes.c_void_p * 1)(down.ctypes.data)
        for off, v in ((BC_N, N), (BC_NE, E), (BC_NK, K), (BC_M, M),
                       (BC_QG, qts[0]), (BC_QU, qts[1]), (BC_QD, qts[2])):
            ctypes.c_int.from_address(base + off).value = v
        for off, p in ((BC_ROUTER, self.pr), (BC_GATE, self.pg), (BC_UP, self.pu), (BC_DOWN, self.pd)):
            ctypes.c_void_p.from_address(base + off).value = ctypes.addressof(p)

    def ptr(self):
        return ctypes.addressof(self.buf)


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
