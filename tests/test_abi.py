"""The C-ABI library loads and exports every symbol include/mllm.h declares
(CPU-only: no compute call is made)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mllm.h")


def declared_symbols():
    text = open(HEADER).read()
    return re.findall(r"MLLM_API\s+[\w\s\*]+?\b(\w+)\s*\(", text)


@pytest.fixture(scope="module")
def libpath():
    from mojollama_amd import kernels
    if not os.path.exists(kernels.LIB_PATH):
        kernels.build()
    return kernels.LIB_PATH


def test_header_declares_the_reference_symbols():
    names = set(declared_symbols())
    # the drop-in surface the reference's caller binds (TE:251-392) and the north-star entry points
    for n in ("quant_matmul_omp", "f32_matmul_omp", "batch_qkv_omp", "batch_gate_up_omp", "set_num_threads",
              "moe_forward_omp", "q6_k_dequantize_row", "q4_k_dequantize_row", "ssm_layer_fused",
              "qwen36_batch_forward", "ssm_decode_step", "q4_0_batch_matmul", "q8_0_batch_matmul",
              "q4_k_batch_matmul", "q6_k_batch_matmul", "q5_k_batch_matmul", "mxfp4_batch_matmul", "moe_ffn",
              "quantize_row_q8_0", "get_max_threads"):
        assert n in names, n


def test_library_exports_every_declared_symbol(libpath):
    so = ctypes.CDLL(libpath)
    missing = [n for n in declared_symbols() if not hasattr(so, n)]
    assert not missing, missing


def test_exports_are_exactly_the_declared_ones(libpath):
    out = subprocess.run(["nm", "-D", "--defined-only", libpath], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert exported == set(declared_symbols())


def test_bindings_mirror_reference_argtypes(libpath):
    from mojollama_amd import kernels
    so = kernels.load_kernels()
    cu, cf, ci = kernels.cu, kernels.cf, kernels.ci
    assert so.quant_matmul_omp.argtypes == [cu, cf, cf, ci, ci, ci]          # TE:251
    assert so.f32_matmul_omp.argtypes == [cf, cf, cf, ci, ci]                # TE:253
    assert len(so.moe_forward_omp.argtypes) == 15                             # TE:363-377
    assert so.q4_k_batch_matmul.argtypes == [cu, cf, cf, ci, ci, ci]         # CE:256
