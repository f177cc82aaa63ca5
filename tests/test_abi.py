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


def test_gqa_binding_mirrors_te(libpath):
    from mojollama_amd import kernels
    so = kernels.load_kernels()
    cf, ci = kernels.cf, kernels.ci
    assert so.gqa_attention_decode.argtypes == [cf, cf, cf, cf, ci, ci, ci, ci, cf]   # TE:383-385


def test_page_table_follows_ce(libpath):
    """CE:173-201 (host code, no GPU): allocation hands out 0, 1, 2, ...; a freed
    page is handed out next; exhaustion gives -1; the logical map has 1024
    entries (MAX_BLOCKS, CE:23), -1 when unmapped, and ignores indices outside."""
    from mojollama_amd import kernels
    so = kernels.load_kernels()
    pt = so.mllm_page_table_create(5, 64)
    try:
        assert [so.mllm_page_table_alloc(pt) for _ in range(3)] == [0, 1, 2]
        so.mllm_page_table_free(pt, 1)
        assert so.mllm_page_table_alloc(pt) == 1
        assert [so.mllm_page_table_alloc(pt) for _ in range(3)] == [3, 4, -1]
        so.mllm_page_table_map(pt, 7, 3)
        so.mllm_page_table_map(pt, 1024, 2)
        so.mllm_page_table_map(pt, -1, 2)
        assert so.mllm_page_table_lookup(pt, 7) == 3
        assert so.mllm_page_table_lookup(pt, 8) == -1
        ent = so.mllm_page_table_entries(pt)
        assert [ent[i] for i in range(1024)].count(-1) == 1023 and ent[7] == 3
        for _ in range(10):
            so.mllm_page_table_free(pt, 0)          # the free list never grows past n_pages
        assert [so.mllm_page_table_alloc(pt) for _ in range(6)] == [0] * 5 + [-1]
    finally:
        so.mllm_page_table_destroy(pt)
    assert so.mllm_page_table_create(0, 64) is None
