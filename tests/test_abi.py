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


def test_qwen36_and_ssm_refusals_touch_nothing(libpath):
    """Arguments the drop-ins refuse (the reference would write past its KV
    cache, or shapes its stack buffers cannot hold) leave every output
    untouched and record an error -- decided before any device call."""
    import numpy as np
    from mojollama_amd import kernels
    from mojollama_amd import workloads as W
    so = kernels.load_kernels()
    c = W.qwen36_case(0, 2, 0)
    call = W.Qwen36Call(c)
    call.kv_lens[1] = c["max_ctx"]            # an attention layer at max_ctx
    call.logits[:] = 7.0
    st0, ws0 = call.state.copy(), call.ws.copy()
    call.call(so, c["tokens"][0])
    assert (call.logits == 7.0).all() and np.array_equal(call.state, st0) and np.array_equal(call.ws, ws0)
    assert b"kv_lens" in so.mllm_last_error()
    s = W.ssm_case(91, 2, 256, 256)
    out, state = W.ssm_call(so, s, True, gate_nc=288)   # gate columns other than N
    assert np.isnan(out).all() and np.array_equal(state, s["state"])
    assert b"ssm_layer_fused" in so.mllm_last_error()
    s = W.ssm_case(92, 2, 256, 4200)           # 2*inner beyond the reference's 8192-float buffer
    out, state = W.ssm_call(so, s, False)
    assert np.isnan(out).all() and np.array_equal(state, s["state"])
    assert b"ssm_decode_step" in so.mllm_last_error()


def test_attention_rejects_bad_strides(libpath):
    """mllm_gqa_decode / mllm_kv_append refuse a contiguous view whose
    sequence stride is misaligned for the float4 row loads or, with several
    sequences, shorter than a sequence's rows -- before any launch."""
    from mojollama_amd import kernels
    so = kernels.load_kernels()
    fake = 4096   # never dereferenced: the checks come first
    for stride, B, ok_msg in ((6, 1, "multiple of 4"), (-4, 1, "multiple of 4"), (64 * 2 * 64 - 4, 2, "max_seq")):
        kv = kernels.KVView(fake, fake, stride, None, 0, 0, 0)
        r = so.mllm_gqa_decode(0, fake, ctypes.byref(kv), fake, 64, B, 4, 2, 64, fake, fake, 1 << 30, None)
        assert r == -1 and b"seq_stride" in so.mllm_last_error()
    kv = kernels.KVView(fake, fake, 64, None, 0, 0, 0)
    assert so.mllm_kv_append(ctypes.byref(kv), fake, fake, fake, 2, 2, 64, None) == -1
    assert b"seq_stride" in so.mllm_last_error()
