"""ctypes bindings of libmllm_gpu.so.

``load_kernels()`` binds the drop-in symbols with exactly the ``argtypes``
the reference's Python engine uses for its C library
(src/mojollama/kernels/turbo_engine_v7_moe.py:_load_kernels, TE:240-392), so
engine code written against that library runs unchanged on this one.

``DeviceOps`` wraps the mllm_* device-pointer entry points for torch tensors
already on the GPU (the benchmark and batched paths).

There is no CPU fallback: if the library is missing or cannot be loaded,
``load_kernels()`` raises.
"""
import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmllm_gpu.so")

cf = ctypes.POINTER(ctypes.c_float)
cu = ctypes.POINTER(ctypes.c_uint8)
ci = ctypes.c_int
cvp = ctypes.c_void_p

# Semantic ids (mllm_sem, mojollama_amd/csrc/mllm_common.h).
F32, Q4_0, Q4_1, Q5_0_F32, Q5_0_Q8, Q8_0, Q4_K_GGML, Q4_K_Q8 = range(8)
Q5_K_GGML, Q5_K_CE, Q6_K_GGML, Q6_K_LOWNIB, Q6_K_SEQ, MXFP4, MXFP4_CLAMP, MXFP4_Q8 = range(8, 16)
SEM_NAMES = ["F32", "Q4_0", "Q4_1", "Q5_0_F32", "Q5_0_Q8", "Q8_0", "Q4_K_GGML", "Q4_K_Q8",
             "Q5_K_GGML", "Q5_K_CE", "Q6_K_GGML", "Q6_K_LOWNIB", "Q6_K_SEQ", "MXFP4",
             "MXFP4_CLAMP", "MXFP4_Q8"]
# Reference entry points, for mllm_sem_for().
ENT_QMM, ENT_BMM, ENT_ROWS, ENT_MOE_GU, ENT_MOE_DOWN = range(5)


def build(verbose=False):
    """Compile libmllm_gpu.so for gfx950 in-tree (hipcc)."""
    r = subprocess.run(["make", "-s", "-C", os.path.join(HERE, "csrc")], capture_output=not verbose, text=True)
    if r.returncode != 0:
        raise RuntimeError("libmllm_gpu build failed:\n" + (r.stdout or "") + (r.stderr or ""))


class GemvFusion(ctypes.Structure):
    """mllm_gemv_fusion (include/mllm.h): the prologue/epilogue fused into a decode GEMV."""
    _fields_ = [("x_up", cvp), ("silu_clamp", ci), ("x_res", cvp), ("res_out", cvp), ("rms_w", cvp),
                ("rms_eps", ctypes.c_float), ("rms_div", ci), ("out_add", cvp), ("x_ld", ci), ("silu_pair", ci)]


class KVView(ctypes.Structure):
    """mllm_kv_view (include/mllm.h): a contiguous or paged KV cache on the device."""
    _fields_ = [("k", cvp), ("v", cvp), ("seq_stride", ctypes.c_long), ("block_tables", cvp), ("max_blocks", ci),
                ("page_size", ci), ("n_pages", ci)]


ATTN_CE, ATTN_GQA_C = 0, 1   # CE:141-158 gqa / gqa_attention.c:93 softmax


class GptOssDesc(ctypes.Structure):
    """mllm_gptoss_desc (include/mllm.h): host pointers to gptoss_forward's weights."""
    _fields_ = [(n, ci) for n in ("L", "N", "NH", "NKH", "HD", "E", "K", "M", "max_ctx", "rope_dim", "outNR")] + [
        ("eps", ctypes.c_float), ("wQ", ctypes.POINTER(cu)), ("wK", ctypes.POINTER(cu)), ("wV", ctypes.POINTER(cu)),
        ("wO", ctypes.POINTER(cu)), ("wAN", ctypes.POINTER(cf)), ("wFN", ctypes.POINTER(cf)), ("wOut", cu),
        ("w_gate_inp", ctypes.POINTER(cf)), ("w_gate_exps", ctypes.POINTER(cu)), ("w_up_exps", ctypes.POINTER(cu)),
        ("w_down_exps", ctypes.POINTER(cu)), ("qt_gate", ci), ("qt_up", ci), ("qt_down", ci), ("cos_t", cf),
        ("sin_t", cf)]


# The reference caller's bindings of its whole-layer entry points, kept here
# so the drop-in and the reference's own C are called identically:
# ssm_layer_fused (TE:263-271, CE:803-849), qwen36_batch_forward (TE:273-310,
# CE:859-1231) and ssm_decode_step (TE:401-405, CE:736-802).
_pf, _pu, _pi = ctypes.POINTER(cf), ctypes.POINTER(cu), ctypes.POINTER(ci)
SSM_LAYER_FUSED_ARGTYPES = [cf, cf, cf, cf, cf, cf, cf, cf, cf, cf, cu, ci, ci, ci, cu, ci, ci, ci] + [ci] * 7
SSM_DECODE_STEP_ARGTYPES = [cf] * 9 + [ci] * 7
QWEN36_ARGTYPES = (
    [ci] * 7 + [ci, ci, ci, ctypes.c_float] + [ci] * 7        # B, L, N, NH, n_kv_h, HD, FF; E, K, M, eps; rope..dt_rank
    + [cf, ci]                                                # emb, emb_quant
    + [_pi, _pi, cf]                                          # layer_types, tokens, logits
    + [_pf, _pf]                                              # attn_norm_w, ffn_norm_w
    + [_pu, _pi, _pi, _pi] * 4                                # qkv, attn gate, ssm out, attn out: raw, nr, nc, qt
    + [_pu, _pi] * 3                                          # gate/up/down experts, quant types
    + [_pf, _pf, _pf, _pf, _pi]                               # shared expert gate/up/down, router, intermediate
    + [_pu, _pi, _pi, _pi, _pi]                               # moe router + qt, shared expert quant types
    + [cf, cu, ci, ci, ci]                                    # out_norm_w, out_w, nr, nc, qt
    + [_pf] * 6 + [cf]                                        # ssm conv1d, a, dt_bias, alpha, beta, norm; state
    + [cf, cf, _pi, cf, cf]                                   # kv_k, kv_v, kv_lens, cos_table, sin_table
    + [cf, cu])                                               # ws, q8_ws


def bind_model_entry_points(so):
    """Bind ssm_layer_fused / qwen36_batch_forward / ssm_decode_step as TE does."""
    so.ssm_layer_fused.argtypes = SSM_LAYER_FUSED_ARGTYPES
    so.ssm_layer_fused.restype = None
    so.qwen36_batch_forward.argtypes = QWEN36_ARGTYPES
    so.qwen36_batch_forward.restype = None
    so.ssm_decode_step.argtypes = SSM_DECODE_STEP_ARGTYPES
    so.ssm_decode_step.restype = None


_LIB = None


def load_kernels(path=LIB_PATH):
    """Load the library and bind the reference engine's symbols (TE:251-392) plus mllm_*."""
    global _LIB
    if _LIB is not None and path == LIB_PATH:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built: run mojollama_amd.kernels.build() (needs hipcc)")
    # PyTorch-ROCm ships its own libamdhip64.so.7 and links it by another name.
    # Loading torch first makes this library bind to that same runtime, so one
    # HIP runtime serves both (and torch streams are valid handles here).
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    so = ctypes.CDLL(path)
    # --- as bound by TE:251-261, 363-377, 389-392
    so.quant_matmul_omp.argtypes = [cu, cf, cf, ci, ci, ci]
    so.quant_matmul_omp.restype = None
    so.f32_matmul_omp.argtypes = [cf, cf, cf, ci, ci]
    so.f32_matmul_omp.restype = None
    # QK:1139-1145 takes three quant types (TE:255 lists only two: its third is dropped there)
    so.batch_qkv_omp.argtypes = [cu, cu, cu, cf, cf, cf, cf, ci, ci, ci, ci, ci, ci, ci]
    so.batch_qkv_omp.restype = None
    so.batch_gate_up_omp.argtypes = [cu, cu, cf, cf, cf, ci, ci, ci, ci, ci]
    so.batch_gate_up_omp.restype = None
    so.set_num_threads.argtypes = [ci]
    so.set_num_threads.restype = None
    so.moe_forward_omp.argtypes = [ctypes.POINTER(cu), ctypes.POINTER(cu), ctypes.POINTER(cu), cf, ci, ci,
                                   ci, ci, ci, ctypes.POINTER(ctypes.c_int), cf, ci, cf, cf, cu]
    so.moe_forward_omp.restype = None
    for name in ("q6_k_dequantize_row", "q4_k_dequantize_row", "q5_k_dequantize_row", "q8_0_dequantize_row"):
        getattr(so, name).argtypes = [cu, cf, ci]
        getattr(so, name).restype = None
    # --- the engine's other kernel entry points (CE:68-534, 591; QK:1406, 1029)
    for name in ("q4_0_batch_matmul", "q8_0_batch_matmul", "q4_k_batch_matmul", "q6_k_batch_matmul",
                 "q5_k_batch_matmul", "mxfp4_batch_matmul"):
        getattr(so, name).argtypes = [cu, cf, cf, ci, ci, ci]
        getattr(so, name).restype = None
    bind_model_entry_points(so)
    so.moe_ffn.argtypes = [cvp, ci, cf, cf, cf, cf, ci]
    so.moe_ffn.restype = None
    so.moe_ffn_batched.argtypes = [cvp, ci, cf, cf, ci]
    so.moe_ffn_batched.restype = None
    so.quantize_row_q8_0.argtypes = [cf, cu, ci]
    so.quantize_row_q8_0.restype = ci
    so.get_max_threads.argtypes = []
    so.get_max_threads.restype = ci
    so.mllm_last_error.argtypes = []
    so.mllm_last_error.restype = ctypes.c_char_p
    so.mllm_cache_clear.argtypes = []
    so.mllm_cache_clear.restype = None
    # --- device-pointer API
    so.mllm_sem_for.argtypes = [ci, ci]
    so.mllm_sem_for.restype = ci
    so.mllm_raw_size.argtypes = [ci, ci, ci]
    so.mllm_raw_size.restype = ctypes.c_long
    so.mllm_packed_size.argtypes = [ci, ci, ci]
    so.mllm_packed_size.restype = ctypes.c_long
    so.mllm_pack.argtypes = [ci, cvp, cvp, ci, ci, cvp]
    so.mllm_pack.restype = ci
    so.mllm_gemv_workspace_size.argtypes = [ci, ci, ci, ci]
    so.mllm_gemv_workspace_size.restype = ctypes.c_long
    so.mllm_gemv.argtypes = [ci, cvp, cvp, cvp, ci, ci, ci, cvp, cvp]
    so.mllm_gemv.restype = ci
    so.mllm_gemv_fused_workspace_size.argtypes = [ci, ci, ci, ci, ctypes.POINTER(GemvFusion)]
    so.mllm_gemv_fused_workspace_size.restype = ctypes.c_long
    so.mllm_gemv_fused.argtypes = [ci, cvp, cvp, cvp, ci, ci, ci, ctypes.POINTER(GemvFusion), cvp, cvp]
    so.mllm_gemv_fused.restype = ci
    so.requantize_output_q8_0.argtypes = [cu, ci, ci, ci, cu]
    so.requantize_output_q8_0.restype = ci
    so.mllm_requantize_workspace_size.argtypes = [ci, ci, ci]
    so.mllm_requantize_workspace_size.restype = ctypes.c_long
    so.mllm_requantize_q8_0.argtypes = [ci, cvp, ci, ci, cvp, cvp, cvp]
    so.mllm_requantize_q8_0.restype = ci
    so.mllm_read_probe.argtypes = [cvp, ctypes.c_long, cvp, cvp]
    so.mllm_read_probe.restype = ci
    so.mllm_quantize_q8_0.argtypes = [cvp, ci, ci, cvp, cvp]
    so.mllm_quantize_q8_0.restype = ci
    so.mllm_router_packed_size.argtypes = [ci, ci]
    so.mllm_router_packed_size.restype = ctypes.c_long
    so.mllm_router_pack.argtypes = [cvp, ci, ci, cvp, cvp]
    so.mllm_router_pack.restype = ci
    so.mllm_route_workspace_size.argtypes = [ci, ci]
    so.mllm_route_workspace_size.restype = ctypes.c_long
    so.mllm_route.argtypes = [cvp, cvp, ci, ci, ci, ci, ci, cvp, cvp, cvp, cvp]
    so.mllm_route.restype = ci
    so.mllm_dequant.argtypes = [ci, cvp, ci, ci, cvp, cvp]
    so.mllm_dequant.restype = ci
    so.mllm_moe_dense_experts.argtypes = [cvp, cvp]
    so.mllm_moe_dense_experts.restype = ctypes.c_long
    so.mllm_moe_prepare.argtypes = [ci, ci, ci, ci, ci, ci, ci, ctypes.POINTER(cvp), ctypes.POINTER(cvp),
                                    ctypes.POINTER(cvp), cvp, ci]
    so.mllm_moe_prepare.restype = cvp
    so.mllm_moe_release.argtypes = [cvp]
    so.mllm_moe_release.restype = None
    so.mllm_moe_workspace_size.argtypes = [cvp, ci]
    so.mllm_moe_workspace_size.restype = ctypes.c_long
    so.mllm_moe_layer_info.argtypes = [cvp]
    so.mllm_moe_layer_info.restype = ci
    so.mllm_moe_forward.argtypes = [cvp, cvp, ci, cvp, cvp, ctypes.c_long, cvp, cvp, cvp]
    so.mllm_moe_forward.restype = ci
    so.mllm_moe_forward_noalloc.argtypes = [cvp, cvp, ci, cvp, cvp, cvp, cvp]
    so.mllm_moe_forward_noalloc.restype = ci
    so.mllm_moe_bucket.argtypes = [cvp, ci, ci, cvp, cvp, cvp, cvp, cvp]
    so.mllm_moe_bucket.restype = ci
    # --- decode attention and the KV cache (TE:383-385 binds gqa_attention_decode so)
    so.gqa_attention_decode.argtypes = [cf, cf, cf, cf, ci, ci, ci, ci, cf]
    so.gqa_attention_decode.restype = None
    so.mllm_gqa_workspace_size.argtypes = [ci, ci, ci, ci]
    so.mllm_gqa_workspace_size.restype = ctypes.c_long
    so.mllm_gqa_decode.argtypes = [ci, cvp, ctypes.POINTER(KVView), cvp, ci, ci, ci, ci, ci, cvp, cvp, ctypes.c_long,
                                   cvp]
    so.mllm_gqa_decode.restype = ci
    so.mllm_kv_append.argtypes = [ctypes.POINTER(KVView), cvp, cvp, cvp, ci, ci, ci, cvp]
    so.mllm_kv_append.restype = ci
    so.mllm_rope.argtypes = [cvp, ci, ci, ci, cvp, cvp, cvp, ci, cvp]
    so.mllm_rope.restype = ci
    # gptoss_forward (GO:96-130 argument list)
    pcu, pcf, pci = ctypes.POINTER(cu), ctypes.POINTER(cf), ctypes.POINTER(ci)
    so.gptoss_forward.argtypes = ([pci, ci, cf, ci] + [pcu] * 4 + [pcf] * 2 + [pci] * 8 + [cu, ci, ci, ci, cf, cf, pci,
                                  cf, cf, ci, ci, cf, ci] + [ci] * 6 + [ctypes.c_float] + [ci] * 3 + [pcf] +
                                  [pcu] * 3 + [ci] * 3 + [cf, cf, cu, cf])
    so.gptoss_forward.restype = None
    so.mllm_gptoss_create.argtypes = [cvp]
    so.mllm_gptoss_create.restype = cvp
    so.mllm_gptoss_release.argtypes = [cvp]
    so.mllm_gptoss_release.restype = None
    so.mllm_gptoss_kv_floats.argtypes = [cvp]
    so.mllm_gptoss_kv_floats.restype = ctypes.c_long
    so.mllm_gptoss_step.argtypes = [cvp, cvp, cvp, cvp, cvp, cvp, cvp, cvp]
    so.mllm_gptoss_step.restype = ci
    so.mllm_page_table_create.argtypes = [ci, ci]
    so.mllm_page_table_create.restype = cvp
    so.mllm_page_table_destroy.argtypes = [cvp]
    so.mllm_page_table_destroy.restype = None
    so.mllm_page_table_alloc.argtypes = [cvp]
    so.mllm_page_table_alloc.restype = ci
    so.mllm_page_table_free.argtypes = [cvp, ci]
    so.mllm_page_table_free.restype = None
    so.mllm_page_table_map.argtypes = [cvp, ci, ci]
    so.mllm_page_table_map.restype = None
    so.mllm_page_table_lookup.argtypes = [cvp, ci]
    so.mllm_page_table_lookup.restype = ci
    so.mllm_page_table_entries.argtypes = [cvp]
    so.mllm_page_table_entries.restype = ctypes.POINTER(ci)
    if path == LIB_PATH:
        _LIB = so
    return so


def last_error(so=None):
    so = so or load_kernels()
    return so.mllm_last_error().decode()


class DeviceOps:
    """mllm_* calls on torch tensors that live on the current GPU."""

    def __init__(self, so=None):
        import torch
        self.torch = torch
        self.so = so or load_kernels()

    def _stream(self):
        return ctypes.c_void_p(self.torch.cuda.current_stream().cuda_stream)

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {last_error(self.so)}")

    def pack(self, sem, raw_dev, n_rows, n_cols):
        """raw GGUF bytes (uint8 tensor on GPU) -> packed uint8 tensor."""
        torch = self.torch
        n = self.so.mllm_packed_size(sem, n_rows, n_cols)
        packed = torch.empty(n, dtype=torch.uint8, device=raw_dev.device)
        self._check(self.so.mllm_pack(sem, raw_dev.data_ptr(), packed.data_ptr(), n_rows, n_cols, self._stream()),
                    "mllm_pack")
        return packed

    def workspace(self, sem, n_cols, B, device, n_rows=0):
        n = self.so.mllm_gemv_workspace_size(sem, n_rows, n_cols, B)
        return self.torch.empty(max(n, 256), dtype=self.torch.uint8, device=device) if n > 0 else None

    def gemv(self, sem, packed, x, n_rows, n_cols, out=None, ws=None):
        torch = self.torch
        B = x.numel() // n_cols
        if out is None:
            out = torch.empty((B, n_rows), dtype=torch.float32, device=x.device)
        if ws is None:
            ws = self.workspace(sem, n_cols, B, x.device, n_rows)
        self._check(self.so.mllm_gemv(sem, packed.data_ptr(), x.data_ptr(), out.data_ptr(), n_rows, n_cols, B,
                                      ws.data_ptr() if ws is not None else None, self._stream()), "mllm_gemv")
        return out

    def fusion(self, x_up=None, silu_clamp=True, x_res=None, res_out=None, rms_w=None, rms_eps=1e-6, rms_div=False,
               out_add=None, x_ld=0, silu_pair=False):
        """An mllm_gemv_fusion over torch tensors or device addresses (None = field unused)."""
        p = lambda t: (t if isinstance(t, int) else t.data_ptr()) if t is not None else None  # noqa: E731
        return GemvFusion(p(x_up), int(silu_clamp), p(x_res), p(res_out), p(rms_w), float(rms_eps), int(rms_div),
                          p(out_add), int(x_ld), int(silu_pair))

    def gemv_fused(self, sem, packed, x, n_rows, n_cols, fusion, out=None, ws=None, B=None):
        """mllm_gemv_fused: y = W * prologue(x) (+ out_add), one launch where it fits.
        x: a tensor, or a device address with B given (a strided view inside a wider row)."""
        torch = self.torch
        if B is None:
            B = x.numel() // n_cols
        xp = x if isinstance(x, int) else x.data_ptr()
        dev = torch.device("cuda")
        if out is None:
            out = torch.empty((B, n_rows), dtype=torch.float32, device=dev)
        if ws is None:
            n = self.so.mllm_gemv_fused_workspace_size(sem, n_rows, n_cols, B, ctypes.byref(fusion))
            ws = torch.empty(max(n, 256), dtype=torch.uint8, device=dev) if n > 0 else None
        self._check(self.so.mllm_gemv_fused(sem, packed.data_ptr(), xp, out.data_ptr(), n_rows, n_cols, B,
                                            ctypes.byref(fusion), ws.data_ptr() if ws is not None else None,
                                            self._stream()), "mllm_gemv_fused")
        return out

    def quantize_q8_0(self, x, n_cols):
        torch = self.torch
        T = x.numel() // n_cols
        q8 = torch.empty(T * (n_cols // 32) * 34, dtype=torch.uint8, device=x.device)
        self._check(self.so.mllm_quantize_q8_0(x.data_ptr(), T, n_cols, q8.data_ptr(), self._stream()),
                    "mllm_quantize_q8_0")
        return q8

    def router_pack(self, router):
        """fp32 router [E][N] (device) -> the routing layout (mllm_router_pack)."""
        torch = self.torch
        E, N = router.shape
        out = torch.empty(self.so.mllm_router_packed_size(N, E) // 4, dtype=torch.float32, device=router.device)
        self._check(self.so.mllm_router_pack(router.data_ptr(), N, E, out.data_ptr(), self._stream()),
                    "mllm_router_pack")
        return out

    def route(self, router, x, K, renorm, packed=None, slices=True):
        """Top-K routing of x [T][N] by the fp32 router [E][N] (device); slices=False
        keeps one workgroup per token at T <= 8 (no workspace)."""
        torch = self.torch
        E, N = router.shape
        rp = self.router_pack(router) if packed is None else packed
        T = x.numel() // N
        idx = torch.empty((T, K), dtype=torch.int32, device=x.device)
        w = torch.empty((T, K), dtype=torch.float32, device=x.device)
        ws = torch.empty(self.so.mllm_route_workspace_size(T, E) // 4, dtype=torch.float32, device=x.device) \
            if slices else None
        self._check(self.so.mllm_route(rp.data_ptr(), x.data_ptr(), T, N, E, K, int(renorm), idx.data_ptr(),
                                       w.data_ptr(), ws.data_ptr() if ws is not None else None, self._stream()),
                    "mllm_route")
        return idx, w

    def dequant(self, sem, packed, n_rows, n_cols):
        torch = self.torch
        out = torch.empty((n_rows, n_cols), dtype=torch.float32, device=packed.device)
        self._check(self.so.mllm_dequant(sem, packed.data_ptr(), n_rows, n_cols, out.data_ptr(), self._stream()),
                    "mllm_dequant")
        return out

    # ------------------------------------------------------------ MoE layer
    def kv_view(self, k, v, seq_stride=0, block_tables=None, page_size=0, n_pages=0):
        """An mllm_kv_view over fp32 GPU tensors k, v (block_tables: int32 [B][max_blocks] GPU).
        The view keeps the tensors alive."""
        view = KVView(k.data_ptr(), v.data_ptr(), int(seq_stride),
                      block_tables.data_ptr() if block_tables is not None else None,
                      int(block_tables.shape[-1]) if block_tables is not None else 0, int(page_size), int(n_pages))
        view._tensors = (k, v, block_tables)
        return view

    def gqa_decode(self, mode, q, kv, seq_lens, max_seq, NH, NKH, HD, out=None, ws=None):
        """mllm_gqa_decode: q [B][NH*HD] fp32, seq_lens int32 [B] (GPU)."""
        torch = self.torch
        B = q.numel() // (NH * HD)
        if out is None:
            out = torch.empty((B, NH * HD), dtype=torch.float32, device=q.device)
        n = self.so.mllm_gqa_workspace_size(B, NH, HD, max_seq)
        if ws is None:
            ws = torch.empty(n, dtype=torch.uint8, device=q.device)
        self._check(self.so.mllm_gqa_decode(mode, q.data_ptr(), ctypes.byref(kv), seq_lens.data_ptr(), max_seq, B, NH,
                                            NKH, HD, out.data_ptr(), ws.data_ptr(), ws.numel(), self._stream()),
                    "mllm_gqa_decode")
        return out

    def kv_append(self, kv, pos, k_new, v_new, NKH, HD):
        B = pos.numel()
        self._check(self.so.mllm_kv_append(ctypes.byref(kv), pos.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), B,
                                           NKH, HD, self._stream()), "mllm_kv_append")

    def rope(self, buf, NH, HD, pos, cos_t, sin_t, rope_dim=0):
        T = pos.numel()
        self._check(self.so.mllm_rope(buf.data_ptr(), T, NH, HD, pos.data_ptr(), cos_t.data_ptr(), sin_t.data_ptr(),
                                      rope_dim, self._stream()), "mllm_rope")
        return buf

    def moe_prepare(self, qts, N, M, E, K, gates, ups, downs, router, renorm):
        """gates/ups/downs: per-expert raw GGUF uint8 tensors (GPU) in the
        reference's layout; router: fp32 [E][N] (GPU).  Returns a MoELayer."""
        return MoELayer(self, qts, N, M, E, K, gates, ups, downs, router, renorm)

    def moe_bucket(self, idx, E):
        """Stable bucketing of entries idx (int32 GPU, flat) over E experts."""
        torch = self.torch
        TK = idx.numel()
        max_tiles = TK // 64 + E + 1
        off = torch.empty(E + 1, dtype=torch.int32, device=idx.device)
        perm = torch.empty(TK, dtype=torch.int32, device=idx.device)
        pos_of = torch.empty(TK, dtype=torch.int32, device=idx.device)
        tiles = torch.empty(3 * max_tiles + 1, dtype=torch.int32, device=idx.device)
        self._check(self.so.mllm_moe_bucket(idx.data_ptr(), TK, E, off.data_ptr(), perm.data_ptr(), pos_of.data_ptr(),
                                            tiles.data_ptr(), self._stream()), "mllm_moe_bucket")
        n = int(tiles[3 * max_tiles].item())
        return off, perm, pos_of, (tiles[:n], tiles[max_tiles:max_tiles + n], tiles[2 * max_tiles:2 * max_tiles + n])


class MoELayer:
    """A prepared MoE layer (mllm_moe_prepare) holding its packed expert weights."""

    def __init__(self, ops, qts, N, M, E, K, gates, ups, downs, router, renorm):
        torch = ops.torch
        self.ops, self.N, self.M, self.E, self.K = ops, N, M, E, K
        sg = ops.so.mllm_sem_for(ENT_MOE_GU, qts[0]) if not (qts[0] == 39 and qts[1] == 39) else MXFP4
        su = ops.so.mllm_sem_for(ENT_MOE_GU, qts[1]) if not (qts[0] == 39 and qts[1] == 39) else MXFP4
        sd = ops.so.mllm_sem_for(ENT_MOE_DOWN, qts[2])
        self.gp = [ops.pack(sg, g, M, N) for g in gates]
        self.up = [ops.pack(su, u, M, N) for u in ups]
        self.dp = [ops.pack(sd, d, N, M) for d in downs] if sd >= 0 else [self.gp[0]] * E
        self.router = router.contiguous()
        arr = ctypes.c_void_p * E
        self.h = ops.so.mllm_moe_prepare(qts[0], qts[1], qts[2], N, M, E, K,
                                         arr(*[t.data_ptr() for t in self.gp]), arr(*[t.data_ptr() for t in self.up]),
                                         arr(*[t.data_ptr() for t in self.dp]), self.router.data_ptr(), int(renorm))
        if not self.h:
            raise RuntimeError("mllm_moe_prepare failed")
        self._ws = None

    def dense_experts(self):
        """Load-time bf16 copies of the bf16-exact expert matrices (mllm_moe_dense_experts);
        returns the bytes they take (0: no matrix of this layer qualifies)."""
        n = self.ops.so.mllm_moe_dense_experts(self.h, self.ops._stream())
        if n < 0:
            raise RuntimeError("mllm_moe_dense_experts failed: " + last_error(self.ops.so))
        return n

    def info(self):
        """mllm_moe_layer_info: bit 1 gate/up and bit 2 down on the fp16-plane GEMM,
        bit 4 the whole layer on the per-token GEMVs."""
        return self.ops.so.mllm_moe_layer_info(self.h)

    def workspace(self, T):
        n = self.ops.so.mllm_moe_workspace_size(self.h, T)
        if self._ws is None or self._ws.numel() < n:
            self._ws = self.ops.torch.empty(n, dtype=self.ops.torch.uint8, device=self.router.device)
        return self._ws

    def forward(self, x, out=None, idx=None, w=None):
        torch = self.ops.torch
        T = x.numel() // self.N
        if out is None:
            out = torch.empty((T, self.N), dtype=torch.float32, device=x.device)
        ws = self.workspace(T)
        self.ops._check(self.ops.so.mllm_moe_forward(self.h, x.data_ptr(), T, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                                     idx.data_ptr() if idx is not None else None,
                                                     w.data_ptr() if w is not None else None, self.ops._stream()),
                        "mllm_moe_forward")
        return out

    def __del__(self):
        try:
            if self.h:
                self.ops.so.mllm_moe_release(self.h)
        except Exception:
            pass
