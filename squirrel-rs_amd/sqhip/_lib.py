"""Loads libsquirrel_hip.so and declares the C ABI (include/squirrel_hip.h).

There is no fallback: if the library is missing the import fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("SQHIP_LIB", os.path.join(PKG_DIR, "libsquirrel_hip.so"))

SQ_OK = 0
SQ_ERR_SHAPE, SQ_ERR_INVALID_TYPE, SQ_ERR_EMPTY, SQ_ERR_ALIGN = 1, 2, 3, 4
SQ_ERR_IO, SQ_ERR_FORMAT, SQ_ERR_CONFIG, SQ_ERR_WEIGHTS = 16, 17, 18, 19
SQ_ERR_UNSUPPORTED, SQ_ERR_CACHE_FULL, SQ_ERR_ARG, SQ_ERR_HIP = 20, 21, 22, 64
SQ_F32, SQ_Q4_0, SQ_Q8_0, SQ_BF16 = 0, 2, 8, 30
SQ_CTX_F32_ACTS, SQ_CTX_NO_GRAPH, SQ_CTX_MULTI_KERNEL = 1, 2, 4
SQ_GEN_IGNORE_EOS, SQ_GEN_NO_KV_CACHE = 1, 2


class SynthSpec(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("dim", C.c_uint32), ("ffn_dim", C.c_uint32),
                ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("vocab", C.c_uint32),
                ("context_length", C.c_uint32), ("wtype", C.c_uint32), ("seed", C.c_uint64),
                ("std_dev", C.c_float), ("rope_base", C.c_float), ("rms_eps", C.c_float),
                ("bos", C.c_uint32), ("eos", C.c_uint32)]


class ModelInfo(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("dim", C.c_uint32), ("ffn_dim", C.c_uint32),
                ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
                ("vocab", C.c_uint32), ("context_length", C.c_uint32), ("bos", C.c_uint32),
                ("eos", C.c_uint32), ("wtype", C.c_uint32), ("tied_output", C.c_uint32),
                ("rope_base", C.c_float), ("rms_eps", C.c_float), ("weight_bytes", C.c_uint64)]


vp, sz, i32, u32, f32 = C.c_void_p, C.c_size_t, C.c_int, C.c_uint32, C.c_float
PROTOS = {
    "sq_last_error": ([], C.c_char_p),
    "sq_version": ([], C.c_char_p),
    "sq_device_count": ([C.POINTER(i32)], i32),
    "sq_malloc": ([C.POINTER(vp), sz], i32),
    "sq_free": ([vp], i32),
    "sq_memcpy_h2d": ([vp, vp, sz], i32),
    "sq_memcpy_d2h": ([vp, vp, sz], i32),
    "sq_memset": ([vp, i32, sz], i32),
    "sq_synchronize": ([], i32),
    "sq_synth_write_gguf": ([C.c_char_p, C.POINTER(SynthSpec)], i32),
    "sq_gguf_inspect": ([C.c_char_p, C.POINTER(ModelInfo), vp, sz], i32),
    "sq_model_load_gguf": ([C.c_char_p, C.POINTER(vp)], i32),
    "sq_model_info_get": ([vp, C.POINTER(ModelInfo)], i32),
    "sq_model_rope_inv_freq": ([vp, vp, sz], i32),
    "sq_model_free": ([vp], None),
    "sq_ctx_new": ([vp, sz, u32, C.POINTER(vp)], i32),
    "sq_ctx_free": ([vp], None),
    "sq_ctx_reset": ([vp], i32),
    "sq_ctx_seq_len": ([vp], sz),
    "sq_ctx_act_taps": ([vp, i32], i32),
    "sq_ctx_act_tap_read": ([vp, vp, sz], i32),
    "sq_ctx_decode_kernel": ([vp], i32),
    "sq_ctx_step_trace": ([vp, i32], i32),
    "sq_ctx_step_trace_read": ([vp, vp, sz, C.POINTER(i32), C.POINTER(i32)], i32),
    "sq_forward": ([vp, vp, vp, sz], i32),
    "sq_logits": ([vp, vp, sz], i32),
    "sq_argmax": ([vp, C.POINTER(u32)], i32),
    "sq_ctx_last_hidden": ([vp, vp, sz], i32),
    "sq_ctx_debug_act": ([vp, vp, vp], i32),
    "sq_generate": ([vp, vp, vp, sz, sz, u32, vp, C.POINTER(sz), vp], i32),
    "sq_weight_upload": ([i32, vp, sz, sz, C.POINTER(vp)], i32),
    "sq_weight_free": ([vp], None),
    "sq_quantize_row_q8_0": ([vp, sz, vp], i32),
    "sq_linear": ([vp, sz, sz, vp, vp, u32], i32),
    "sq_linear_noalloc": ([vp, sz, sz, vp, vp, u32], i32),
    "sq_linear_shared": ([vp, sz, sz, vp, vp, sz, u32], i32),
    "sq_block_isums": ([vp, vp, sz, vp], i32),
    "sq_embed": ([vp, sz, vp, vp], i32),
    "sq_rms_norm": ([vp, vp, vp, sz, sz, f32], i32),
    "sq_rope_rows": ([vp, sz, sz, sz, vp, sz], i32),
    "sq_sdpa": ([vp, vp, vp, vp, sz, sz, sz, sz, sz], i32),
    "sq_silu": ([vp, sz], i32),
    "sq_elementwise_mul": ([vp, vp, vp, sz], i32),
    "sq_elementwise_add": ([vp, vp, sz], i32),
    "sq_greedy": ([vp, sz, C.POINTER(u32)], i32),
    "sq_softmax": ([vp, vp, sz], i32),
    "sq_ctx_time_kernel": ([vp, i32, i32, C.POINTER(C.c_double), C.POINTER(C.c_uint64)], i32),
    "sq_ctx_score": ([vp, vp, sz, sz, vp], i32),
    "sq_gemm_counters": ([i32, vp], i32),
    "sq_device_wall_clock_khz": ([vp], i32),
    "sq_log_softmax_at": ([vp, sz, u32, vp], i32),
    "sq_ctx_prefill_phases": ([vp, vp, sz, vp], i32),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it first (python squirrel-rs_amd/build.py)")
        L = C.CDLL(LIB_PATH)
        for name, (args, res) in PROTOS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


class SqError(Exception):
    """A non-zero status from the library, with sq_last_error()'s message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class KernelError(SqError):
    """Codes 1..4: KernelError (src/kernels/kernel_error.rs:2-7)."""

    NAMES = {1: "ShapeMismatch", 2: "InvalidType", 3: "EmptyInput", 4: "TensorAlignmentError"}

    @property
    def kind(self) -> str:
        return self.NAMES[self.code]


class LLMError(SqError):
    """Load-path errors: config, weights, file format (models/common/error.rs:5-10)."""


def check(code: int) -> None:
    if code == SQ_OK:
        return
    msg = lib().sq_last_error().decode(errors="replace")
    if 1 <= code <= 4:
        raise KernelError(code, msg)
    if 16 <= code < 64:
        raise LLMError(code, msg)
    raise SqError(code, msg)
