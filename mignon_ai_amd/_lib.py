"""ctypes binding of the C ABI in include/mignon_hip.h (library: mignon_ai_amd/_build/libmignon_hip.so).

There is no fallback: if the library is missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libmignon_hip.so")

MG_OK = 0
MG_ERR_INVALID = -1
MG_ERR_FORMAT = -2
MG_ERR_DEVICE = -3
MG_ERR_NOMEM = -4
MG_ERR_UNSUPPORTED = -5
MG_PTR_DEVICE = 1
MG_OPT_GEMM_KERNEL, MG_OPT_ATTENTION_KERNEL, MG_OPT_SCAN_KERNEL = 0, 1, 2
MG_GEMM_STREAM, MG_GEMM_SLAB = 1, 2
MG_ATTN_EXACT, MG_ATTN_MFMA, MG_ATTN_FUSED = 1, 2, 3
MG_SCAN_SEPARATE, MG_SCAN_FUSED = 1, 2
MG_OPT_STEP_GRAPH, MG_STEP_EAGER, MG_STEP_GRAPH = 3, 1, 2
MG_OPT_STEP_KERNEL, MG_STEP_LAYERED, MG_STEP_FUSED, MG_STEP_TILED = 4, 1, 2, 3
MG_OPT_OPERANDS, MG_OPERANDS_LIMBS, MG_OPERANDS_FP32 = 5, 1, 2
MG_OPT_KV_RINGS, MG_KV_FP32, MG_KV_PACKED = 6, 1, 2

_vp = ctypes.c_void_p
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_int = ctypes.c_int
_ll = ctypes.c_longlong


class ModelInfo(ctypes.Structure):
    _fields_ = [("vocab_size", _int), ("state_size", _int), ("hidden_size", _int), ("num_blocks", _int),
                ("attn_heads", _int), ("attn_window", _int), ("max_context", _int), ("tied_embed", _int),
                ("norm_ring", _int), ("attn_cache", _int), ("num_params", _ll)]


class Sampling(ctypes.Structure):
    """mg_sampling_t: generate.Sampling's numeric fields."""
    _fields_ = [("temperature", ctypes.c_double), ("rep_penalty", ctypes.c_double), ("top_p", ctypes.c_double),
                ("top_k", _int), ("penalize_prompt", _int)]


class HeldOut(ctypes.Structure):
    """eval.HeldOut (internal/eval/eval.go:12-17)."""
    _fields_ = [("loss", ctypes.c_double), ("ppl", ctypes.c_double), ("bpb", ctypes.c_double), ("tokens", _ll)]


class KernelTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 32), ("launches", _ll), ("total_ms", ctypes.c_double),
                ("bytes", ctypes.c_double), ("ops", ctypes.c_double)]


# name -> (restype, argtypes); the exported set of include/mignon_hip.h
SIGNATURES = {
    "mg_last_error": (ctypes.c_char_p, []),
    "mg_model_load": (_int, [_u8p, ctypes.c_size_t, _int, ctypes.POINTER(_vp)]),
    "mg_model_file_info": (_int, [_u8p, ctypes.c_size_t, _int, ctypes.POINTER(ModelInfo)]),
    "mg_model_info": (_int, [_vp, ctypes.POINTER(ModelInfo)]),
    "mg_model_set_stream": (_int, [_vp, _vp]),
    "mg_model_stream": (_vp, [_vp]),
    "mg_model_sync": (_int, [_vp]),
    "mg_model_set_cancel": (_int, [_vp, _vp]),
    "mg_model_profile": (_int, [_vp, _int]),
    "mg_model_profile_read": (_int, [_vp, _vp, _int]),
    "mg_model_free": (None, [_vp]),
    "mg_model_call": (_int, [_vp, _vp, _int, _vp]),
    "mg_forward_batch": (_int, [_vp, _vp, _int, _int, _vp, _vp, _vp, _vp, _int]),
    "mg_sessions_create": (_int, [_vp, _int, _int, ctypes.POINTER(_vp)]),
    "mg_sessions_prefill": (_int, [_vp, _vp, _vp, _int, _vp, _vp, _vp, _int]),
    "mg_sessions_step": (_int, [_vp, _vp, _vp, _vp, _vp, _int]),
    "mg_sessions_step_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp]),
    "mg_sessions_decode_greedy": (_int, [_vp, _vp, _vp, _int, _int, _vp, _vp, _int]),
    "mg_sessions_decode_greedy_until": (_int, [_vp, _vp, _vp, _int, _int, _vp, _int, _vp, _vp, _vp, _int]),
    "mg_sessions_state_bytes": (_ll, [_vp]),
    "mg_sessions_device_bytes": (_ll, [_vp]),
    "mg_sessions_count": (_int, [_vp]),
    "mg_sessions_free": (None, [_vp]),
    "mg_gemm_i8": (_int, [_vp, _int, _int, _vp, _int, _vp, _vp, _vp, _int, _vp]),
    "mg_quantize_f32": (_int, [_vp, _ll, _vp, _vp, _int, _vp]),
    "mg_engine_option": (_int, [_int, _int]),
    "mg_score_sequences": (_int, [_vp, _vp, _vp, _int, _int, _vp]),
    "mg_tokenizer_load": (_int, [_u8p, ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "mg_tokenizer_free": (None, [_vp]),
    "mg_tokenizer_vocab_size": (_int, [_vp]),
    "mg_tokenizer_special": (_int, [_vp, _int]),
    "mg_tokenizer_encode": (_ll, [_vp, ctypes.c_char_p, ctypes.c_size_t, _int, _vp, _ll]),
    "mg_tokenizer_decode": (_ll, [_vp, _vp, _ll, _vp, _ll]),
    "mg_tokenizer_decode_rows": (_ll, [_vp, _vp, _vp, _int, _int, _int, _vp, _ll, _vp]),
    "mg_tokenizer_token": (_ll, [_vp, _int, _vp, _ll]),
    "mg_tokenizer_token_bytes": (_int, [_vp, _vp]),
    "mg_pretokenize": (_ll, [ctypes.c_char_p, ctypes.c_size_t, _vp, _ll]),
    "mg_generate_greedy": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp, _vp, _vp]),
    "mg_perplexity": (_int, [_vp, _vp, ctypes.c_char_p, ctypes.c_size_t, _int, _int, _int, _vp]),
    "mg_sample_logits": (_int, [_vp, _int, _int, _vp, _vp, _int, _vp, _vp, _vp]),
    "mg_sessions_decode_sample": (_int, [_vp, _vp, _vp, _int, _int, _vp, _vp, _vp, _int, _vp, _vp, _int]),
    "mg_generate_sample": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp, _vp, _vp, _vp]),
}

_lib = None


class MignonError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP engine library not built: {LIB_PATH} (run python -m mignon_ai_amd.build)")
        # PyTorch ships its own HIP runtime. Two runtimes in one process do not share the device (the
        # one initialised second finds none), so when torch is installed it is loaded first and the
        # library binds to the same libamdhip64.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> int:
    if rc < 0:
        raise MignonError(rc, (lib().mg_last_error() or b"").decode(errors="replace"))
    return rc


def ptr(a) -> int | None:
    """Address of a numpy array or torch tensor (None stays None)."""
    if a is None:
        return None
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data
