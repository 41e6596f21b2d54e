"""The C-ABI library (include/mignon_hip.h) on a machine without a GPU: it loads, exports every declared
entry point, rejects bad arguments before touching the device, and fails loudly when there is no
device instead of falling back to anything."""
import ctypes
import os
import re

import pytest

from helpers import ROOT, model_bytes
from mignon_ai_amd import _lib


def declared_functions():
    with open(os.path.join(ROOT, "include", "mignon_hip.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(mg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("mg_model_load", "mg_forward_batch", "mg_sessions_create", "mg_sessions_prefill",
                     "mg_sessions_step", "mg_sessions_decode_greedy", "mg_sessions_state_bytes",
                     "mg_gemm_i8", "mg_quantize_f32", "mg_model_call", "mg_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(_lib.SIGNATURES), "binding and header disagree"


def test_null_arguments_are_errors():
    L = _lib.lib()
    assert L.mg_model_info(None, None) == _lib.MG_ERR_INVALID
    assert b"null" in L.mg_last_error()
    assert L.mg_gemm_i8(None, 1, 1, None, 1, None, None, None, 0, None) == _lib.MG_ERR_INVALID
    assert L.mg_forward_batch(None, None, 1, 1, None, None, None, None, 0) == _lib.MG_ERR_INVALID
    assert L.mg_sessions_state_bytes(None) == -1
    assert L.mg_model_set_cancel(None, None) == _lib.MG_ERR_INVALID
    assert L.mg_sessions_step_noalloc(None, None, None, None, None) == _lib.MG_ERR_INVALID


def _has_gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.mark.skipif(_has_gpu(), reason="checks the no-device path")
def test_load_without_device_fails_loudly():
    data = model_bytes("c1")
    buf = (ctypes.c_uint8 * len(data)).from_buffer_copy(data)
    h = ctypes.c_void_p()
    rc = _lib.lib().mg_model_load(buf, len(data), 0, ctypes.byref(h))
    assert rc == _lib.MG_ERR_DEVICE and not h.value
    assert _lib.lib().mg_last_error()


def test_engine_option_validates():
    L = _lib.lib()
    assert L.mg_engine_option(7, 0) == _lib.MG_ERR_INVALID
    assert b"mg_engine_option" in L.mg_last_error()
    assert L.mg_engine_option(_lib.MG_OPT_GEMM_KERNEL, 3) == _lib.MG_ERR_INVALID
    assert L.mg_engine_option(_lib.MG_OPT_STEP_KERNEL, 4) == _lib.MG_ERR_INVALID
    assert L.mg_engine_option(_lib.MG_OPT_OPERANDS, 3) == _lib.MG_ERR_INVALID
    assert L.mg_engine_option(_lib.MG_OPT_KV_RINGS, 3) == _lib.MG_ERR_INVALID
    for opt, val in ((_lib.MG_OPT_GEMM_KERNEL, _lib.MG_GEMM_SLAB), (_lib.MG_OPT_ATTENTION_KERNEL, _lib.MG_ATTN_EXACT),
                     (_lib.MG_OPT_SCAN_KERNEL, _lib.MG_SCAN_FUSED), (_lib.MG_OPT_STEP_GRAPH, _lib.MG_STEP_EAGER),
                     (_lib.MG_OPT_STEP_KERNEL, _lib.MG_STEP_LAYERED), (_lib.MG_OPT_STEP_KERNEL, _lib.MG_STEP_TILED),
                     (_lib.MG_OPT_OPERANDS, _lib.MG_OPERANDS_LIMBS), (_lib.MG_OPT_OPERANDS, _lib.MG_OPERANDS_FP32),
                     (_lib.MG_OPT_KV_RINGS, _lib.MG_KV_FP32), (_lib.MG_OPT_KV_RINGS, _lib.MG_KV_PACKED)):
        prev = L.mg_engine_option(opt, val)
        assert prev in (0, 1, 2)
        assert L.mg_engine_option(opt, -1) == val
        assert L.mg_engine_option(opt, prev) == val


def test_stage_hooks_load_against_the_engine():
    """The stage-level parity tests' hooks (test infrastructure, not part of the ABI) load against the
    engine library and export their entry points."""
    import stage_hooks

    L = stage_hooks.lib()
    for name in ("mgt_row", "mgt_latch_scan", "mgt_attention", "mgt_attention_step", "mgt_attention_step_packed",
                 "mgt_export_kv_packed"):
        assert hasattr(L, name)
