"""Build and ctypes binding of the stage hooks (tests/stage_hooks.hip): single-stage launches of the
engine's kernels on torch device buffers, for the stage-level parity tests. Test infrastructure only.

    python tests/stage_hooks.py     # -> tests/_build/libmg_stage_hooks.so (after the engine build)
"""
from __future__ import annotations

import ctypes
import hashlib
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "stage_hooks.hip")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libmg_stage_hooks.so")
ENGINE_DIR = os.path.join(ROOT, "mignon_ai_amd", "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

_lib = None

# The hooks fill the engine's argument structs (kernels.hpp) and pass them to its launchers: a hooks
# library compiled against other headers than the engine's would hand the launchers misplaced fields
# (pointers read as sizes, buffers swapped), so the build records a digest of the headers it compiled
# against and the loader refuses a library whose digest differs from the current headers'.
HEADERS = [os.path.join(ROOT, "mignon_ai_amd", "csrc", h) for h in ("kernels.hpp", "common.hpp", "gemm.hpp")]


def headers_digest() -> str:
    h = hashlib.sha256()
    for p in HEADERS:
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def build() -> str:
    """Compile the hooks for gfx950 against the engine library (which must be built first)."""
    if not os.path.exists(os.path.join(ENGINE_DIR, "libmignon_hip.so")):
        raise RuntimeError("build the engine first (python -m mignon_ai_amd.build)")
    os.makedirs(OUT_DIR, exist_ok=True)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(ROOT, "mignon_ai_amd", "csrc"), f'-DMGT_HEADERS_DIGEST="{headers_digest()}"',
           "-shared", SRC, "-o", tmp,
           "-L", ENGINE_DIR, "-lmignon_hip", "-Wl,-rpath,$ORIGIN/../../mignon_ai_amd/_build"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed on stage_hooks.hip")
    os.replace(tmp, LIB)
    return LIB


def lib():
    """The hooks library, loaded after the engine library (the hooks call into that same copy)."""
    global _lib
    if _lib is None:
        from mignon_ai_amd import _lib as engine

        engine.lib()
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is missing: run python tests/stage_hooks.py after building the engine")
        L = ctypes.CDLL(LIB)
        L.mgt_headers_digest.restype = ctypes.c_char_p
        built, now = L.mgt_headers_digest().decode(), headers_digest()
        if built != now:
            raise RuntimeError(f"{LIB} was compiled against other engine headers ({built}, now {now}): "
                               "rebuild it (python tests/stage_hooks.py) after the engine")
        p, i = ctypes.c_void_p, ctypes.c_int
        sig = {
            "mgt_row": [p, i, i, i, p, p, p, p],
            "mgt_latch_scan": [p, p, i, i, i, i, p],
            "mgt_attention": [p, i, i, i, i, i, i, i, p, i],
            "mgt_attention_step": [p, p, p, p, i, i, i, i, i, i, p, p, p, i],
            "mgt_attention_step_packed": [p, p, p, p, p, p, i, i, i, i, i, i, p, p, p, i],
            "mgt_export_kv_packed": [i, i, i, i, i, p, p, p, p, p, p],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.restype = ctypes.c_int
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(t):
    """Device address of a torch tensor (None for None). The caller keeps the tensor referenced until the
    hook returns: a temporary's memory goes back to torch's allocator at once and is handed to the next
    allocation."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed with HIP status {rc}")


if __name__ == "__main__":
    print(build())
