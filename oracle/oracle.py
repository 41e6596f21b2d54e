"""ctypes wrapper around the CPU oracle (oracle/mgn_oracle.cpp) plus an independent MGNN reader.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
as the checker / timed CPU baseline, never by the product (mignon_ai_amd/).

The reader restates the reference container and array order so that a model file can be fed to the
oracle without going through the product's own loader:
  - container: internal/binfmt/binfmt.go:1-144 (magic "MGNN", uint16 version 1, uint8 kind 2 = INT8,
    uint8 reserved, uint32 header length, JSON header, then uint32-count-prefixed arrays);
  - arrays: internal/quant/checkpoint.go:74-89 (embed; per block W1, b1, W2, b2, gamma, W_select and,
    for hybrid blocks, attn norm, QKV, Out; then final norm, head W, head bias);
  - legacy JSON files: internal/quant/checkpoint.go:162-180;
  - model construction: internal/quant/checkpoint.go:183-211 (tied head aliases the embedding).
"""
from __future__ import annotations

import ctypes
import json
import os
import struct
import subprocess
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libmgn_oracle.so")
_lib = None

_i8p = ctypes.POINTER(ctypes.c_int8)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)


def build() -> str:
    """Compile the oracle with its Makefile (g++ only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        v = ctypes.c_void_p
        sig = {
            "or_model_new": (v, [ctypes.c_int] * 8),
            "or_model_free": (None, [v]),
            "or_model_max_context": (ctypes.c_int, [v]),
            "or_model_set_embed": (None, [v, _i8p, ctypes.c_float]),
            "or_model_set_block": (None, [v, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i8p,
                                          ctypes.c_float, _f32p, _i8p, ctypes.c_float, _f32p, _f32p, ctypes.c_int,
                                          _i8p, ctypes.c_float]),
            "or_model_set_attn": (None, [v, ctypes.c_int, _f32p, _i8p, ctypes.c_float, _i8p, ctypes.c_float]),
            "or_model_set_head": (None, [v, _f32p, ctypes.c_int, _i8p, ctypes.c_float, _f32p, ctypes.c_int]),
            "or_call": (ctypes.c_int, [v, _i32p, ctypes.c_int, _f64p]),
            "or_session_new": (v, [v, ctypes.c_int]),
            "or_session_free": (None, [v]),
            "or_session_prefill": (ctypes.c_int, [v, _i32p, ctypes.c_int, _f64p]),
            "or_session_append": (ctypes.c_int, [v, ctypes.c_int, _f64p]),
            "or_session_state_bytes": (ctypes.c_longlong, [v]),
            "or_forward_all": (ctypes.c_int, [v, _i32p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int]),
            "or_greedy": (ctypes.c_int, [v, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _i32p,
                                         _f64p, ctypes.c_int]),
            "or_force_scalar": (None, [ctypes.c_int]),
            "or_has_avx2": (ctypes.c_int, []),
            "or_dot_f32": (ctypes.c_float, [_f32p, _f32p, ctypes.c_int]),
            "or_dot_i8_f32": (ctypes.c_float, [_f32p, _i8p, ctypes.c_int]),
            "or_fast_exp": (ctypes.c_float, [ctypes.c_float]),
            "or_sigmoid_clamped": (ctypes.c_float, [ctypes.c_float]),
            "or_rmsnorm": (None, [_f32p, _f32p, _f32p, ctypes.c_int]),
            "or_softmax": (None, [_f32p, ctypes.c_int]),
            "or_add_scaled": (None, [_f32p, _f32p, ctypes.c_float, ctypes.c_int]),
            "or_matvec_i8": (None, [_f32p, ctypes.c_int, _i8p, ctypes.c_int, ctypes.c_float, _f32p, ctypes.c_int,
                                    _f32p]),
            "or_latch_base": (None, [ctypes.c_int, _f32p]),
            "or_latch_seq": (None, [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]),
            "or_attend_seq": (None, [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, _f32p, ctypes.c_int]),
            "or_quantize": (None, [_f32p, ctypes.c_longlong, _i8p, _f32p]),
            "or_gemm_i8_ref": (ctypes.c_int, [_i8p, ctypes.c_int, ctypes.c_int, _i8p, ctypes.c_int, _f32p, _f32p,
                                              ctypes.c_int]),
            "or_gemm_i8_exact": (ctypes.c_int, [_i8p, ctypes.c_int, ctypes.c_int, _i8p, ctypes.c_int, _f32p, _f32p,
                                                _i32p, ctypes.c_int]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t) if a is not None else None


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------------------------------------
# kernel-level entry points
# ------------------------------------------------------------------------------------------------

def force_scalar(on: bool):
    """Use the scalar restatement of the dot kernels instead of the AVX2 path (identical bits)."""
    lib().or_force_scalar(1 if on else 0)


def has_avx2() -> bool:
    return bool(lib().or_has_avx2())


def dot_f32(x, y) -> np.float32:
    x, y = _c(x, np.float32), _c(y, np.float32)
    return np.float32(lib().or_dot_f32(_p(x, _f32p), _p(y, _f32p), min(len(x), len(y))))


def dot_i8_f32(x, w) -> np.float32:
    x, w = _c(x, np.float32), _c(w, np.int8)
    return np.float32(lib().or_dot_i8_f32(_p(x, _f32p), _p(w, _i8p), min(len(x), len(w))))


def fast_exp(x) -> np.float32:
    return np.float32(lib().or_fast_exp(float(np.float32(x))))


def sigmoid_clamped(x) -> np.float32:
    return np.float32(lib().or_sigmoid_clamped(float(np.float32(x))))


def rmsnorm(x, gamma) -> np.ndarray:
    x, g = _c(x, np.float32), _c(gamma, np.float32)
    out = np.empty_like(x)
    lib().or_rmsnorm(_p(x, _f32p), _p(g, _f32p), _p(out, _f32p), len(x))
    return out


def softmax(logits) -> np.ndarray:
    a = _c(logits, np.float32).copy()
    lib().or_softmax(_p(a, _f32p), len(a))
    return a


def add_scaled(y, x, alpha) -> np.ndarray:
    y = _c(y, np.float32).copy()
    x = _c(x, np.float32)
    lib().or_add_scaled(_p(y, _f32p), _p(x, _f32p), float(np.float32(alpha)), len(y))
    return y


def matvec_i8(w, stride, scale, x, bias=None, rows=None) -> np.ndarray:
    w, x = _c(w, np.int8), _c(x, np.float32)
    rows = rows if rows is not None else len(w) // stride
    y = np.empty(rows, np.float32)
    b = _c(bias, np.float32) if bias is not None else None
    lib().or_matvec_i8(_p(y, _f32p), rows, _p(w, _i8p), stride, float(np.float32(scale)), _p(x, _f32p), len(x),
                       _p(b, _f32p))
    return y


def latch_base(D: int) -> np.ndarray:
    out = np.empty(D, np.float32)
    lib().or_latch_base(D, _p(out, _f32p))
    return out


def latch_seq(lam, nf):
    """updateLatch's recurrence (internal/quant/stream.go:195-205) over [B][T][D] lambda and normalised
    cells, the latch starting from zero: the latch after every position, [B][T][D]."""
    lam, nf = _c(lam, np.float32), _c(nf, np.float32)
    B, T, D = lam.shape
    g = np.empty_like(lam)
    lib().or_latch_seq(_p(lam, _f32p), _p(nf, _f32p), B, T, D, D, _p(g, _f32p))
    return g


def attend_seq(qkv, heads, window, cap):
    """attendPosition's attention (internal/quant/attention.go:82-101) for every position of [B][T][3D]
    q | k | v rows, over a ring of cap positions: [B][T][D]."""
    qkv = _c(qkv, np.float32)
    B, T, D3 = qkv.shape
    D = D3 // 3
    att = np.empty((B, T, D), np.float32)
    lib().or_attend_seq(_p(qkv, _f32p), B, T, D, heads, window, cap, _p(att, _f32p), D)
    return att


def quantize(w):
    """quant.NewTensorF32 restated (internal/quant/tensor.go:12-42) -> (int8 data, fp32 scale)."""
    w = _c(w, np.float32).ravel()
    q = np.empty(w.shape, np.int8)
    s = ctypes.c_float()
    lib().or_quantize(_p(w, _f32p), len(w), _p(q, _i8p), ctypes.byref(s))
    return q, np.float32(s.value)


def gemm_i8_exact(A, W, scale, want_acc=True, nthreads=8):
    A, W, s = _c(A, np.int8), _c(W, np.int8), _c(scale, np.float32)
    M, K = A.shape
    N = W.shape[0]
    C = np.empty((M, N), np.float32)
    acc = np.empty((M, N), np.int32) if want_acc else None
    rc = lib().or_gemm_i8_exact(_p(A, _i8p), M, K, _p(W, _i8p), N, _p(s, _f32p), _p(C, _f32p), _p(acc, _i32p),
                                nthreads)
    if rc != 0:
        raise OverflowError("int32 accumulator overflow")
    return C, acc


def gemm_i8_ref(A, W, scale, nthreads=8):
    """Reference method for config 2: MatVecInt8 per row on float32-converted int8 activations."""
    A, W, s = _c(A, np.int8), _c(W, np.int8), _c(scale, np.float32)
    M, K = A.shape
    N = W.shape[0]
    C = np.empty((M, N), np.float32)
    lib().or_gemm_i8_ref(_p(A, _i8p), M, K, _p(W, _i8p), N, _p(s, _f32p), _p(C, _f32p), nthreads)
    return C


# ------------------------------------------------------------------------------------------------
# model files
# ------------------------------------------------------------------------------------------------

@dataclass
class RefBlock:
    steps: int
    dilation_base: int
    initial_dilation: int
    w1: np.ndarray
    s1: np.float32
    b1: np.ndarray
    w2: np.ndarray
    s2: np.float32
    b2: np.ndarray
    gamma: np.ndarray
    wsel: np.ndarray
    ssel: np.float32
    attn: dict | None = None


@dataclass
class RefModel:
    V: int
    D: int
    H: int
    tied: bool
    embed: np.ndarray
    embed_scale: np.float32
    blocks: list
    final_norm: np.ndarray
    head_w: np.ndarray | None
    head_scale: np.float32
    head_b: np.ndarray
    heads: int
    window: int
    context_size: int
    metadata: dict = field(default_factory=dict)


class ModelFileError(ValueError):
    pass


def _decode_binary(data: bytes):
    """binfmt.Decode + File.Fill (internal/binfmt/binfmt.go:87-144)."""
    if not data.startswith(b"MGNN"):
        raise ModelFileError("not a binary model file")
    if len(data) < 12:
        raise ModelFileError("binary model file is truncated")
    version, kind, _res, n = struct.unpack_from("<HBBI", data, 4)
    if version != 1:
        raise ModelFileError(f"binary model file version {version} is not supported")
    if kind not in (1, 2):
        raise ModelFileError(f"unknown model kind {kind}")
    if 12 + n > len(data):
        raise ModelFileError("binary model file is truncated (header)")
    if kind != 2:
        raise ModelFileError("not an INT8 model file")
    return json.loads(data[12:12 + n]), memoryview(data)[12 + n:]


def _array_order(cp):
    """quant.CheckpointJSON.arrays (internal/quant/checkpoint.go:74-89): (path, dtype) in file order."""
    out = [(("embed", "data"), "i8")]
    for i, b in enumerate(cp["blocks"]):
        out += [(("blocks", i, "rule_w1", "data"), "i8"), (("blocks", i, "rule_b1"), "f32"),
                (("blocks", i, "rule_w2", "data"), "i8"), (("blocks", i, "rule_b2"), "f32"),
                (("blocks", i, "gamma"), "f32"), (("blocks", i, "rule_w_select", "data"), "i8")]
        if b.get("attn") is not None:
            out += [(("blocks", i, "attn", "norm"), "f32"), (("blocks", i, "attn", "qkv", "data"), "i8"),
                    (("blocks", i, "attn", "out", "data"), "i8")]
    out += [(("final_norm",), "f32"), (("head_w", "data"), "i8"), (("head_b",), "f32")]
    return out


def _set_path(obj, path, value):
    for p in path[:-1]:
        if isinstance(p, str) and (p not in obj or obj[p] is None):
            obj[p] = {}
        obj = obj[p]
    obj[path[-1]] = value


def _get_path(obj, path):
    for p in path:
        if obj is None:
            return None
        obj = obj[p] if isinstance(p, int) else obj.get(p)
    return obj


def read_model(data: bytes) -> RefModel:
    """quant.Decode (internal/quant/checkpoint.go:162-212), binary or legacy JSON."""
    if data.startswith(b"MGNN"):
        cp, rest = _decode_binary(data)
        off = 0
        for i, (path, dt) in enumerate(_array_order(cp)):
            if len(rest) - off < 4:
                raise ModelFileError(f"binary model file is truncated (array {i})")
            (n,) = struct.unpack_from("<I", rest, off)
            off += 4
            width = 1 if dt == "i8" else 4
            if n > (len(rest) - off) // width:
                raise ModelFileError(f"binary model file is truncated (array {i})")
            arr = np.frombuffer(rest, dtype=np.int8 if dt == "i8" else "<f4", count=n, offset=off).copy()
            off += n * width
            _set_path(cp, path, arr)
        if off != len(rest):
            raise ModelFileError(f"binary model file has {len(rest) - off} unexpected trailing bytes")
    else:
        cp = json.loads(data)
        for path, dt in _array_order(cp):
            v = _get_path(cp, path)
            _set_path(cp, path, np.asarray(v if v is not None else [], np.int8 if dt == "i8" else np.float32))
    V, D, H = cp["vocab_size"], cp["state_size"], cp["hidden_size"]
    want = 2 * H * 3 * D
    blocks = []
    for i, b in enumerate(cp["blocks"]):
        if len(b["rule_w1"]["data"]) != want:
            raise ModelFileError(f"block {i} rule_w1 has {len(b['rule_w1']['data'])} weights, want {want}")
        attn = None
        if b.get("attn") is not None:
            a = b["attn"]
            attn = dict(norm=a["norm"], qkv=a["qkv"]["data"], sqkv=np.float32(a["qkv"]["scale"]),
                        wo=a["out"]["data"], so=np.float32(a["out"]["scale"]))
        blocks.append(RefBlock(b["steps"], b["dilation_base"], b["initial_dilation"], b["rule_w1"]["data"],
                               np.float32(b["rule_w1"]["scale"]), b["rule_b1"], b["rule_w2"]["data"],
                               np.float32(b["rule_w2"]["scale"]), b["rule_b2"], b["gamma"],
                               b["rule_w_select"]["data"], np.float32(b["rule_w_select"]["scale"]), attn))
    meta = cp.get("metadata") or {}
    tied = bool(cp.get("tied_embed"))
    hw = cp.get("head_w") or {}
    return RefModel(V=V, D=D, H=H, tied=tied, embed=cp["embed"]["data"], embed_scale=np.float32(cp["embed"]["scale"]),
                    blocks=blocks, final_norm=cp["final_norm"], head_w=None if tied else hw.get("data"),
                    head_scale=np.float32(hw.get("scale", 0) or 0), head_b=cp["head_b"],
                    heads=int(meta.get("attn_heads", 0) or 0), window=int(meta.get("attn_window", 0) or 0),
                    context_size=int(meta.get("context_size", 0) or 0), metadata=meta)


class OracleModel:
    """The oracle's quant.Model. Keeps the numpy arrays alive for the C side."""

    def __init__(self, rm: RefModel, max_context: int | None = None):
        L = lib()
        self.rm = rm
        ctx = rm.context_size if max_context is None else max_context
        self.h = L.or_model_new(rm.V, rm.D, rm.H, len(rm.blocks), int(rm.tied), rm.heads, rm.window, ctx)
        self.max_context = L.or_model_max_context(self.h)
        self._keep = []

        def k(a, dt):
            a = _c(a, dt)
            self._keep.append(a)
            return a

        L.or_model_set_embed(self.h, _p(k(rm.embed, np.int8), _i8p), float(rm.embed_scale))
        for i, b in enumerate(rm.blocks):
            g = k(b.gamma, np.float32)
            L.or_model_set_block(self.h, i, b.steps, b.dilation_base, b.initial_dilation, _p(k(b.w1, np.int8), _i8p),
                                 float(b.s1), _p(k(b.b1, np.float32), _f32p), _p(k(b.w2, np.int8), _i8p),
                                 float(b.s2), _p(k(b.b2, np.float32), _f32p), _p(g, _f32p), len(g),
                                 _p(k(b.wsel, np.int8), _i8p), float(b.ssel))
            if b.attn is not None:
                a = b.attn
                L.or_model_set_attn(self.h, i, _p(k(a["norm"], np.float32), _f32p), _p(k(a["qkv"], np.int8), _i8p),
                                    float(a["sqkv"]), _p(k(a["wo"], np.int8), _i8p), float(a["so"]))
        fn = k(rm.final_norm, np.float32)
        hb = k(rm.head_b, np.float32)
        hw = k(rm.head_w, np.int8) if rm.head_w is not None else None
        L.or_model_set_head(self.h, _p(fn, _f32p), len(fn), _p(hw, _i8p), float(rm.head_scale), _p(hb, _f32p),
                            len(hb))

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_model_free(self.h)
            self.h = None

    @property
    def V(self):
        return self.rm.V

    def call(self, ids):
        ids = _c(ids, np.int32)
        out = np.empty(self.V, np.float64)
        n = lib().or_call(self.h, _p(ids, _i32p), len(ids), _p(out, _f64p))
        return out if n else None

    def forward_all(self, ids2d, nthreads=8):
        ids = _c(ids2d, np.int32)
        B, T = ids.shape
        out = np.empty((B, T, self.V), np.float32)
        lib().or_forward_all(self.h, _p(ids, _i32p), B, T, _p(out, _f32p), nthreads)
        return out

    def greedy(self, prompts2d, max_tokens, ctx=0, nthreads=8):
        p = _c(prompts2d, np.int32)
        B, P = p.shape
        ids = np.zeros((B, max_tokens), np.int32)
        probs = np.zeros((B, max_tokens), np.float64)
        lib().or_greedy(self.h, _p(p, _i32p), B, P, max_tokens, ctx, _p(ids, _i32p), _p(probs, _f64p), nthreads)
        return ids, probs

    def new_session(self, ctx):
        return OracleSession(self, ctx)


class OracleSession:
    def __init__(self, m: OracleModel, ctx: int):
        self.m = m
        self.h = lib().or_session_new(m.h, ctx)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_session_free(self.h)
            self.h = None

    def prefill(self, ids):
        ids = _c(ids, np.int32)
        out = np.empty(self.m.V, np.float64)
        n = lib().or_session_prefill(self.h, _p(ids, _i32p), len(ids), _p(out, _f64p))
        return out if n else None

    def append(self, tok):
        out = np.empty(self.m.V, np.float64)
        lib().or_session_append(self.h, int(tok), _p(out, _f64p))
        return out

    def state_bytes(self):
        return lib().or_session_state_bytes(self.h)


def logprob_f64(logits: np.ndarray, target: int) -> float:
    """eval.logProb (internal/eval/suite.go:200-208) in float64."""
    l = np.asarray(logits, np.float64)
    mx = l.max()
    return float(l[target] - mx - np.log(np.exp(l - mx).sum()))
