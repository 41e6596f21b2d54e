"""Python host API over the C ABI, mirroring the reference's Go interfaces for this path:

  Model        quant.Model      (internal/quant/model.go:60-137): info accessors, call/forward (LogitsFn),
                                new_session (infer.SessionProvider, internal/infer/infer.go:17-20)
  Session      infer.Session    (internal/infer/infer.go:8-15) as quantSession implements it
                                (internal/quant/session.go:11-68)
  Sessions     the batched form: n sessions advancing together on the GPU
  forward_batch                 every position of B sequences at once (teacher-forced scoring)

Arrays are numpy on the host; the *_device methods take torch CUDA tensors and only enqueue work on
the model's stream.
"""
from __future__ import annotations

import ctypes
import json
import struct

import numpy as np

from ._lib import MG_PTR_DEVICE, ModelInfo, check, lib, ptr


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def read_metadata(data: bytes) -> dict:
    """The metadata object of a model file's JSON header (binary container or legacy JSON file)."""
    if len(data) >= 12 and data[:4] == b"MGNN":
        n = struct.unpack_from("<I", data, 8)[0]
        hdr = json.loads(data[12:12 + n])
    else:
        hdr = json.loads(data)
    return hdr.get("metadata") or {}


class Model:
    def __init__(self, data: bytes, max_context: int = 0):
        self._cancel_flags = []  # every cancellation flag this model was given (set_cancel)
        buf = (ctypes.c_uint8 * len(data)).from_buffer_copy(data)
        h = ctypes.c_void_p()
        check(lib().mg_model_load(buf, len(data), int(max_context), ctypes.byref(h)))
        self._h = h
        self.info = ModelInfo()
        check(lib().mg_model_info(self._h, ctypes.byref(self.info)))

    @classmethod
    def load(cls, path: str, max_context: int = 0) -> "Model":
        with open(path, "rb") as f:
            return cls(f.read(), max_context)

    def close(self):
        if getattr(self, "_h", None):
            lib().mg_model_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def handle(self):
        return self._h

    # quant.Model accessors
    def vocab_size(self) -> int:
        return self.info.vocab_size

    def state_size(self) -> int:
        return self.info.state_size

    def hidden_size(self) -> int:
        return self.info.hidden_size

    def num_blocks(self) -> int:
        return self.info.num_blocks

    def num_params(self) -> int:
        return self.info.num_params

    @property
    def max_context(self) -> int:
        return self.info.max_context

    def set_stream(self, stream_ptr: int | None):
        check(lib().mg_model_set_stream(self._h, stream_ptr))

    def sync(self):
        check(lib().mg_model_sync(self._h))

    def set_cancel(self, flag: "ctypes.c_int32 | None"):
        """mg_model_set_cancel: while flag.value is nonzero (any thread may set it), a batched decode on this
        model stops before its next token and returns the replies produced so far. None removes it. The
        model keeps every flag it was given alive for its own lifetime: a decode running on another thread
        may still read the one this call replaces."""
        if flag is not None:
            self._cancel_flags.append(flag)
        check(lib().mg_model_set_cancel(self._h, ctypes.addressof(flag) if flag is not None else None))

    def profile(self, on: bool):
        """Start (clearing earlier records) or stop per-kernel HIP-event timing on the model's stream."""
        check(lib().mg_model_profile(self._h, 1 if on else 0))

    def profile_read(self) -> dict:
        """{kernel class: (launches, total ms, algorithmic bytes, algorithmic int8 ops)} of the launches
        recorded while profiling was on (bytes and ops summed over the launches; 0 where not stated)."""
        from ._lib import KernelTime
        buf = (KernelTime * 32)()
        n = check(lib().mg_model_profile_read(self._h, buf, 32))
        return {buf[i].name.decode(): (buf[i].launches, buf[i].total_ms, buf[i].bytes, buf[i].ops)
                for i in range(min(n, 32))}

    # quant.Model.Call / Forward (LogitsFn)
    def call(self, ids):
        ids = _i32(ids)
        out = np.empty(self.vocab_size(), np.float64)
        n = check(lib().mg_model_call(self._h, ptr(ids), len(ids), ptr(out)))
        return out if n else None

    forward = call

    def forward_batch(self, ids2d, logits=True, logprob=False, probs=False, bits=False):
        ids = _i32(ids2d)
        B, T = ids.shape
        V = self.vocab_size()
        out = {}
        lg = np.empty((B, T, V), np.float32) if logits else None
        lp = np.empty((B, T), np.float32) if logprob else None
        pr = np.empty((B, T, V), np.float32) if probs else None
        bt = np.empty(B, np.float32) if bits else None
        check(lib().mg_forward_batch(self._h, ptr(ids), B, T, ptr(lg), ptr(lp), ptr(pr), ptr(bt), 0))
        for k, v in (("logits", lg), ("logprob", lp), ("probs", pr), ("bits", bt)):
            if v is not None:
                out[k] = v
        return out

    def forward_batch_device(self, ids, logits=None, logprob=None, probs=None, bits=None):
        B, T = ids.shape
        check(lib().mg_forward_batch(self._h, ptr(ids), B, T, ptr(logits), ptr(logprob), ptr(probs), ptr(bits),
                                     MG_PTR_DEVICE))

    def new_session(self, context_size: int = 0) -> "Session":
        return Session(self, context_size)

    def sessions(self, n: int, context_size: int = 0) -> "Sessions":
        return Sessions(self, n, context_size)


class Sessions:
    def __init__(self, model: Model, n: int, context_size: int = 0):
        self.model = model
        h = ctypes.c_void_p()
        check(lib().mg_sessions_create(model.handle, int(n), int(context_size), ctypes.byref(h)))
        self._h = h
        self.n = n

    def close(self):
        if getattr(self, "_h", None):
            lib().mg_sessions_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def state_bytes(self) -> int:
        return lib().mg_sessions_state_bytes(self._h)

    def device_bytes(self) -> int:
        return lib().mg_sessions_device_bytes(self._h)

    def prefill(self, prompts2d, lens=None, logits=True):
        p = _i32(prompts2d)
        n, L = p.shape
        lens = _i32(lens if lens is not None else np.full(n, L))
        V = self.model.vocab_size()
        lg = np.empty((n, V), np.float32) if logits else None
        am = np.empty(n, np.int32)
        pb = np.empty(n, np.float64)
        check(lib().mg_sessions_prefill(self._h, ptr(p), ptr(lens), L, ptr(lg), ptr(am), ptr(pb), 0))
        return lg, am, pb

    def step(self, ids, logits=True):
        ids = _i32(ids)
        V = self.model.vocab_size()
        lg = np.empty((self.n, V), np.float32) if logits else None
        am = np.empty(self.n, np.int32)
        pb = np.empty(self.n, np.float64)
        check(lib().mg_sessions_step(self._h, ptr(ids), ptr(lg), ptr(am), ptr(pb), 0))
        return lg, am, pb

    def step_device(self, ids, logits=None, argmax=None, prob=None):
        """mg_sessions_step on device arrays (ids [n] int32; logits [n][V] fp32, argmax [n] int32, prob [n]
        float64, each optional); enqueued on the model's stream."""
        check(lib().mg_sessions_step(self._h, ptr(ids), ptr(logits), ptr(argmax), ptr(prob), MG_PTR_DEVICE))

    def step_noalloc(self, ids, logits=None, argmax=None, prob=None):
        """mg_sessions_step_noalloc: step_device without any allocation (the library's static per-GPU
        scratch holds the workspace); device arrays only."""
        check(lib().mg_sessions_step_noalloc(self._h, ptr(ids), ptr(logits), ptr(argmax), ptr(prob)))

    def decode_greedy(self, prompts2d, max_tokens, lens=None):
        p = _i32(prompts2d)
        n, L = p.shape
        lens = _i32(lens if lens is not None else np.full(n, L))
        ids = np.empty((n, max_tokens), np.int32)
        probs = np.empty((n, max_tokens), np.float64)
        check(lib().mg_sessions_decode_greedy(self._h, ptr(p), ptr(lens), L, int(max_tokens), ptr(ids), ptr(probs), 0))
        return ids, probs

    def decode_greedy_until(self, prompts2d, max_tokens, stops, lens=None):
        """greedyLoop with stop tokens: (ids [n][max_tokens], probs, counts [n]); row i's reply is
        ids[i, :counts[i]] (it ends before the first stop token); later entries are unspecified."""
        p = _i32(prompts2d)
        n, L = p.shape
        lens = _i32(lens if lens is not None else np.full(n, L))
        st = _i32(list(stops))
        ids = np.empty((n, max_tokens), np.int32)
        probs = np.empty((n, max_tokens), np.float64)
        counts = np.empty(n, np.int32)
        check(lib().mg_sessions_decode_greedy_until(self._h, ptr(p), ptr(lens), L, int(max_tokens),
                                                    ptr(st) if st.size else None, int(st.size), ptr(ids), ptr(probs),
                                                    ptr(counts), 0))
        return ids, probs, counts

    def decode_sample(self, prompts2d, max_tokens, seeds, temperature=1.0, top_k=0, top_p=1.0, rep_penalty=1.0,
                      penalize_prompt=False, stops=(), lens=None):
        """sampleContinuation for every session (mg_sessions_decode_sample): (ids [n][max_tokens], counts [n]);
        row i's reply is ids[i, :counts[i]]. seeds[i] fixes session i's draws."""
        from ._lib import Sampling
        p = _i32(prompts2d)
        n, L = p.shape
        lens = _i32(lens if lens is not None else np.full(n, L))
        st = _i32(list(stops))
        sd = np.ascontiguousarray(np.asarray([int(x) & (2 ** 64 - 1) for x in seeds], np.uint64))
        sp = Sampling(temperature=temperature, rep_penalty=rep_penalty, top_p=top_p, top_k=top_k,
                      penalize_prompt=int(penalize_prompt))
        ids = np.empty((n, max_tokens), np.int32)
        counts = np.empty(n, np.int32)
        check(lib().mg_sessions_decode_sample(self._h, ptr(p), ptr(lens), L, int(max_tokens), ctypes.byref(sp), ptr(sd),
                                              ptr(st) if st.size else None, int(st.size), ptr(ids), ptr(counts), 0))
        return ids, counts

    def decode_greedy_device(self, prompts, lens, max_tokens, out_ids, out_probs):
        n, L = prompts.shape
        check(lib().mg_sessions_decode_greedy(self._h, ptr(prompts), ptr(lens), L, int(max_tokens), ptr(out_ids),
                                              ptr(out_probs), MG_PTR_DEVICE))


class Session:
    """One streaming session with quantSession's semantics (internal/quant/session.go:30-56): Prefill
    resets and keeps the last `window` tokens, an empty Prefill returns None and leaves the state, Append
    streams on (a never-prefilled session starts from an empty state, as the reference's re-prefill of a
    single held token does)."""

    def __init__(self, model: Model, context_size: int = 0):
        self._s = Sessions(model, 1, context_size)
        self.V = model.vocab_size()
        # Append's host buffers and their addresses, kept across calls (the call is latency-bound)
        self._ids = np.empty(1, np.int32)
        self._lg = np.empty((1, self.V), np.float32)
        self._ptrs = (ptr(self._ids), ptr(self._lg))
        self._step = lib().mg_sessions_step

    def prefill(self, tokens):
        tokens = _i32(tokens)
        if len(tokens) == 0:
            return None
        lg, _, _ = self._s.prefill(tokens[None, :])
        return lg[0].astype(np.float64)

    def append(self, token):
        self._ids[0] = token
        check(self._step(self._s._h, self._ptrs[0], self._ptrs[1], None, None, 0))
        return self._lg[0].astype(np.float64)

    def state_bytes(self) -> int:
        return self._s.state_bytes()


def gemm_i8(A, W, scale, want_acc=False):
    """mg_gemm_i8 on host arrays: A [M][K] int8, W [N][K] int8, scale [N] -> C [M][N] (and int32 acc)."""
    A = np.ascontiguousarray(A, np.int8)
    W = np.ascontiguousarray(W, np.int8)
    s = np.ascontiguousarray(scale, np.float32)
    M, K = A.shape
    N = W.shape[0]
    C = np.empty((M, N), np.float32)
    acc = np.empty((M, N), np.int32) if want_acc else None
    check(lib().mg_gemm_i8(ptr(A), M, K, ptr(W), N, ptr(s), ptr(C), ptr(acc), 0, None))
    return (C, acc) if want_acc else C


def gemm_i8_device(A, W, scale, C, acc=None, stream=None):
    M, K = A.shape
    N = W.shape[0]
    check(lib().mg_gemm_i8(ptr(A), M, K, ptr(W), N, ptr(scale), ptr(C), ptr(acc), MG_PTR_DEVICE, stream))


def quantize_f32(w):
    """mg_quantize_f32 on a host array -> (int8 data, fp32 scale): quant.NewTensorF32 on the GPU."""
    w = np.ascontiguousarray(w, np.float32).ravel()
    q = np.empty(w.shape, np.int8)
    s = np.zeros(1, np.float32)
    check(lib().mg_quantize_f32(ptr(w), len(w), ptr(q), ptr(s), 0, None))
    return q, np.float32(s[0])


_OPTIONS = {"gemm": (0, ["auto", "stream", "slab"]), "attention": (1, ["auto", "exact", "mfma", "fused"]),
            "scan": (2, ["auto", "separate", "fused"]), "step_graph": (3, ["auto", "off", "on"]),
            "step_kernel": (4, ["auto", "layered", "fused", "tiled"]), "operands": (5, ["auto", "limbs", "fp32"]),
            "kv_rings": (6, ["auto", "fp32", "packed"])}


def sample_logits(logits, recent=None, temperature=1.0, top_k=0, top_p=1.0, rep_penalty=1.0, u=None):
    """generate.SampleRawLogitsAdvanced on the current GPU for every row of float64 logits [n][V]
    (mg_sample_logits): recent is a list of per-row token lists (the repetition window), u the per-row
    uniforms standing for rand.Float64()."""
    from ._lib import Sampling
    lg = np.ascontiguousarray(logits, np.float64)
    n, V = lg.shape
    uu = np.ascontiguousarray(u if u is not None else np.zeros(n), np.float64)
    rp = rl = None
    ld = 0
    if recent is not None:
        ld = max([len(r) for r in recent] + [1])
        rp = np.zeros((n, ld), np.int32)
        rl = np.array([len(r) for r in recent], np.int32)
        for i, r in enumerate(recent):
            rp[i, :len(r)] = r
    sp = Sampling(temperature=temperature, rep_penalty=rep_penalty, top_p=top_p, top_k=top_k, penalize_prompt=0)
    out = np.empty(n, np.int32)
    check(lib().mg_sample_logits(ptr(lg), n, V, ptr(rp), ptr(rl), ld, ctypes.byref(sp), ptr(uu), ptr(out)))
    return out


def engine_option(name: str, value: str | None = None) -> str:
    """mg_engine_option: which implementation runs for "gemm" ("auto", "stream", "slab"), "attention"
    ("auto", "exact", "mfma", "fused": the projection fused with matrix-core attention), "scan" ("auto",
    "separate", "fused"), "step_graph" (decode steps replayed from a captured HIP graph: "auto", "off",
    "on"), "step_kernel" (decode steps: "auto", "layered", "fused": one workgroup per session, "tiled":
    one per 16 sessions) or "operands" (batched forward: "auto", "limbs": every GEMM operand's limb planes
    written by a pass of their own, "fp32": the GLU and attention outputs read as fp32 by the GEMMs that
    take them) or "kv_rings" (session K/V rings, fixed when a set is created: "auto" or "packed": 24-bit
    mantissas with a power-of-two scale per row where the decode attention kernels take the model,
    "fp32"), for the whole process. Returns the previous value (value None only reads it)."""
    opt, names = _OPTIONS[name]
    prev = lib().mg_engine_option(opt, -1 if value is None else names.index(value))
    check(prev if prev < 0 else 0)
    return names[prev]
