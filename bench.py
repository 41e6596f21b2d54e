#!/usr/bin/env python3
"""Benchmark of the batched INT8 engine on one MI355X.

    python bench.py [--config c5] [--steps K] [--warmup W] [--gpus 1]

Prints one JSON line. A step is one pass of the hot path over one batch of seeded synthetic input that
is already resident in HBM:
  c5 (default)  16384 x 128-token teacher-forced scoring of the D384/H1024/4-block model: full softmax
                probabilities [16384, 128, 8192] fp32 and per-sequence bits per token
  c3            1024 x 128 tokens of the D128 model: logits + per-token log-probs
  c4            4096 sessions: 32-token prefill + 64 greedy tokens (value counts generated tokens)
  c2            the standalone INT8 GEMM 262144 x 384 x 512 (value counts rows = tokens)
  c1            64 x 128 tokens of the tiny model: logits
  score         eval.Perplexity over a 65536-token stream of the c3 model, context 128: one batched pass
                over every target's window (mg_score_sequences; value counts scored targets)
  sample        c4's sessions and lengths with sampled tokens (temperature 0.7, top-k 40, top-p 0.9,
                repetition penalty 1.2, trigram blocking; mg_sessions_decode_sample; value counts tokens)
  chat          infer.Generate (greedy, chat template, at most 80 tokens) for the 168 order-search requests
                x 24 on the reference's trained orders.mgn, all in one batch (mg_generate_greedy; value
                counts requests)
  append        one session's streaming latency (BenchmarkAppend of the reference's genbench on the medium
                shape, c3's model): microseconds per Append with host logits

Timing: W warmup steps, then K steps timed with HIP events and nothing else on the stream (value,
ms_per_step); then K more steps with HIP events around every launch on the model's stream (the per-kernel
breakdown, kernel_classes, and profiled_ms_per_step: per-launch events slow launch-bound configurations
down, so they stay out of the timed steps).
kernel_classes: every kernel class of the profiled steps with its algorithmic work per launch as the
engine states it (bytes its operands and results must move; int8 MACs x 2 for GEMMs), its bound (the
larger of the issued-MFMA and HBM floors at the published peaks) and the achieved fraction of that peak.
roofline: the same for the class with the largest share of the profiled time.
cpu_baseline: the CPU restatement of the reference engine (oracle/, AVX2 dot kernels) timed on this host
on a bounded sample of the same workload.
single_session_append (c5 line) and --config append: one session's Append latency beside the reference's
published figure for that shape.
The c5 line (the default) also carries compact objects of the other workloads measured in the same run
(decode = c4, c1, c2, c3, score, sample, chat; --no-extras leaves them and single_session_append out).
  copy          a device-to-device copy of --copy-mib MiB: the HBM counters' calibration (FETCH_SIZE and
                WRITE_SIZE of this copy against its known size) and the practical bandwidth ceiling
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "INT8 tokens/sec (batched forward + decode); % of int8-MFMA / HBM roofline"
PEAK_MFMA_TOPS = 5000.0   # MI355X dense int8 MFMA, TOP/s
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E, GB/s
# What the slab GEMM's K step sustains on this part with random int8 operands (a matrix-core probe whose
# recorded runs profiles/mfma_ceiling.md holds): the clock the part holds while every MAC switches stays
# below the one the published peak assumes (zero operands reach 4728).
SUSTAINED_MFMA_TOPS = 3664.0
LIMB_PLANES = 3
# kernel classes whose int8 work runs on limb-expanded activations (the fused attention class counts its
# projection GEMM; its fp32 attention flops are not in ops)
LIMB_GEMMS = ("gemm_glu", "gemm_highway", "gemm_latch", "gemm_qkv", "gemm_out", "gemm_logits", "gemm_probs",
              "qkv_attention", "tile_step")
SCORE_TOKENS, SCORE_CONTEXT = 65536, 128
CHAT_REPEAT, CHAT_MAX_TOKENS = 24, 80   # max reply tokens: examples/order-search/orders.js:20
SAMPLE_PARAMS = dict(temperature=0.7, top_k=40, top_p=0.9, rep_penalty=1.2)


def per_token_macs(spec):
    """int8-weight MACs per token, per GEMM class (reference layout, internal/ca/layout.go:96-162)."""
    D, H, V = spec.D, spec.H, spec.V
    bsteps = sum(b.steps for b in spec.blocks)
    nattn = len(spec.blocks) if spec.heads > 0 else 0
    return {
        "gemm_glu": bsteps * 3 * D * 2 * H,
        "gemm_highway": bsteps * H * 2 * D,
        "gemm_latch": bsteps * D * D,
        "gemm_qkv": nattn * D * 3 * D,
        "gemm_out": nattn * D * D,
        "gemm_logits": D * V,
        "gemm_probs": D * V,
    }


def host_cores():
    """Cores this process may run on (its affinity set), which on a shared box can be fewer than the
    machine's count."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


# Worker threads of the CPU baselines: every core this process may use, up to the 16 cores a one-GPU
# share of the GPU box holds (its MAX_JOBS / OMP_NUM_THREADS setting).
CPU_SHARE = 16


def cpu_threads():
    return max(1, min(CPU_SHARE, host_cores()))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_fields(thr):
    """What a CPU baseline states about the host beside its thread count."""
    return {"cpu_model": cpu_model(), "host_cores": host_cores(), "machine_cores": os.cpu_count(),
            "threads_note": f"{thr} worker threads: every core of this process's affinity set, capped at the "
                            f"{CPU_SHARE}-core share of one GPU on the box"}


def measured_traffic(config, cls):
    """HBM bytes per launch of a kernel class, from the committed rocprofv3 counter summary of this
    configuration (FETCH_SIZE + WRITE_SIZE scaled by a copy kernel's ratio; see that file's commands)."""
    from mignon_ai_amd.profsum import traffic_for
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{config}_hbm_traffic.md")
    v = traffic_for(path, cls)
    return (None, None) if v is None else (round(v), f"profiles/{config}_hbm_traffic.md")


def class_work(prof, extra=None):
    """Per kernel class: (launches, ms, algorithmic bytes, algorithmic int8 ops), summed over the profiled
    steps. The engine states bytes and ops per launch (mg_kernel_time_t); `extra` supplies the bytes of
    classes whose work the host cannot know (decode attention's spans): {class: bytes over the steps}."""
    out = {}
    for k, v in prof.items():
        launches, ms, by, ops = v
        if extra and k in extra:
            by = extra[k]
        out[k] = (launches, ms, by, ops)
    return out


def class_roofline(cls, launches, ms, by, ops):
    """Roofline of one kernel class from its algorithmic work. The bound is whichever floor is larger at
    the published peaks: issued int8 MFMA ops (every limb GEMM issues each algorithmic op once per
    activation limb plane) against 5.0 POP/s, or bytes against 8 TB/s. Returns None without stated work."""
    if ms <= 0 or (by <= 0 and ops <= 0):
        return None
    planes = LIMB_PLANES if cls in LIMB_GEMMS else 1
    t_mfma = ops * planes / (PEAK_MFMA_TOPS * 1e12)
    t_hbm = by / (PEAK_HBM_GBS * 1e9)
    secs = ms / 1e3
    if t_mfma >= t_hbm:
        achieved = ops / secs / 1e12
        r = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_MFMA_TOPS, "unit": "TFLOP/s",
             "frac": round(achieved / PEAK_MFMA_TOPS, 4)}
        if planes > 1:
            r["issued"] = round(achieved * planes, 2)
            r["issued_frac"] = round(achieved * planes / PEAK_MFMA_TOPS, 4)
            r["issued_frac_of_sustained"] = round(achieved * planes / SUSTAINED_MFMA_TOPS, 4)
    else:
        achieved = by / secs / 1e9
        r = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
             "frac": round(achieved / PEAK_HBM_GBS, 4)}
    r["bytes_per_launch"] = round(by / launches)
    r["ops_per_launch"] = round(ops / launches)
    r["avg_launch_ms"] = round(ms / launches, 4)
    return r


def class_table(work, steps):
    """Every kernel class of the profiled steps: launches and ms per step, and its roofline."""
    table = {}
    for k, (launches, ms, by, ops) in sorted(work.items(), key=lambda kv: -kv[1][1]):
        row = {"launches_per_step": round(launches / steps, 2), "ms_per_step": round(ms / steps, 3)}
        r = class_roofline(k, launches, ms, by, ops)
        if r:
            row.update({x: r[x] for x in ("bound", "achieved", "unit", "frac", "bytes_per_launch", "ops_per_launch")})
            if "issued_frac_of_sustained" in r:
                row["issued_frac_of_sustained"] = r["issued_frac_of_sustained"]
        table[k] = row
    return table


def roofline_for(work, config=None):
    """The roofline of the kernel class with the largest share of the profiled time (among classes whose
    work is stated), with the HBM traffic its counters measured where a summary is committed."""
    cands = [k for k, v in work.items() if v[2] > 0 or v[3] > 0]
    if not cands:
        return None, None
    dom = max(cands, key=lambda k: work[k][1])
    launches, ms, by, ops = work[dom]
    r = class_roofline(dom, launches, ms, by, ops)
    r["kernel"] = dom
    r["traffic"] = None
    if config:
        r["traffic"], src = measured_traffic(config, dom)
        if src:
            r["traffic_source"] = src
        # the kernel's shader clock and busy fractions from the committed counter summary: the limb GEMMs
        # run at a power-limited clock, which is what separates the issued rate from the published peak
        from mignon_ai_amd.profsum import clock_for
        cpath = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"{config}_clock_busy.md")
        c = clock_for(cpath, dom)
        if c:
            r["counters"] = dict(c, source=f"profiles/{config}_clock_busy.md")
    return dom, r


def timed(step, warmup, steps, torch, before=None):
    """W warmup steps, then K timed steps with nothing else on the stream (HIP events around the K steps:
    ms per step and wall seconds). With `before` (it turns the per-launch profiler on), K more steps follow
    with HIP events around every launch, for the kernel breakdown and the roofline; their ms per step is
    returned third (None without). Per-launch events cost launch-bound configurations up to 2x, so they
    are kept out of the timed steps."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / steps
    ms_prof = None
    if before:
        before()
        ev0.record()
        for _ in range(steps):
            step()
        ev1.record()
        torch.cuda.synchronize()
        ms_prof = ev0.elapsed_time(ev1) / steps
    return ms, wall, ms_prof


def _repeat(fn, seconds):
    """Runs fn() until at least `seconds` have passed (at least once); returns (passes, elapsed)."""
    t0 = time.perf_counter()
    n = 0
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            return n, dt


def cpu_baseline_forward(data, spec, B, T, seconds, seed):
    from oracle import oracle as O
    om = O.OracleModel(O.read_model(data))
    thr = cpu_threads()
    # a first batch of full-length sequences sizes the sample (at most the whole workload) so that it
    # takes about `seconds`; a sample that is the whole workload is repeated to fill that time
    probe = synth_ids(seed, "cpu-probe", (thr, T), spec.V)
    t0 = time.perf_counter()
    om.forward_all(probe, nthreads=thr)
    rate = probe.size / max(time.perf_counter() - t0, 1e-6)
    nseq = int(max(min(thr, B), min(B, rate * seconds / T)))
    ids = synth_ids(seed, "cpu-sample", (nseq, T), spec.V)
    passes, dt = _repeat(lambda: om.forward_all(ids, nthreads=thr), seconds / 2)
    return {"value": round(passes * ids.size / dt, 1), "unit": "tokens/s", "cores": thr, **cpu_fields(thr), "kind": "port",
            "sample": f"{nseq} of {B} sequences x {T} tokens, {passes} pass(es), teacher-forced (session route: "
                      f"every position's logits), {dt:.1f} s; C++ restatement of the reference Go engine with AVX2 "
                      f"dot kernels"}


def cpu_baseline_decode(data, spec, S, P, G, seconds, seed):
    from oracle import oracle as O
    om = O.OracleModel(O.read_model(data))
    thr = cpu_threads()
    probe = synth_ids(seed, "cpu-probe", (thr, P), spec.V)
    t0 = time.perf_counter()
    om.greedy(probe, 4, nthreads=thr)
    rate = thr * (P + 4) / max(time.perf_counter() - t0, 1e-6)  # positions per second
    nses = int(max(min(thr, S), min(S, rate * seconds / (P + G))))
    prompts = synth_ids(seed, "cpu-sample", (nses, P), spec.V)
    passes, dt = _repeat(lambda: om.greedy(prompts, G, nthreads=thr), seconds / 2)
    return {"value": round(passes * nses * G / dt, 1), "unit": "generated tokens/s", "cores": thr, **cpu_fields(thr),
            "kind": "port",
            "sample": f"{nses} of {S} sessions x ({P}-token prefill + {G} greedy tokens), {passes} pass(es), "
                      f"{dt:.1f} s; C++ restatement of the reference Go engine with AVX2 dot kernels"}


def cpu_baseline_gemm(A, W, s, seconds):
    from oracle import oracle as O
    thr = cpu_threads()
    rows = max(thr, 256)
    t0 = time.perf_counter()
    O.gemm_i8_ref(A[:rows], W, s, nthreads=thr)
    rate = rows / max(time.perf_counter() - t0, 1e-6)
    n = int(min(len(A), max(rows, rate * seconds)))
    passes, dt = _repeat(lambda: O.gemm_i8_ref(A[:n], W, s, nthreads=thr), seconds / 2)
    return {"value": round(passes * n / dt, 1), "unit": "rows/s", "cores": thr, **cpu_fields(thr), "kind": "port",
            "sample": f"{n} of {len(A)} rows, {passes} pass(es), {dt:.1f} s; MatVecInt8 per row (DotInt8F32, AVX2) "
                      f"as the reference"}


def cpu_baseline_score(data, tokens, context, seconds):
    """eval.Perplexity's loop as the reference runs it: one Call of the target's window per target, on one
    core, over the first targets of the stream."""
    from oracle import oracle as O
    om = O.OracleModel(O.read_model(data))
    tok = [int(t) for t in tokens]
    done = [0]

    def one():
        t = 1 + done[0] % (len(tok) - 1)
        om.call(tok[max(0, t - context):t])
        done[0] += 1
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds / 2:
        for _ in range(8):
            one()
    dt = time.perf_counter() - t0
    return {"value": round(done[0] / dt, 1), "unit": "targets/s", "cores": 1, **cpu_fields(1), "kind": "port",
            "sample": f"the first {done[0]} targets of the stream, one {context}-token window Call each (the "
                      f"reference's sequential nll.score loop), {dt:.1f} s; C++ restatement of the reference Go "
                      f"engine with AVX2 dot kernels"}


def cpu_baseline_chat(data, requests, max_tokens, seconds):
    """infer.Generate per request, sequentially, as the reference's web page and check.js run it."""
    from oracle import oracle as O
    from oracle import text as T
    om = O.OracleModel(O.read_model(data))
    tok = T.Tokenizer.from_model_file(data)
    ctx = T.read_header(data)["metadata"]["context_size"]
    n, gen = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds / 2:
        _, ids, _ = T.generate(om, tok, requests[n % len(requests)], ctx, max_tokens)
        n += 1
        gen += len(ids)
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 1), "unit": "requests/s", "cores": 1, **cpu_fields(1), "kind": "port",
            "sample": f"{n} requests ({gen} generated tokens) one after another, {dt:.1f} s; the restated "
                      f"tokenizer and greedy loop over the C++ restatement of the reference Go engine"}


APPEND_CONTEXT, APPEND_TOKENS, APPEND_REPEATS = 128, 64, 20  # genbench's ctx=128 run, appendTokens
APPEND_PUBLISHED_US = 125.0  # medium preset, INT8 generation (internal/train/presets.go:95)


def append_latency(seed, repeats=APPEND_REPEATS, cpu_seconds=0.0):
    """Single-session streaming latency as the reference's BenchmarkAppend measures it
    (internal/genbench/genbench_test.go:88-123): the `medium` shape (c3's model: D128 H256, 2 blocks x 1
    step, 4 heads, window 64, V2048) at context 128, a session prefilled with 64 ids in [0, 1000) outside
    the timed region, then 64 Appends timed, each returning the position's logits to the host (one
    mg_sessions_step of one session with host pointers). Reported as microseconds per token: the median
    over `repeats` prefill + 64-append rounds, and the oracle's (the CPU restatement, one core) beside it."""
    from mignon_ai_amd import Model, mgnn, quantize_f32, synth
    spec = synth.CONFIGS["c3"]["spec"]
    data = mgnn.build_model_file(spec, seed, quantize_f32)
    m = Model(data)
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, 1000, APPEND_CONTEXT - APPEND_TOKENS)
    toks = rng.integers(0, 1000, (repeats + 1, APPEND_TOKENS))
    sess = m.new_session(APPEND_CONTEXT)
    rounds = []
    for r in range(repeats + 1):  # the first round warms up
        sess.prefill(prompt)
        t0 = time.perf_counter()
        for t in toks[r]:
            sess.append(int(t))
        rounds.append((time.perf_counter() - t0) / APPEND_TOKENS * 1e6)
    us = float(np.median(rounds[1:]))
    out = {"us_per_token": round(us, 2), "us_per_token_min": round(float(min(rounds[1:])), 2),
           "reference_published_us_per_token": APPEND_PUBLISHED_US,
           "workload": f"BenchmarkAppend, medium shape (D{spec.D} H{spec.H} {len(spec.blocks)} blocks heads "
                       f"{spec.heads} window {spec.window} V{spec.V}), context {APPEND_CONTEXT}: prefill "
                       f"{APPEND_CONTEXT - APPEND_TOKENS} ids, then {APPEND_TOKENS} Appends with host logits; median "
                       f"of {repeats} rounds"}
    if cpu_seconds > 0:
        from oracle import oracle as O
        om = O.OracleModel(O.read_model(data))
        osess = om.new_session(APPEND_CONTEXT)
        n, t_total = 0, 0.0
        while t_total < cpu_seconds:
            osess.prefill([int(x) for x in prompt])
            t0 = time.perf_counter()
            for t in toks[n % len(toks)]:
                osess.append(int(t))
            t_total += time.perf_counter() - t0
            n += 1
        out["cpu_us_per_token"] = round(t_total / (n * APPEND_TOKENS) * 1e6, 2)
        out["cpu_kind"] = "port: the oracle's session (C++ restatement of the reference Go engine), one core"
    return out


def synth_ids(seed, tag, shape, V):
    from mignon_ai_amd import synth
    return synth.token_ids(seed, tag, shape, V)


def run(args):
    import torch

    from mignon_ai_amd import Model, engine_option, gemm_i8_device, mgnn, quantize_f32, synth

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    engine_option("gemm", args.gemm)
    engine_option("attention", args.attention)
    engine_option("scan", args.scan)
    engine_option("operands", args.operands)
    engine_option("kv_rings", args.kv_rings)
    torch.cuda.set_device(0)
    # Everything runs on one non-default stream: the engine's launches, its HIP-event kernel timing and
    # the torch events bracketing the timed region.
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    name = args.config
    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic"}
    cpu = None

    if name == "copy":
        # The HBM counters' calibration: a device-to-device copy of a known size (rocprofv3 --pmc FETCH_SIZE,
        # then WRITE_SIZE, over this mode gives the factor by which those counters are scaled to bytes for
        # the engine's kernels), and the copy's own rate as the practical bandwidth ceiling.
        n = args.copy_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda")
        src.fill_(1)
        dst = torch.empty_like(src)

        def step():
            dst.copy_(src)

        ms, wall, _ = timed(step, args.warmup, args.steps, torch)
        gbs = 2 * n / (ms / 1e3) / 1e9
        out.update(metric="HBM device-to-device copy (counter calibration)", value=round(gbs, 1), unit="GB/s",
                   ms_per_step=round(ms, 4), dtype="u8",
                   config={"workload": f"copy of {args.copy_mib} MiB, read + write bytes per second",
                           "bytes_each_way": n})
        out["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": 2 * n, "kernel": "copy"}
        out["cpu_baseline"] = None
        return out
    if name == "append":
        a = append_latency(args.seed, cpu_seconds=0 if args.no_cpu_baseline else min(args.cpu_seconds, 10.0))
        us = a["us_per_token"]
        out.update(metric="single-session INT8 Append latency", value=us, unit="us/token", ms_per_step=round(us / 1e3, 5),
                   higher_is_better=False, config={"workload": a.pop("workload"), "context": APPEND_CONTEXT,
                                                   "appended": APPEND_TOKENS})
        out.update(a)
        out["roofline"] = None
        if "cpu_us_per_token" in a:
            cpu = {"value": a["cpu_us_per_token"], "unit": "us/token", "cores": 1, "kind": "port",
                   "sample": "the same prefill + 64 Appends through the oracle's session, repeated for up to 10 s"}
    elif name == "c2":
        c = synth.C2
        M, K, N = c["M"], c["K"], c["N"]
        A = (synth.u64_stream(args.seed, "A", M * K) % np.uint64(255)).astype(np.int64) - 127
        W = (synth.u64_stream(args.seed, "W", N * K) % np.uint64(255)).astype(np.int64) - 127
        A = A.astype(np.int8).reshape(M, K)
        W = W.astype(np.int8).reshape(N, K)
        s = (1e-3 + 9e-3 * synth.uniform(args.seed, "s", N)).astype(np.float32)
        dA, dW, ds = (torch.from_numpy(x).cuda() for x in (A, W, s))
        dC = torch.empty((M, N), dtype=torch.float32, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream

        def step():
            gemm_i8_device(dA, dW, ds, dC, None, stream)

        ms, wall, ms_prof = timed(step, args.warmup, args.steps, torch)
        bytes_ = M * K + N * K + 4 * N + 4 * M * N
        gbs = bytes_ / (ms / 1e3) / 1e9
        out.update(value=round(M / (ms / 1e3), 1), unit="tokens/s", ms_per_step=round(ms, 4),
                   config={"workload": "c2: INT8 GEMM A[262144x384] x W[512x384]^T, int32 accumulate, "
                                       "per-channel fp32 scale, fp32 out", "M": M, "K": K, "N": N})
        traffic, src = measured_traffic("c2", "gemm_i8")
        out["roofline"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                           "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic, "kernel": "gemm_i8",
                           "per_launch": bytes_, "avg_launch_ms": round(ms, 4)}
        if src:
            out["roofline"]["traffic_source"] = src
        if not args.no_cpu_baseline:
            cpu = cpu_baseline_gemm(A, W, s, args.cpu_seconds)
        out["wall_s"] = round(wall, 3)
    elif name == "score":
        from mignon_ai_amd.evaluate import score_sequences
        cfg = synth.CONFIGS["c3"]
        spec = cfg["spec"]
        data = mgnn.build_model_file(spec, args.seed, quantize_f32)
        m = Model(data)
        m.set_stream(torch.cuda.current_stream().cuda_stream)
        N, W = SCORE_TOKENS, SCORE_CONTEXT
        stream_ids = synth.token_ids(args.seed, "score:stream", (N,), spec.V)

        def step():
            score_sequences(m, [stream_ids], W)

        ms, wall, ms_prof = timed(step, args.warmup, args.steps, torch, before=lambda: m.profile(True))
        prof = m.profile_read()
        out["profiled_ms_per_step"] = round(ms_prof, 4)  # the second, instrumented pass
        m.profile(False)
        targets = N - 1
        rows = 1 + (N - 1 - W)
        positions = W + (rows - 1) * W
        out.update(value=round(targets / (ms / 1e3), 1), unit="targets/s", ms_per_step=round(ms, 4))
        out["config"] = {"workload": f"score: eval.Perplexity over a {N}-token stream, context {W}, of the c3 model "
                                     f"(D{spec.D} H{spec.H} {len(spec.blocks)} blocks heads {spec.heads} window "
                                     f"{spec.window} V{spec.V}); host token stream in, per-target log-probs out",
                         "tokens": N, "context": W, "window_rows": rows, "body_positions": positions,
                         "params": spec.n_params}
        work = class_work(prof)
        dom, roof = roofline_for(work, None)
        out["roofline"] = roof
        out["kernel_classes"] = class_table(work, args.steps)
        out["wall_s"] = round(wall, 3)
        if not args.no_cpu_baseline:
            cpu = cpu_baseline_score(data, stream_ids, W, args.cpu_seconds)
    elif name == "chat":
        from mignon_ai_amd.generate import Generator
        with open(os.path.join(ROOT, "tests", "golden", "orders.mgn"), "rb") as f:
            data = f.read()
        with open(os.path.join(ROOT, "tests", "golden", "orders_handwritten.json")) as f:
            requests = [p["instruction"].strip() for p in json.load(f)]
        g = Generator.from_bytes(data)
        g.model.set_stream(torch.cuda.current_stream().cuda_stream)
        batch = requests * CHAT_REPEAT
        res = [None]

        def step():
            res[0] = g.generate_batch(batch, CHAT_MAX_TOKENS)

        ms, wall, ms_prof = timed(step, args.warmup, args.steps, torch, before=lambda: g.model.profile(True))
        prof = g.model.profile_read()
        out["profiled_ms_per_step"] = round(ms_prof, 4)  # the second, instrumented pass
        g.model.profile(False)
        gen = sum(len(r.tokens) for r in res[0])
        out.update(value=round(len(batch) / (ms / 1e3), 1), unit="requests/s", ms_per_step=round(ms, 4))
        out["config"] = {"workload": f"chat: infer.Generate (greedy, chat template, max {CHAT_MAX_TOKENS} tokens) "
                                     f"for the {len(requests)} order-search requests x {CHAT_REPEAT} in one batch, "
                                     f"orders.mgn (the reference's trained 538k-parameter model); text in, text out",
                         "requests": len(batch), "generated_tokens": gen,
                         "generated_tokens_per_s": round(gen / (ms / 1e3), 1)}
        out["data"] = "the reference's order-search requests (tests/golden/orders_handwritten.json)"
        work = class_work(prof)
        out["kernel_classes"] = class_table(work, args.steps)
        out["roofline"] = roofline_for(work, None)[1]
        out["wall_s"] = round(wall, 3)
        if not args.no_cpu_baseline:
            cpu = cpu_baseline_chat(data, requests, CHAT_MAX_TOKENS, args.cpu_seconds)
    else:
        cfg = synth.CONFIGS["c4" if name == "sample" else name]
        spec = cfg["spec"]
        data = mgnn.build_model_file(spec, args.seed, quantize_f32)
        m = Model(data)
        m.set_stream(torch.cuda.current_stream().cuda_stream)
        macs = per_token_macs(spec)
        if name in ("c1", "c3", "c5"):
            B, T = cfg["B"], cfg["T"]
            ids = torch.from_numpy(synth.token_ids(args.seed, name + ":ids", (B, T), spec.V)).cuda()
            kw = {}
            if name == "c5":
                kw["probs"] = torch.empty((B, T, spec.V), dtype=torch.float32, device="cuda")
                kw["bits"] = torch.empty(B, dtype=torch.float32, device="cuda")
                outputs = "full softmax probabilities [B,T,V] fp32 + bits/token per sequence"
            elif name == "c3":
                kw["logits"] = torch.empty((B, T, spec.V), dtype=torch.float32, device="cuda")
                kw["logprob"] = torch.empty((B, T), dtype=torch.float32, device="cuda")
                outputs = "logits [B,T,V] fp32 + per-token log-probs"
            else:
                kw["logits"] = torch.empty((B, T, spec.V), dtype=torch.float32, device="cuda")
                outputs = "logits [B,T,V] fp32"

            def step():
                m.forward_batch_device(ids, **kw)

            tokens = B * T
            extra = None
            ms, wall, ms_prof = timed(step, args.warmup, args.steps, torch, before=lambda: m.profile(True))
            prof = m.profile_read()
            out["profiled_ms_per_step"] = round(ms_prof, 4)  # the second, instrumented pass
            m.profile(False)
            value = tokens / (ms / 1e3)
            out.update(value=round(value, 1), unit="tokens/s", ms_per_step=round(ms, 4))
            out["config"] = {"workload": f"{name}: {B} sequences x {T} tokens, D{spec.D} H{spec.H} "
                                         f"{len(spec.blocks)} blocks heads {spec.heads} window {spec.window} "
                                         f"V{spec.V}; {outputs}", "B": B, "T": T, "params": spec.n_params}
            if not args.no_cpu_baseline:
                cpu = cpu_baseline_forward(data, spec, B, T, args.cpu_seconds, args.seed)
        else:  # c4, sample
            S, P, G = cfg["B"], cfg["P"], cfg["G"]
            prompts_h = synth.token_ids(args.seed, "c4:prompts", (S, P), spec.V)
            prompts = torch.from_numpy(prompts_h).cuda()
            lens = torch.full((S,), P, dtype=torch.int32, device="cuda")
            oid = torch.empty((S, G), dtype=torch.int32, device="cuda")
            opb = torch.empty((S, G), dtype=torch.float64, device="cuda")
            sess = m.sessions(S)
            if name == "sample":
                seeds = list(range(S))

                def step():
                    sess.decode_sample(prompts_h, G, seeds, **SAMPLE_PARAMS)
            else:
                def step():
                    sess.decode_greedy_device(prompts, lens, G, oid, opb)

            # decode attention's bytes (the engine cannot state them: the spans live on the device): per
            # session, attention block and appended position, the K/V ring rows of the attended span in,
            # this position's q, k and v in (fp32), its K/V rows out and the output row out (limb planes and
            # scale). A ring row of all heads is 4D bytes, or packed 3D plus a 4-byte scale per head; the
            # set's device bytes tell which format the engine chose.
            packed = kv_rings_packed(spec, sess.device_bytes())
            nattn = len(spec.blocks) if spec.heads else 0
            Dp = -(-spec.D // 64) * 64
            row = 3 * spec.D + 4 * spec.heads if packed else 4 * spec.D  # unknown format: counted as fp32
            span = sum(min(p + 1, spec.window) for p in range(P, P + G - 1))
            per_pos = 12 * spec.D + 2 * row + 3 * Dp + 4
            extra = {"attention_step": args.steps * S * nattn * (2 * span * row + (G - 1) * per_pos)}
            out["kv_rings_packed"] = packed
            ms, wall, ms_prof = timed(step, args.warmup, args.steps, torch, before=lambda: m.profile(True))
            prof = m.profile_read()
            out["profiled_ms_per_step"] = round(ms_prof, 4)  # the second, instrumented pass
            m.profile(False)
            value = S * G / (ms / 1e3)
            out.update(value=round(value, 1), unit="generated tokens/s", ms_per_step=round(ms, 4))
            how = "greedy" if name == "c4" else "sampled (" + ", ".join(f"{k} {v}" for k, v in SAMPLE_PARAMS.items()) + ")"
            out["config"] = {"workload": f"{name}: {S} sessions, {P}-token prefill + {G} {how} tokens, D{spec.D} "
                                         f"H{spec.H} {len(spec.blocks)} blocks heads {spec.heads} window "
                                         f"{spec.window} V{spec.V}", "sessions": S, "prompt": P, "generated": G,
                             "params": spec.n_params}
            if not args.no_cpu_baseline:
                cpu = cpu_baseline_decode(data, spec, S, P, G, args.cpu_seconds, args.seed)
                if name == "sample":
                    cpu["sample"] += "; greedy choice in place of sampling (a lower bound of the reference's time)"
        work = class_work(prof, extra)
        dom, roof = roofline_for(work, name)
        out["roofline"] = roof
        total_macs = sum(v for k, v in macs.items() if k != "gemm_probs")
        tok = (cfg["B"] * cfg["T"]) if name not in ("c4", "sample") else cfg["B"] * (cfg["P"] + cfg["G"] - 1)
        path_tops = 2 * total_macs * tok / (ms / 1e3) / 1e12
        out["path_roofline"] = {"bound": "mfma", "achieved": round(path_tops, 2), "peak": PEAK_MFMA_TOPS,
                                "unit": "TFLOP/s", "frac": round(path_tops / PEAK_MFMA_TOPS, 4),
                                "note": "whole step: algorithmic int8 MACs x 2 (one pass of every weight "
                                        "GEMM; the probability head's recompute not counted)"}
        out["kernel_classes"] = class_table(work, args.steps)
        out["wall_s"] = round(wall, 3)
        if name == "c5" and not args.no_extras:
            # the one latency figure the reference publishes for this path, measured beside the headline
            out["single_session_append"] = append_latency(args.seed, repeats=10)
    out["cpu_baseline"] = cpu
    out["kernels"] = {"gemm": args.gemm, "attention": args.attention, "scan": args.scan, "operands": args.operands,
                      "kv_rings": args.kv_rings}
    return out


# Compact objects added to the c5 line: (key, configuration)
EXTRAS = [("decode", "c4"), ("c1", "c1"), ("c2", "c2"), ("c3", "c3"), ("score", "score"), ("sample", "sample"),
          ("chat", "chat")]


def kv_rings_packed(spec, device_bytes: int):
    """Whether a session set holds its K/V rings packed, from its device bytes per session
    (mg_sessions_device_bytes: the latch states and norm rings, nbs * (ring + 1) rows of Dp floats, plus
    per attention block two rings of cap rows of D floats, or packed 3D bytes and a scale per head);
    None when the figure is neither."""
    dil = [min(b.initial_dilation * b.dilation_base ** s, 32) for b in spec.blocks for s in range(b.steps)]
    ring = max(dil, default=0) + 1
    Dp = -(-spec.D // 64) * 64
    nattn = len(spec.blocks) if spec.heads else 0
    cap = spec.window if spec.window > 0 else spec.context
    base = sum(b.steps for b in spec.blocks) * (ring + 1) * Dp * 4 + 8
    fp32 = base + nattn * 2 * cap * spec.D * 4
    packed = base + nattn * 2 * cap * (3 * spec.D + 4 * spec.heads)
    return True if device_bytes == packed else False if device_bytes == fp32 else None


def compact(r):
    """The figures of one configuration's line that the headline carries: its throughput and step time,
    the roofline of its dominant kernel class (for a decode, also decode attention's fraction of HBM) and
    its CPU baseline."""
    c = {"workload": r["config"]["workload"], "value": r["value"], "unit": r["unit"], "ms_per_step": r["ms_per_step"],
         "steps": r["steps"]}
    roof = r.get("roofline")
    if roof:
        c["roofline"] = {k: roof[k] for k in ("kernel", "bound", "achieved", "unit", "frac") if k in roof}
    path = r.get("path_roofline")
    if path:
        c["path_roofline_frac"] = path["frac"]
    att = r.get("kernel_classes", {}).get("attention_step")
    if att and "frac" in att:
        c["decode_attention"] = {"ms_per_step": att["ms_per_step"], "bound": att["bound"], "achieved": att["achieved"],
                                 "unit": att["unit"], "frac": att["frac"]}
    for k in ("generated_tokens", "generated_tokens_per_s"):
        if k in r["config"]:
            c[k] = r["config"][k]
    cpu = r.get("cpu_baseline")
    if cpu:
        c["cpu_baseline"] = {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample") if k in cpu}
        if cpu.get("value"):
            c["gpu_over_cpu"] = round(r["value"] / cpu["value"], 1) if not r.get("higher_is_better") is False else None
    return c


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c5", choices=["c1", "c2", "c3", "c4", "c5", "score", "chat", "sample",
                                                       "append", "copy"])
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="c5 only: leave out the compact objects of the other configurations and the Append "
                         "latency (so that a profile of the run holds c5's own launches only)")
    ap.add_argument("--copy-mib", type=int, default=1024, help="--config copy: bytes copied each way (MiB)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--gemm", default="auto", choices=["auto", "stream", "slab"],
                    help="limb-expanded GEMM kernel (mg_engine_option); both give identical results")
    ap.add_argument("--attention", default="auto", choices=["auto", "exact", "mfma"],
                    help="attention kernel (mg_engine_option): reference order or matrix cores")
    ap.add_argument("--operands", default="auto", choices=["auto", "limbs", "fp32"],
                    help="batched forward: GLU and attention outputs as limb planes written by a row pass, or read "
                         "as fp32 by the GEMMs that take them (mg_engine_option)")
    ap.add_argument("--scan", default="auto", choices=["auto", "separate", "fused"],
                    help="latch scan and rule-input packing as two kernels or one (mg_engine_option); both "
                         "give identical results")
    ap.add_argument("--kv-rings", default="auto", choices=["auto", "fp32", "packed"],
                    help="decodes: session K/V rings as fp32 rows or packed 24-bit mantissas with a power-of-two "
                         "scale per row (mg_engine_option)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the path shards by sequence (one process "
                                   "per GPU on its share of the batch, weights replicated, no exchange step), "
                                   "so N>1 is not run",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    out = run(args)
    if args.config == "c5" and not args.no_extras:
        # every other configuration and workload from the same run, each as a compact object: c4's decode
        # first (the metric's "+ decode"), then c1-c3, scoring, sampled decode and chat
        for key, cfg in EXTRAS:
            sub = argparse.Namespace(**vars(args))
            sub.config = cfg
            sub.cpu_seconds = args.cpu_seconds / 4
            out[key] = compact(run(sub))
            print(f"[bench] {key} done", file=sys.stderr, flush=True)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
