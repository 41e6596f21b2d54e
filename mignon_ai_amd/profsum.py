"""Summaries of rocprofv3 output as short markdown tables (what the profiles/ folder holds).

    python -m mignon_ai_amd.profsum stats OUT.md CMD  STATS.csv
        per-kernel launch count, average and total duration from `rocprofv3 --kernel-trace --stats`
    python -m mignon_ai_amd.profsum pmc OUT.md CMD  COUNTERS.csv [...] [--calib BYTES CAL.csv [...]]
        per-kernel average of every counter per dispatch from `rocprofv3 --pmc` runs; with --calib, the
        copy kernel in the CAL files moved BYTES each way per dispatch, and FETCH_SIZE / WRITE_SIZE of
        every kernel are also given in bytes, scaled by the copy kernel's counter-to-bytes ratio, under
        the engine's kernel-class name (what bench.py reports and reads back as roofline traffic)

    python -m mignon_ai_amd.profsum clock OUT.md CMD  COUNTERS.csv AGENT_INFO.csv
        per kernel from one `rocprofv3 --pmc GRBM_GUI_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_VALU`
        run: the average shader clock over the dispatch (GPU-active cycles per XCD over the dispatch's
        duration) and the fraction of SIMD cycles the matrix core and the VALU were busy

    python -m mignon_ai_amd.profsum memory OUT.md CMD  PASS.csv [...] AGENT_INFO.csv
        per kernel from the `rocprofv3 --pmc` runs of MEMORY_PASSES (one run each): shader clock, matrix-core
        busy and VALU co-execution, L2 and address-unit busy, L2 hit rate, L1-to-L2 read traffic and latency

CMD is the command line that produced the files, recorded in the summary.
"""
from __future__ import annotations

import csv
import re
import sys
from collections import defaultdict


def _short(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "").replace("mg::", "")
    return re.sub(r"\(mg::GemmArgs.*\)|\(mg::RowArgs.*\)|\(.*\)$", "", name).strip()[:80]


def stats(out: str, cmd: str, path: str) -> None:
    rows = list(csv.DictReader(open(path)))
    lines = [f"Command (from the repository root, one MI355X):", "", "```", cmd, "```", "",
             "| kernel | calls | avg ms | total ms | % |", "|---|---:|---:|---:|---:|"]
    for r in rows:
        if float(r["Percentage"]) < 0.05:
            continue
        lines.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e6:.4f} | "
                     f"{float(r['TotalDurationNs']) / 1e6:.2f} | {float(r['Percentage']):.1f} |")
    _write(out, lines)


# kernel name -> the engine's kernel class (mg_model_profile names; GEMM classes by epilogue number)
_GEMM_EPI = {1: "gemm_qkv", 2: "gemm_latch", 3: "gemm_glu", 4: "gemm_highway", 5: "gemm_out", 6: "gemm_logits",
             7: "gemm_probs"}
_CLASSES = [("gemm_c2_kernel", "gemm_i8"), ("row_kernel", "row_norm_pack"), ("scan_rule_kernel", "latch_scan"),
            ("scan_kernel", "latch_scan"),
            ("latch_step_kernel", "latch_step"), ("attention_step", "attention_step"),
            ("qkv_attention_kernel", "qkv_attention"), ("attention", "attention"), ("head_combine_kernel", "head_combine"), ("bits_kernel", "bits"),
            ("export_", "state_export"), ("step1_kernel", "session_step"), ("tile_step_kernel", "tile_step")]


def kernel_class(name: str) -> str:
    m = re.search(r"gemm_(?:slab|lx|slab_fa)_kernel<(\d+)", name)
    if m:
        return _GEMM_EPI.get(int(m.group(1)), "")
    for key, cls in _CLASSES:
        if key in name:
            return cls
    return ""


def _counters(paths: list[str]):
    acc = defaultdict(lambda: defaultdict(list))  # kernel -> counter -> values per dispatch
    for p in paths:
        per_dispatch = defaultdict(float)
        names = {}
        for r in csv.DictReader(open(p)):
            key = (r["Dispatch_Id"], r["Counter_Name"])
            per_dispatch[key] += float(r["Counter_Value"])  # sum over dimensions (XCC, SE) if split
            names[r["Dispatch_Id"]] = r["Kernel_Name"]
        for (d, c), v in per_dispatch.items():
            acc[_short(names[d])][c].append(v)
    return acc


def _avg(v):
    return sum(v) / len(v)


def pmc(out: str, cmd: str, paths: list[str], calib: tuple[int, list[str]] | None) -> None:
    acc = _counters(paths)
    counters = sorted({c for k in acc.values() for c in k})
    lines = [f"Command(s) (from the repository root, one MI355X):", "", "```", cmd, "```", "",
             "Average per dispatch (FETCH_SIZE / WRITE_SIZE in KiB as the counters report them).", ""]
    lines += ["| kernel | dispatches | " + " | ".join(counters) + " |",
              "|---|---:|" + "---:|" * len(counters)]
    for k in sorted(acc):
        n = max(len(v) for v in acc[k].values())
        cells = [f"{_avg(acc[k][c]):.4g}" if acc[k].get(c) else "" for c in counters]
        lines.append(f"| `{k}` | {n} | " + " | ".join(cells) + " |")
    if calib:
        nbytes, cal_paths = calib
        cal = _counters(cal_paths)
        ck = [k for k in cal if "copyBuffer" in k or "copy" in k.lower()]
        if ck:
            lines += ["", f"Calibration: `{ck[0]}` (a device-to-device copy) moves {nbytes} bytes each way per "
                          "dispatch.", ""]
            factors = {}
            for c in ("FETCH_SIZE", "WRITE_SIZE"):
                v = cal[ck[0]].get(c)
                if v:
                    factors[c] = nbytes / _avg(v)
                    lines.append(f"- {c}: {_avg(v):.6g} per dispatch -> {factors[c]:.1f} bytes per counter unit")
            lines += ["", "HBM traffic per dispatch (counter x factor):", "",
                      "| class | kernel | read bytes | write bytes | total bytes |", "|---|---|---:|---:|---:|"]
            for k in sorted(acc):
                rd, wr = acc[k].get("FETCH_SIZE"), acc[k].get("WRITE_SIZE")
                if not (rd and wr and "FETCH_SIZE" in factors and "WRITE_SIZE" in factors):
                    continue
                r_b, w_b = _avg(rd) * factors["FETCH_SIZE"], _avg(wr) * factors["WRITE_SIZE"]
                lines.append(f"| {kernel_class(k) or '-'} | `{k}` | {r_b:.6g} | {w_b:.6g} | {r_b + w_b:.6g} |")
    _write(out, lines)


def traffic_for(path: str, cls: str) -> float | None:
    """Total HBM bytes per dispatch recorded for a kernel class in a summary written by `pmc` (the
    kernel with the most bytes when several implement the class), or None."""
    try:
        text = open(path).read()
    except OSError:
        return None
    best = None
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[0] == cls:
            try:
                v = float(cells[4])
            except ValueError:
                continue
            best = v if best is None else max(best, v)
    return best


def clock(out: str, cmd: str, path: str, agent_path: str) -> None:
    gpu = [a for a in csv.DictReader(open(agent_path)) if a["Agent_Type"] == "GPU"][0]
    nxcc, simds, cus = int(gpu["Num_Xcc"]), int(gpu["Simd_Count"]), int(gpu["Cu_Count"])
    fmax = float(gpu["Max_Engine_Clk_Fcompute"]) / 1e3
    per = defaultdict(dict)  # dispatch -> counter -> value (summed over dimensions), plus duration
    names = {}
    for r in csv.DictReader(open(path)):
        d = r["Dispatch_Id"]
        per[d][r["Counter_Name"]] = per[d].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        per[d]["ns"] = float(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        names[d] = _short(r["Kernel_Name"])
    acc = defaultdict(lambda: defaultdict(float))
    for d, v in per.items():
        k = acc[names[d]]
        k["n"] += 1
        for c, x in v.items():
            k[c] += x
    lines = [f"Command (from the repository root, one MI355X):", "", "```", cmd, "```", "",
             f"Shader clock: GRBM_GUI_ACTIVE per XCD ({nxcc} XCDs) over the dispatch duration (maximum "
             f"{fmax:.2f} GHz). Matrix core busy: SQ_VALU_MFMA_BUSY_CYCLES over the {simds} SIMDs' cycles "
             "(rocprofv3's MfmaUtil); VALU busy: SQ_ACTIVE_INST_VALU over the CUs' cycles (its VALUBusy). "
             "Kernels with at least 0.5% of the run's kernel time; for dispatches of a few tens of "
             "microseconds the clock figure is approximate (the counter's window is wider than the "
             "dispatch).", "",
             "| kernel | dispatches | avg ms | clock GHz | matrix core busy | VALU busy |",
             "|---|---:|---:|---:|---:|---:|"]
    total_ns = sum(v["ns"] for v in acc.values())
    for k, v in sorted(acc.items(), key=lambda kv: -kv[1]["ns"]):
        n = v["n"]
        cyc = v["GRBM_GUI_ACTIVE"] / n / nxcc
        ms = v["ns"] / n / 1e6
        if cyc <= 0 or v["ns"] < 0.005 * total_ns:
            continue
        mf = v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / n / (cyc * simds)
        va = v.get("SQ_ACTIVE_INST_VALU", 0.0) / n / (cyc * cus)
        lines.append(f"| `{k}` | {int(n)} | {ms:.3f} | {cyc / (ms * 1e-3) / 1e9:.2f} | {100 * mf:.1f}% | "
                     f"{100 * va:.1f}% |")
    _write(out, lines)


def clock_for(path: str, cls: str) -> dict | None:
    """Shader clock and busy fractions recorded by `clock` for a kernel class (the kernel with the most
    time when several implement the class), or None."""
    try:
        text = open(path).read()
    except OSError:
        return None
    best, best_ms = None, -1.0
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) != 6 or not cells[0].startswith("`") or kernel_class(cells[0]) != cls:
            continue
        try:
            n, ms, ghz = int(cells[1]), float(cells[2]), float(cells[3])
            mf, va = float(cells[4].rstrip("%")) / 100, float(cells[5].rstrip("%")) / 100
        except ValueError:
            continue
        if n * ms > best_ms:
            best, best_ms = {"clock_ghz": ghz, "matrix_core_busy": mf, "valu_busy": va}, n * ms
    return best


# memory mode: the counters of its passes (one rocprofv3 --pmc run each)
MEMORY_PASSES = [
    "TA_BUSY_avr TCP_TCC_READ_REQ_sum TCP_TCC_READ_REQ_LATENCY_sum",
    "TCC_HIT_sum TCC_MISS_sum TCC_BUSY_avr",
    "SQ_VALU_MFMA_BUSY_CYCLES SQ_VALU_MFMA_COEXEC_CYCLES GRBM_GUI_ACTIVE",
]


def memory(out: str, cmd: str, paths: list[str], agent_path: str) -> None:
    """Per kernel, from the memory passes' CSVs: shader clock, matrix-core busy and how much of it had a VALU
    instruction co-executing, L2 (TCC) busy, address unit (TA) busy, L2 hit rate, L1-to-L2 read requests
    (128 bytes each) and their mean latency."""
    gpu = [a for a in csv.DictReader(open(agent_path)) if a["Agent_Type"] == "GPU"][0]
    nxcc, simds = int(gpu["Num_Xcc"]), int(gpu["Simd_Count"])
    acc = defaultdict(lambda: defaultdict(float))
    for p in paths:
        per = defaultdict(dict)
        names = {}
        for r in csv.DictReader(open(p)):
            d = r["Dispatch_Id"]
            per[d][r["Counter_Name"]] = per[d].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            per[d]["ns"] = float(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
            names[d] = _short(r["Kernel_Name"])
        for d, v in per.items():
            k = acc[names[d]]
            for c, x in v.items():
                if c == "ns":
                    k["ns"] += x
                    k["n"] += 1
                else:
                    k[c] += x
    lines = [f"Command (from the repository root, one MI355X):", "", "```", cmd, "```", "",
             f"Per kernel (dispatches of all passes; counters averaged per dispatch): shader clock from "
             f"GRBM_GUI_ACTIVE per XCD ({nxcc} XCDs); matrix core busy = SQ_VALU_MFMA_BUSY_CYCLES over the "
             f"{simds} SIMDs' cycles, and the share of those cycles with a VALU instruction co-executing "
             "(SQ_VALU_MFMA_COEXEC_CYCLES); L2 busy = TCC_BUSY_avr and address unit busy = TA_BUSY_avr over "
             "the XCD cycles; L2 hit rate from TCC_HIT/TCC_MISS; L1-to-L2 read requests (128 bytes each) "
             "per dispatch in GB and their mean latency in cycles (TCP_TCC_READ_REQ_LATENCY over "
             "TCP_TCC_READ_REQ). Kernels with at least 0.5% of the run's kernel time.", "",
             "| kernel | avg ms | clock GHz | matrix busy | co-exec | L2 busy | TA busy | L2 hit | L1→L2 GB | latency |",
             "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    total_ns = sum(v["ns"] for v in acc.values())
    for k, v in sorted(acc.items(), key=lambda kv: -kv[1]["ns"]):
        n = v["n"]
        if n == 0 or v["ns"] < 0.005 * total_ns:
            continue
        ms = v["ns"] / n / 1e6
        npass = len(paths)
        per_pass = n / npass  # dispatches of this kernel per pass
        cyc = v["GRBM_GUI_ACTIVE"] / per_pass / nxcc if v.get("GRBM_GUI_ACTIVE") else 0.0
        if cyc <= 0:
            continue
        mf = v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / per_pass / (cyc * simds)
        co = v.get("SQ_VALU_MFMA_COEXEC_CYCLES", 0.0) / max(v.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0), 1.0)
        l2 = v.get("TCC_BUSY_avr", 0.0) / per_pass / cyc
        ta = v.get("TA_BUSY_avr", 0.0) / per_pass / cyc
        hits, miss = v.get("TCC_HIT_sum", 0.0), v.get("TCC_MISS_sum", 0.0)
        req = v.get("TCP_TCC_READ_REQ_sum", 0.0) / per_pass
        lat = v.get("TCP_TCC_READ_REQ_LATENCY_sum", 0.0) / max(v.get("TCP_TCC_READ_REQ_sum", 0.0), 1.0)
        lines.append(f"| `{k}` | {ms:.3f} | {cyc / (ms * 1e-3) / 1e9:.2f} | {100 * mf:.1f}% | {100 * co:.0f}% | "
                     f"{100 * l2:.0f}% | {100 * ta:.0f}% | {100 * hits / max(hits + miss, 1.0):.0f}% | "
                     f"{req * 128 / 1e9:.2f} | {lat:.0f} |")
    _write(out, lines)


def _write(out: str, lines: list[str]) -> None:
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")


def main(argv: list[str]) -> None:
    if len(argv) < 4 or argv[0] not in ("stats", "pmc", "clock", "memory"):
        raise SystemExit(__doc__)
    mode, out, cmd, rest = argv[0], argv[1], argv[2], argv[3:]
    if mode == "stats":
        stats(out, cmd, rest[0])
        return
    if mode == "memory":
        memory(out, cmd, rest[:-1], rest[-1])
        return
    if mode == "clock":
        clock(out, cmd, rest[0], rest[1])
        return
    calib = None
    if "--calib" in rest:
        i = rest.index("--calib")
        calib = (int(rest[i + 1]), rest[i + 2:])
        rest = rest[:i]
    pmc(out, cmd, rest, calib)


if __name__ == "__main__":
    main(sys.argv[1:])
