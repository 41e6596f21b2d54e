"""Summaries of rocprofv3 output as short markdown tables (what the profiles/ folder holds).

    python -m mignon_ai_amd.profsum stats OUT.md CMD  STATS.csv
        per-kernel launch count, average and total duration from `rocprofv3 --kernel-trace --stats`
    python -m mignon_ai_amd.profsum pmc OUT.md CMD  COUNTERS.csv [COUNTERS.csv ...] [--calib REGEX BYTES]
        per-kernel average of every counter per dispatch from `rocprofv3 --pmc` runs; with --calib, the
        dispatches of the kernel matching REGEX moved BYTES each way, and FETCH_SIZE / WRITE_SIZE of
        every kernel are also given in bytes scaled by that kernel's counter-to-bytes ratio

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


def pmc(out: str, cmd: str, paths: list[str], calib: tuple[str, int] | None) -> None:
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
    counters = sorted({c for k in acc.values() for c in k})
    lines = [f"Command(s) (from the repository root, one MI355X):", "", "```", cmd, "```", "",
             "Average per dispatch (FETCH_SIZE / WRITE_SIZE in KiB as the counters report them).", ""]
    lines += ["| kernel | dispatches | " + " | ".join(counters) + " |",
              "|---|---:|" + "---:|" * len(counters)]
    for k in sorted(acc):
        n = max(len(v) for v in acc[k].values())
        cells = []
        for c in counters:
            v = acc[k].get(c)
            cells.append(f"{sum(v) / len(v):.4g}" if v else "")
        lines.append(f"| `{k}` | {n} | " + " | ".join(cells) + " |")
    if calib:
        rx, nbytes = re.compile(calib[0]), calib[1]
        ck = [k for k in acc if rx.search(k)]
        if ck:
            lines += ["", f"Calibration: `{ck[0]}` copies {nbytes} bytes per dispatch.", ""]
            factors = {}
            for c in ("FETCH_SIZE", "WRITE_SIZE"):
                v = acc[ck[0]].get(c)
                if v:
                    factors[c] = nbytes / (sum(v) / len(v))
                    lines.append(f"- {c}: {sum(v) / len(v):.6g} per dispatch -> {factors[c]:.2f} bytes per unit")
            lines += ["", "| kernel | HBM read bytes/dispatch | HBM write bytes/dispatch |", "|---|---:|---:|"]
            for k in sorted(acc):
                cells = []
                for c in ("FETCH_SIZE", "WRITE_SIZE"):
                    v = acc[k].get(c)
                    cells.append(f"{sum(v) / len(v) * factors[c]:.4g}" if v and c in factors else "")
                lines.append(f"| `{k}` | " + " | ".join(cells) + " |")
    _write(out, lines)


def _write(out: str, lines: list[str]) -> None:
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")


def main(argv: list[str]) -> None:
    if len(argv) < 4 or argv[0] not in ("stats", "pmc"):
        raise SystemExit(__doc__)
    mode, out, cmd, rest = argv[0], argv[1], argv[2], argv[3:]
    if mode == "stats":
        stats(out, cmd, rest[0])
        return
    calib = None
    if "--calib" in rest:
        i = rest.index("--calib")
        calib = (rest[i + 1], int(rest[i + 2]))
        rest = rest[:i] + rest[i + 3:]
    pmc(out, cmd, rest, calib)


if __name__ == "__main__":
    main(sys.argv[1:])
