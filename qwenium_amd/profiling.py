"""Summaries of rocprofv3 CSV output (``--output-format csv``) for the MoE kernels.

    python -m qwenium_amd.profiling stats <prefix>_kernel_stats.csv
        per-kernel calls / average / total duration as a markdown table

    python -m qwenium_amd.profiling medians <prefix>_kernel_trace.csv [--prefix qmoe::]
        per-dispatch median / mean duration, VGPRs and grid of the matching kernels

    python -m qwenium_amd.profiling counters <prefix>_counter_collection.csv [--kernel SUBSTR]
        per-kernel mean of every collected counter (one dispatch = one sample)

    python -m qwenium_amd.profiling mfma <prefix>_counter_collection.csv [--kernel SUBSTR]
        per-kernel MFMA-pipe ratios from a run that collected GRBM_GUI_ACTIVE,
        SQ_VALU_MFMA_BUSY_CYCLES, SQ_VALU_MFMA_COEXEC_CYCLES, SQ_INSTS_MFMA,
        SQ_INSTS_VALU and SQ_INSTS_SALU: the kernel's cycles (GRBM_GUI_ACTIVE is
        summed over the XCDs: it reads 8 x 2.4 GHz x the duration of a timed
        sleep kernel), the fraction of SIMD-cycles the MFMA pipe is busy, the
        share of those in which a VALU instruction co-issues, and the VALU and
        SALU instructions per MFMA instruction

    python -m qwenium_amd.profiling traffic --fetch F.csv --write W.csv --kernel SUBSTR \
            --copy-mib N [--workload NAME] [--out profiles/traffic_<workload>.json]
        HBM bytes per launch of one kernel from a FETCH_SIZE run and a
        WRITE_SIZE run, each scaled by what the same counter reads for the
        calibration copy (torch D2D copy of N MiB, the ``__amd_rocclr_copyBuffer``
        dispatches of ``bench.py --copy-mib N``): factor = N MiB / counter KiB.
"""
from __future__ import annotations

import argparse
import csv
import json
import sys
from collections import defaultdict

COPY_KERNEL = "__amd_rocclr_copyBuffer"


def _rows(path: str):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def kernel_stats(path: str) -> str:
    rows = _rows(path)
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    out = ["| kernel | calls | avg us | min us | max us | total us | % |", "|---|---:|---:|---:|---:|---:|---:|"]
    for r in rows:
        out.append("| `%s` | %s | %.2f | %.2f | %.2f | %.1f | %.2f |" % (
            r["Name"][:110], r["Calls"], float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3,
            float(r["MaxNs"]) / 1e3, float(r["TotalDurationNs"]) / 1e3, float(r["Percentage"])))
    return "\n".join(out)


def dispatch_medians(path: str, prefix: str = "qmoe::") -> str:
    """Markdown table of per-dispatch durations of kernels whose name contains `prefix`."""
    durs = defaultdict(list)
    info = {}
    for r in _rows(path):
        name = r["Kernel_Name"]
        if prefix not in name:
            continue
        durs[name].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        info[name] = (r.get("Workgroup_Size_X"), r.get("Grid_Size_X"))
    out = ["| kernel | dispatches | median us | mean us | workgroup | grid (threads, last dispatch) |",
           "|---|---:|---:|---:|---:|---:|"]
    for name, d in sorted(durs.items(), key=lambda kv: -sum(kv[1])):
        d = sorted(d)
        wg, g = info[name]
        out.append("| `%s` | %d | %.2f | %.2f | %s | %s |" % (name[:110], len(d), d[len(d) // 2], sum(d) / len(d), wg, g))
    return "\n".join(out)


def counter_means(path: str, kernel: str | None = None) -> dict:
    """{kernel name: {counter: mean over dispatches}} (counters summed over the
    dimensions rocprofv3 reports them in, per dispatch)."""
    rows = _rows(path)
    per = defaultdict(lambda: defaultdict(float))  # (kernel, dispatch) -> counter -> value
    for r in rows:
        name = r.get("Kernel_Name") or r.get("Kernel-Name") or ""
        if kernel and kernel not in name:
            continue
        disp = r.get("Dispatch_Id") or r.get("Correlation_Id")
        per[(name, disp)][r["Counter_Name"]] += float(r["Counter_Value"])
    acc = defaultdict(lambda: defaultdict(list))
    for (name, _), cs in per.items():
        for c, v in cs.items():
            acc[name][c].append(v)
    return {n: {c: sum(v) / len(v) for c, v in cs.items()} | {"dispatches": len(next(iter(cs.values())))}
            for n, cs in acc.items()}


def mfma_ratios(path: str, kernel: str | None = None, xcds: int = 8, simds: int = 1024) -> str:
    """Markdown table of the MFMA-pipe ratios of every kernel with MFMA instructions."""
    means = counter_means(path, kernel)
    out = ["| kernel | dispatches | cycles per dispatch | MFMA busy (of SIMD-cycles) | VALU co-issue (of MFMA-busy) "
           "| VALU instr / MFMA instr | SALU instr / MFMA instr |",
           "|---|---:|---:|---:|---:|---:|---:|"]
    for n, m in sorted(means.items()):
        if not m.get("SQ_INSTS_MFMA"):
            continue
        cyc = m["GRBM_GUI_ACTIVE"] / xcds
        busy = m["SQ_VALU_MFMA_BUSY_CYCLES"]
        out.append("| `%s` | %d | %.4g | %.3f | %.3f | %.2f | %.2f |" % (
            n[:90], m["dispatches"], cyc, busy / (simds * cyc), m["SQ_VALU_MFMA_COEXEC_CYCLES"] / busy,
            m["SQ_INSTS_VALU"] / m["SQ_INSTS_MFMA"], m["SQ_INSTS_SALU"] / m["SQ_INSTS_MFMA"]))
    return "\n".join(out)


def copy_counter(path: str, counter: str) -> float:
    """Mean counter value of the calibration copies: the runtime's copy kernel
    also serves small copies, so only dispatches within 2x of the largest count."""
    vals = defaultdict(float)
    for r in _rows(path):
        if r.get("Kernel_Name") == COPY_KERNEL and r["Counter_Name"] == counter:
            vals[r.get("Dispatch_Id") or r.get("Correlation_Id")] += float(r["Counter_Value"])
    if not vals:
        raise SystemExit(f"no {COPY_KERNEL} dispatch with counter {counter}: run bench.py with --copy-mib")
    top = max(vals.values())
    big = [v for v in vals.values() if v >= 0.5 * top]
    return sum(big) / len(big)


def _one(means: dict, substr: str, counter: str) -> tuple[str, float, int]:
    hits = [(n, m) for n, m in means.items() if substr in n and counter in m]
    if not hits:
        raise SystemExit(f"no dispatch of a kernel matching {substr!r} with counter {counter}")
    n, m = max(hits, key=lambda nm: nm[1]["dispatches"])
    return n, m[counter], int(m["dispatches"])


def traffic(fetch_csv: str, write_csv: str, kernel: str, copy_mib: float, workload: str) -> dict:
    fm = counter_means(fetch_csv, kernel)
    wm = counter_means(write_csv, kernel)
    kname, fetch_kib, nf = _one(fm, kernel, "FETCH_SIZE")
    _, write_kib, nw = _one(wm, kernel, "WRITE_SIZE")
    copy_fetch = copy_counter(fetch_csv, "FETCH_SIZE")
    copy_write = copy_counter(write_csv, "WRITE_SIZE")
    copy_kib = copy_mib * 1024.0
    f_fetch = copy_kib / copy_fetch
    f_write = copy_kib / copy_write
    return {
        "workload": workload, "kernel": kname, "dispatches": [nf, nw],
        "fetch_kib_raw": fetch_kib, "write_kib_raw": write_kib,
        "copy_mib": copy_mib, "copy_fetch_kib_raw": copy_fetch, "copy_write_kib_raw": copy_write,
        "fetch_scale": f_fetch, "write_scale": f_write,
        "hbm_bytes_per_launch": (fetch_kib * f_fetch + write_kib * f_write) * 1024.0,
        "fetch_bytes_per_launch": fetch_kib * f_fetch * 1024.0,
        "write_bytes_per_launch": write_kib * f_write * 1024.0,
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    m = sub.add_parser("medians")
    m.add_argument("csv")
    m.add_argument("--prefix", default="qmoe::")
    c = sub.add_parser("counters")
    c.add_argument("csv")
    c.add_argument("--kernel", default=None)
    f = sub.add_parser("mfma")
    f.add_argument("csv")
    f.add_argument("--kernel", default=None)
    f.add_argument("--xcds", type=int, default=8)
    f.add_argument("--simds", type=int, default=1024, help="SIMDs on the device (256 CUs x 4 on MI355X)")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-mib", type=float, required=True)
    t.add_argument("--workload", default="decode")
    t.add_argument("--out", default=None)
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print(kernel_stats(a.csv))
    elif a.cmd == "medians":
        print(dispatch_medians(a.csv, a.prefix))
    elif a.cmd == "mfma":
        print(mfma_ratios(a.csv, a.kernel, a.xcds, a.simds))
    elif a.cmd == "counters":
        means = counter_means(a.csv, a.kernel)
        names = sorted({c for m in means.values() for c in m})
        print("| kernel | " + " | ".join(names) + " |")
        print("|---|" + "---:|" * len(names))
        for n, m in sorted(means.items()):
            print(f"| `{n[:90]}` | " + " | ".join("%.4g" % m.get(c, float("nan")) for c in names) + " |")
    else:
        res = traffic(a.fetch, a.write, a.kernel, a.copy_mib, a.workload)
        txt = json.dumps(res, indent=1)
        if a.out:
            with open(a.out, "w") as f:
                f.write(txt + "\n")
        print(txt)
    return 0


if __name__ == "__main__":
    sys.exit(main())
