"""Turn the rocprofv3 CSV output of profile_rocprof.sh into a report.

    python rocprof_extract.py --root DIR --out report.md [--json report.json]

DIR holds one sub-directory per workload (names from profile_workload.py),
each with up to four rocprofv3 runs:

    trace/run_kernel_stats.csv        --kernel-trace --stats
    fetch/run_counter_collection.csv  --pmc FETCH_SIZE
    write/run_counter_collection.csv  --pmc WRITE_SIZE
    sq/run_counter_collection.csv     --pmc MfmaUtil MfmaFlopsF16 LdsBankConflict OccupancyPercent

and optionally DIR/occupancy.json (flashattn_cuda.occupancy_report()).

Per workload and kernel the report gives: calls, average / min / max
duration, HBM bytes read and written per dispatch (FETCH_SIZE and WRITE_SIZE,
each in KiB, scaled by the factor that makes the copy_1g workload's 1 GiB
copy read and write exactly 1 GiB), MFMA utilisation, fp16 MFMA FLOPs per
dispatch, LDS bank conflicts per access and occupancy; for the workload's main
kernel also the achieved rate of its algorithmic work (FLOP/s or B/s) against
the MI355X peaks. It is the counterpart of the reference's
bench/ncu_extract.py (which turns Nsight Compute exports into summary.md),
kept separate from the capture so the parsing is tested without a GPU.
"""

from __future__ import annotations

import argparse
import csv
import json
import os
import shutil
import statistics
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from profile_workload import WORKLOADS  # noqa: E402

MFMA_FP16_PEAK_FLOPS = 2516.6e12  # MI355X dense fp16 MFMA
HBM_PEAK_BYTES = 8.0e12           # MI355X HBM3E
COPY_BYTES = float(1 << 30)       # the calibration copy reads and writes 1 GiB


_LITERAL_TYPES = {"b": "bool", "i": "int", "j": "unsigned", "l": "long", "m": "unsigned long"}


def _demangle_nested(name: str) -> str | None:
    """The name part of `_ZN <source-name>+ [I <literal args> E] E ...` or
    `_Z <source-name> [I ... E] ...`, with integer and bool literal template
    arguments (`Lb1E` -> true, `Li8E` -> 8): enough for this library's
    kernels, whose argument lists the report drops anyway. None when the
    name has another form."""
    i = 2
    nested = name.startswith("_ZN")
    if nested:
        i = 3
    parts = []
    while i < len(name) and name[i].isdigit():
        j = i
        while j < len(name) and name[j].isdigit():
            j += 1
        n = int(name[i:j])
        ident = name[j:j + n]
        if len(ident) != n:
            return None
        parts.append("(anonymous namespace)" if ident.startswith("_GLOBAL__N") else ident)
        i = j + n
        if not nested:
            break
    if not parts:
        return None
    text = "::".join(parts)
    if i < len(name) and name[i] == "I":
        args = []
        i += 1
        while i < len(name) and name[i] == "L":
            j = name.find("E", i)
            if j < 0 or name[i + 1] not in _LITERAL_TYPES:
                return None
            kind, value = name[i + 1], name[i + 2:j]
            if kind == "b":
                args.append("true" if value == "1" else "false")
            else:
                args.append(value.replace("n", "-", 1) if value.startswith("n") else value)
            i = j + 1
        if i >= len(name) or name[i] != "E":
            return None
        text += "<" + ", ".join(args) + ">"
    return text + "()"


def demangle(name: str) -> str:
    """Itanium-mangled names (`_Z...`): c++filt when it is installed and
    understands the name (older ones reject the _Float16 mangling), else the
    small literal-template demangler above; other names are unchanged."""
    if not name.startswith("_Z"):
        return name
    tool = shutil.which("c++filt")
    if tool is not None:
        out = subprocess.run([tool, name], capture_output=True, text=True,
                             check=False).stdout.strip()
        if out and not out.startswith("_Z"):
            return out
    return _demangle_nested(name) or name


def _mask_templates(text: str) -> str:
    """`text` with every character between a template's outer brackets
    replaced by '.', nested brackets included; the outer '<' and '>' stay.
    The result has the length of `text`, so an index found by a plain
    string search in it (which then only sees top-level characters) is an
    index into `text`."""
    out = []
    depth = 0
    for ch in text:
        if ch == "<":
            out.append("<" if depth == 0 else ".")
            depth += 1
        elif ch == ">" and depth > 0:
            depth -= 1
            out.append(">" if depth == 0 else ".")
        else:
            out.append("." if depth > 0 else ch)
    return "".join(out)


def short_kernel_name(name: str) -> str:
    """`void fa::(anonymous namespace)::prefill_kernel<true, false>(...)` ->
    `prefill_kernel<true, false>`: the kernel's own name with its template
    arguments (they tell the instantiations apart). The parameter list, the
    return type and the qualifiers in front of the name are cut at their
    top-level '(', ' ' and '::' (those inside template arguments stay).
    Mangled names are demangled first."""
    text = demangle(name.strip()).replace("(anonymous namespace)::", "")
    top = _mask_templates(text)
    paren = top.find("(")
    if paren >= 0:
        text, top = text[:paren], top[:paren]
    text = text.rstrip()
    top = top[:len(text)]
    qualifier = top.rfind("::")
    cut = max(top.rfind(" ") + 1, qualifier + 2 if qualifier >= 0 else 0)
    return text[cut:].strip() or "kernel"


def read_kernel_stats(path: str) -> dict:
    """{short kernel name: {calls, avg_us, min_us, max_us, pct}} from
    run_kernel_stats.csv (instantiations that shorten to one name add up)."""
    out: dict = {}
    with open(path, newline="", encoding="utf-8") as handle:
        for row in csv.DictReader(handle):
            try:
                calls = int(row["Calls"])
                avg, lo, hi = (float(row[k]) / 1e3 for k in ("AverageNs", "MinNs", "MaxNs"))
                pct = float(row["Percentage"])
            except (KeyError, ValueError):
                continue
            key = short_kernel_name(row["Name"])
            if key in out:  # merge: weighted mean
                prev = out[key]
                total = prev["calls"] + calls
                prev["avg_us"] = (prev["avg_us"] * prev["calls"] + avg * calls) / total
                prev["min_us"] = min(prev["min_us"], lo)
                prev["max_us"] = max(prev["max_us"], hi)
                prev["pct"] += pct
                prev["calls"] = total
            else:
                out[key] = {"calls": calls, "avg_us": avg, "min_us": lo, "max_us": hi,
                            "pct": pct}
    if not out:
        raise SystemExit(f"{path}: no kernel rows")
    return out


def read_counters(path: str) -> dict:
    """{short kernel name: {counter: mean over its dispatches}} from
    run_counter_collection.csv (one row per dispatch and counter)."""
    acc: dict = {}
    with open(path, newline="", encoding="utf-8") as handle:
        reader = csv.DictReader(handle)
        if reader.fieldnames is None or "Counter_Name" not in reader.fieldnames:
            raise SystemExit(f"{path}: no Counter_Name column")
        for row in reader:
            try:
                value = float(row["Counter_Value"])
            except (KeyError, ValueError):
                continue
            key = short_kernel_name(row["Kernel_Name"])
            acc.setdefault(key, {}).setdefault(row["Counter_Name"], []).append(value)
    return {k: {c: statistics.fmean(v) for c, v in cs.items()} for k, cs in acc.items()}


def _counters_if(path: str) -> dict:
    return read_counters(path) if os.path.exists(path) else {}


def calibration(root: str) -> tuple[float, float]:
    """(fetch factor, write factor): bytes per counted KiB for FETCH_SIZE and
    WRITE_SIZE, from the copy_1g workload; (1024, 1024) when it is absent."""
    fetch = _counters_if(os.path.join(root, "copy_1g", "fetch", "run_counter_collection.csv"))
    write = _counters_if(os.path.join(root, "copy_1g", "write", "run_counter_collection.csv"))

    def factor(table, counter):
        for name, counters in table.items():
            if "copy" in name.lower() and counters.get(counter, 0) > 0:
                return COPY_BYTES / counters[counter]
        return 1024.0

    return factor(fetch, "FETCH_SIZE"), factor(write, "WRITE_SIZE")


def analyse(root: str) -> dict:
    ff, wf = calibration(root)
    report = {"fetch_bytes_per_kib": ff, "write_bytes_per_kib": wf, "workloads": {}}
    for name, (desc, main, unit, work) in WORKLOADS.items():
        wdir = os.path.join(root, name)
        stats_path = os.path.join(wdir, "trace", "run_kernel_stats.csv")
        if not os.path.exists(stats_path):
            continue
        stats = read_kernel_stats(stats_path)
        fetch = _counters_if(os.path.join(wdir, "fetch", "run_counter_collection.csv"))
        write = _counters_if(os.path.join(wdir, "write", "run_counter_collection.csv"))
        sq = _counters_if(os.path.join(wdir, "sq", "run_counter_collection.csv"))
        kernels = {}
        for kname, st in stats.items():
            row = dict(st)
            if "FETCH_SIZE" in fetch.get(kname, {}):
                row["read_bytes"] = fetch[kname]["FETCH_SIZE"] * ff
            if "WRITE_SIZE" in write.get(kname, {}):
                row["write_bytes"] = write[kname]["WRITE_SIZE"] * wf
            for counter, key in (("MfmaUtil", "mfma_util_pct"), ("MfmaFlopsF16", "mfma_flops"),
                                 ("LdsBankConflict", "lds_conflicts_per_access"),
                                 ("OccupancyPercent", "occupancy_pct")):
                if counter in sq.get(kname, {}):
                    row[key] = sq[kname][counter]
            kernels[kname] = row
        entry = {"description": desc, "unit": unit, "work_per_call": work, "kernels": kernels}
        mains = [k for k in kernels if k.startswith(main) or main in k]
        if mains:
            k = max(mains, key=lambda n: kernels[n]["calls"] * kernels[n]["avg_us"])
            rate = work / (kernels[k]["avg_us"] * 1e-6)
            peak = MFMA_FP16_PEAK_FLOPS if unit == "flop" else HBM_PEAK_BYTES
            entry["main"] = {"kernel": k, "rate": rate, "peak": peak, "frac": rate / peak,
                             "traffic_bytes": kernels[k].get("read_bytes", 0.0) +
                             kernels[k].get("write_bytes", 0.0)}
        report["workloads"][name] = entry
    report["bench"] = bench_runs(root)
    occ = os.path.join(root, "occupancy.json")
    if os.path.exists(occ):
        with open(occ, encoding="utf-8") as handle:
            report["occupancy"] = json.load(handle)
    return report


def bench_runs(root: str) -> dict:
    """bench.py's contract runs traced by the harness (bench_prefill,
    bench_decode): the trace average of the roofline kernel and bench.py's own
    live HIP-event figure for it, from the JSON line bench.py printed."""
    out = {}
    for part, section in (("prefill", None), ("decode", "decode")):
        wdir = os.path.join(root, f"bench_{part}")
        stats_path = os.path.join(wdir, "trace", "run_kernel_stats.csv")
        log_path = os.path.join(wdir, "trace.log")
        if not (os.path.exists(stats_path) and os.path.exists(log_path)):
            continue
        result = None
        with open(log_path, encoding="utf-8", errors="replace") as handle:
            for line in handle:
                if line.startswith("{"):
                    try:
                        result = json.loads(line)
                    except ValueError:
                        pass
        if result is None:
            continue
        roof = (result.get(section) or {}).get("roofline") if section else result.get("roofline")
        if not roof:
            continue
        stats = read_kernel_stats(stats_path)
        names = [k for k in stats if k.startswith(roof["kernel"].split("<")[0])]
        if not names:
            continue
        k = max(names, key=lambda n: stats[n]["calls"])
        out[part] = {"kernel": k, "trace_avg_us": stats[k]["avg_us"],
                     "trace_calls": stats[k]["calls"],
                     "bench_event_us": roof["kernel_ms"] * 1e3, "achieved": roof["achieved"],
                     "unit": roof["unit"]}
    return out


def _short(name, width=60):
    return name if len(name) <= width else name[:width - 1] + "…"


def _fmt_bytes(x):
    return "—" if x is None else f"{x / 1e6:,.2f} MB"


def _header(command):
    lines = []
    if command:
        lines += ["Made by (from the repository root, on the GPU box):", "", "```",
                  "cd /tmp && export TMPDIR=/tmp   # then back to the repository root",
                  command, "```", ""]
    return lines


def _base(kernel: str) -> str:
    return "".join(ch if ch.isalnum() or ch == "_" else "_" for ch in kernel.split("<")[0]).strip("_")


def render_workload(report: dict, name: str, command: str = "") -> str:
    """One workload's section: its main kernel's achieved rate and HBM
    traffic, then every kernel of the run."""
    w = report["workloads"][name]
    lines = [f"# rocprofv3: {name} ({w['description']})", "", "MI355X (gfx950), ROCm rocprofv3.", ""]
    lines += _header(command)
    lines += [f"HBM byte counters: FETCH_SIZE x {report['fetch_bytes_per_kib']:.1f} B/KiB, "
              f"WRITE_SIZE x {report['write_bytes_per_kib']:.1f} B/KiB (the factors that make "
              "the copy_1g workload's 1 GiB copy read and write exactly 1 GiB; 1024 means "
              "uncalibrated).", ""]
    if "main" in w:
        m = w["main"]
        unit = "TFLOP/s" if w["unit"] == "flop" else "GB/s"
        scale = 1e12 if w["unit"] == "flop" else 1e9
        lines += [f"Main kernel `{m['kernel']}`: {w['work_per_call']:,.0f} algorithmic "
                  f"{'FLOP' if w['unit'] == 'flop' else 'bytes'} per launch at the trace average "
                  f"= {m['rate'] / scale:,.1f} {unit} = **{100 * m['frac']:.1f} %** of the MI355X "
                  f"peak ({m['peak'] / scale:,.0f} {unit}).", ""]
    lines += ["| kernel | calls | avg µs | min µs | max µs | HBM read | HBM write | "
              "MFMA util | fp16 MFMA GFLOP | LDS conflicts/access | occupancy |",
              "| :-- | ---: | ---: | ---: | ---: | ---: | ---: | ---: | ---: | ---: | ---: |"]
    for kname, r in sorted(w["kernels"].items(), key=lambda kv: -kv[1]["pct"]):
        def opt(key, fmt, scale=1.0):
            return fmt.format(r[key] * scale) if key in r else "—"
        lines.append(
            f"| `{_short(kname)}` | {r['calls']} | {r['avg_us']:.2f} | {r['min_us']:.2f} | "
            f"{r['max_us']:.2f} | {_fmt_bytes(r.get('read_bytes'))} | "
            f"{_fmt_bytes(r.get('write_bytes'))} | {opt('mfma_util_pct', '{:.1f} %')} | "
            f"{opt('mfma_flops', '{:,.2f}', 1e-9)} | "
            f"{opt('lds_conflicts_per_access', '{:.3f}')} | {opt('occupancy_pct', '{:.1f} %')} |")
    lines.append("")
    if "main" in w and w["main"]["traffic_bytes"] > 0:
        lines += ["HBM bytes per launch of the main kernel (read + write), read by bench.py:", "",
                  f"traffic_bytes_per_launch: {w['main']['traffic_bytes']:.0f}", ""]
    return "\n".join(lines).rstrip() + "\n"


def render_bench(report: dict, command: str = "") -> str:
    lines = ["# rocprofv3: bench.py's contract runs under the kernel trace", "",
             "The roofline kernel of each run: rocprofv3's average duration over every traced "
             "launch (clock warm-up, warm-up and timed steps) beside bench.py's live HIP-event "
             "figure over its timed steps, from the same run.", ""]
    lines += _header(command)
    lines += ["| run | kernel | traced launches | trace avg µs | bench events µs | bench achieved |",
              "| :-- | :-- | ---: | ---: | ---: | ---: |"]
    for part, b in report.get("bench", {}).items():
        lines.append(f"| bench.py --only {part} --no-cpu --no-configs --steps 50 --warmup 5 | "
                     f"`{b['kernel']}` | {b['trace_calls']} | {b['trace_avg_us']:.2f} | "
                     f"{b['bench_event_us']:.2f} | {b['achieved']:,.1f} {b['unit']} |")
    return "\n".join(lines).rstrip() + "\n"


def render_occupancy(report: dict, command: str = "") -> str:
    lines = ["# Theoretical occupancy of every kernel (occupancy_report())", ""]
    lines += _header(command)
    lines += ["| kernel | threads/block | VGPRs/thread | LDS/block | blocks/CU | occupancy |",
              "| :-- | ---: | ---: | ---: | ---: | ---: |"]
    for row in report.get("occupancy", []):
        lines.append(f"| `{row['kernel']}` | {row['threads_per_block']} | "
                     f"{row['registers_per_thread']} | {row['shared_bytes_per_block']:,} B | "
                     f"{row['max_active_blocks_per_sm']} | "
                     f"{100 * row['theoretical_occupancy']:.1f} % |")
    return "\n".join(lines).rstrip() + "\n"


def render(report: dict, command: str = "") -> str:
    """Everything in one document."""
    parts = [render_workload(report, n, command) for n in report["workloads"]]
    if report.get("bench"):
        parts.append(render_bench(report, command))
    if report.get("occupancy"):
        parts.append(render_occupancy(report, command))
    return "\n".join(parts)


def write_split(report: dict, out_dir: str, command: str = "") -> list:
    """One file per workload, named `<workload>__<main kernel>.md`, plus
    bench_traces.md and occupancy.md; returns the paths written."""
    os.makedirs(out_dir, exist_ok=True)
    paths = []
    for name, w in report["workloads"].items():
        kernel = _base(w["main"]["kernel"]) if "main" in w else "kernels"
        path = os.path.join(out_dir, f"{name}__{kernel}.md")
        with open(path, "w", encoding="utf-8") as handle:
            handle.write(render_workload(report, name, command))
        paths.append(path)
    for fname, fn, key in (("bench_traces.md", render_bench, "bench"),
                           ("occupancy.md", render_occupancy, "occupancy")):
        if report.get(key):
            path = os.path.join(out_dir, fname)
            with open(path, "w", encoding="utf-8") as handle:
                handle.write(fn(report, command))
            paths.append(path)
    return paths


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--root", required=True)
    ap.add_argument("--out", required=True)
    ap.add_argument("--json")
    ap.add_argument("--split-dir", help="also write one file per workload into this directory")
    ap.add_argument("--command", default="")
    args = ap.parse_args(argv)
    report = analyse(args.root)
    if not report["workloads"]:
        raise SystemExit(f"{args.root}: no workload traces found")
    with open(args.out, "w", encoding="utf-8") as handle:
        handle.write(render(report, args.command))
    if args.split_dir:
        for path in write_split(report, args.split_dir, args.command):
            print(f"wrote {path}")
    if args.json:
        with open(args.json, "w", encoding="utf-8") as handle:
            json.dump(report, handle, indent=1)
    print(f"wrote {args.out}")


if __name__ == "__main__":
    main()
