"""rocprofv3 counter passes over bench.py's workloads, summarised for profiles/.

Run on the GPU box from the repository root (this process starts rocprofv3 as a child per pass
and never touches the GPU itself):

    python3 groupgemm-cktile-optimized_amd/pmc.py [--workloads all|W1,W2] [--op fwd]
        [--raw gpurun_out/pmc] [--profiles profiles] [--commit SHA]

Per workload, four runs of `bench.py --workload W --op OP --steps 3 --warmup 1 --no-cpu-baseline
--power-seconds 0 --baselines ""`, each under `timeout -s KILL`:
  fetch  rocprofv3 --pmc FETCH_SIZE
  write  rocprofv3 --pmc WRITE_SIZE
  sq     rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_VALU_MFMA_BUSY_CYCLES
                         SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE GRBM_COUNT
  trace  rocprofv3 --kernel-trace over the driver's protocol (--warmup 5 --steps 20): every launch's
         duration without counters, the timed 20 averaged for the clock
and once per call two passes over a 1 GiB device copy (bench.py --calibrate-copy), which give the
bytes one KiB of FETCH_SIZE / WRITE_SIZE stands for (the reference's counters, scripts/pmc.sh:4,
16-17, are the SQ ones).

Per workload it writes profiles/hbm_traffic_<workload>[_<op>].json: the per-dispatch counters of
the grouped GEMM kernel (mean over the dispatches after the first), fetch and write bytes per
launch scaled by the copy calibration, their ratio to the algorithmic bytes, LDS bank conflicts,
MFMA busy, issued vs useful MFMA cycles, cycles per launch (GRBM_GUI_ACTIVE per XCD), the share
of the MFMA peak per clock and the clock, with the kernel instance, the plan and the hash of the kernel sources
(kernel_source_sha) they were measured on; bench.py reports `traffic` only for a build with the
same hash and plan. Prints one line per pass; stops at the first pass that fails (exit 1).
FETCH_SIZE counts the L2's read requests to the data fabric, Infinity-Cache hits included, so
the fetch bytes are an upper bound on DRAM reads.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import subprocess
import sys
import time

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
sys.path.insert(0, ROOT)

PASSES = {
    "fetch": ["FETCH_SIZE"],
    "write": ["WRITE_SIZE"],
    "sq": ["SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES",
           "GRBM_GUI_ACTIVE", "GRBM_COUNT"],
}
CALIBRATION_BYTES = 1 << 30
XCDS = 8


def log(msg: str) -> None:
    print(f"[pmc {time.strftime('%H:%M:%S')}] {msg}", flush=True)


def run_pass(tag: str, prof_args, bench_args, raw_dir: str, limit_s: int):
    """One rocprofv3 run; returns (csv files it wrote, bench stderr). Raises on failure."""
    out_dir = os.path.join(raw_dir, tag)
    os.makedirs(out_dir, exist_ok=True)
    cmd = (["timeout", "-s", "KILL", str(limit_s), "rocprofv3"] + prof_args +
           ["-d", out_dir, "-o", tag, "--output-format", "csv", "--", sys.executable, os.path.join(ROOT, "bench.py")]
           + bench_args)
    p = subprocess.run(cmd, cwd="/tmp", capture_output=True, text=True)
    with open(os.path.join(out_dir, "run.log"), "w") as f:
        f.write(" ".join(cmd) + "\n---- stdout ----\n" + p.stdout + "\n---- stderr ----\n" + p.stderr)
    files = glob.glob(os.path.join(out_dir, "**", "*.csv"), recursive=True)
    # rocprofv3 may end with a segmentation fault after the program finished and the files are
    # complete: accept that only when the program printed its last line
    finished = '"metric"' in p.stdout or "calibrate_copy_bytes" in p.stdout
    if p.returncode != 0 and not (p.returncode in (139, -11) and finished and files):
        raise RuntimeError(f"{tag}: rocprofv3 exited {p.returncode}; see {out_dir}/run.log")
    return files, p.stderr


def dispatches(files, match):
    """{dispatch id: {"name": kernel, "counters": {name: value}, "ns": duration}} of kernels whose
    name satisfies match(), from counter-collection or kernel-trace CSVs."""
    out = {}
    for path in files:
        base = os.path.basename(path)
        if not (base.endswith("_counter_collection.csv") or base.endswith("_kernel_trace.csv")):
            continue
        with open(path) as f:
            for row in csv.DictReader(f):
                name = row.get("Kernel_Name", "")
                if not match(name):
                    continue
                d = out.setdefault(int(row["Dispatch_Id"]), {"name": name, "counters": {}, "ns": None})
                if "Counter_Name" in row:
                    d["counters"][row["Counter_Name"]] = float(row["Counter_Value"])
                else:
                    d["ns"] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
    return out


def mean_after_first(ds, key):
    vals = [d["counters"][key] for _, d in sorted(ds.items()) if key in d["counters"]]
    if len(vals) > 1:
        vals = vals[1:]
    return sum(vals) / len(vals) if vals else None


# The GEMM launch of a plan: the persistent kernel, or the small-tile kernel (gg_small.hip).
GEMM_KERNEL = re.compile(r"(?:grouped_gemm_kernel|small_gemm_kernel)<[^>]*>")


def is_gemm(name: str) -> bool:
    return "grouped_gemm_kernel" in name or "small_gemm_kernel" in name


def instance(name: str) -> str:
    m = GEMM_KERNEL.search(name)
    return m.group(0) if m else name


def calibrate(raw: str, limit: int):
    """Bytes per KiB of FETCH_SIZE and of WRITE_SIZE, from a device copy of CALIBRATION_BYTES."""
    res = {}
    for tag, counter in (("calib_fetch", "FETCH_SIZE"), ("calib_write", "WRITE_SIZE")):
        files, _ = run_pass(tag, ["--pmc", counter], ["--calibrate-copy", str(CALIBRATION_BYTES)], raw, limit)
        ds = dispatches(files, lambda n: "copy" in n.lower())
        kib = mean_after_first(ds, counter) if ds else None
        res[counter] = kib
        log(f"calibration {counter}: {kib} KiB per {CALIBRATION_BYTES >> 10} KiB copied "
            f"({len(ds)} copy dispatches)")
    fetch = (CALIBRATION_BYTES / res["FETCH_SIZE"]) if res.get("FETCH_SIZE") else None
    write = (CALIBRATION_BYTES / res["WRITE_SIZE"]) if res.get("WRITE_SIZE") else None
    return {"copy_bytes": CALIBRATION_BYTES, "fetch_size_kib": res.get("FETCH_SIZE"),
            "write_size_kib": res.get("WRITE_SIZE"), "bytes_per_fetch_kib": fetch, "bytes_per_write_kib": write}


def profile_workload(w: str, op: str, raw: str, limit: int, cal, commit: str, sha: str, workloads):
    bench_args = ["--workload", w, "--op", op, "--steps", "3", "--warmup", "1", "--no-cpu-baseline",
                  "--power-seconds", "0", "--baselines", ""]
    tag0 = w if op == "fwd" else f"{w}_{op}"
    counters, plan, name, trace_ns = {}, None, None, None
    for p, names in PASSES.items():
        files, err = run_pass(f"{tag0}_{p}", ["--pmc"] + names + ["--kernel-trace"], bench_args, raw, limit)
        ds = dispatches(files, is_gemm)
        if not ds:
            raise RuntimeError(f"{tag0}_{p}: no GEMM kernel dispatch in the counters")
        name = next(iter(ds.values()))["name"]
        for c in names:
            counters[c] = mean_after_first(ds, c)
        m = re.search(r"\[bench\] \S+ \S+: (.*)", err)
        plan = m.group(1).strip() if m else plan
        log(f"{tag0} {p}: " + ", ".join(f"{c}={counters[c]:.6g}" for c in names if counters[c] is not None))
    trace_args = ["--workload", w, "--op", op, "--steps", "20", "--warmup", "5", "--no-cpu-baseline",
                  "--power-seconds", "0", "--baselines", ""]
    files, _ = run_pass(f"{tag0}_trace", ["--kernel-trace"], trace_args, raw, limit)
    ds = dispatches(files, is_gemm)
    ns = [d["ns"] for _, d in sorted(ds.items()) if d["ns"]]
    timed = ns[-20:] if len(ns) >= 25 else ns[1:] or ns
    trace_ns = sum(timed) / len(timed) if timed else None
    log(f"{tag0} trace: {len(ns)} dispatches, {trace_ns} ns over the last {len(timed)}")

    dtype, b, m, n, k = workloads[w]
    fp8 = "fp8" in op
    es = 1 if fp8 else 2
    algo = es * (b * m * k + b * n * k) + 2 * b * m * n
    flops = 2.0 * b * m * n * k
    flop_per_simd_clk = 2048.0 if fp8 else 1024.0  # dense MFMA peak per SIMD per clock
    cycles = counters["GRBM_GUI_ACTIVE"] / XCDS if counters.get("GRBM_GUI_ACTIVE") else None
    mfma = counters.get("SQ_VALU_MFMA_BUSY_CYCLES")
    fetch = counters["FETCH_SIZE"] * cal["bytes_per_fetch_kib"] if counters.get("FETCH_SIZE") and cal.get(
        "bytes_per_fetch_kib") else None
    write = counters["WRITE_SIZE"] * cal["bytes_per_write_kib"] if counters.get("WRITE_SIZE") and cal.get(
        "bytes_per_write_kib") else None
    busy = counters.get("SQ_BUSY_CU_CYCLES")
    cus = 256
    res = {
        "workload": w, "op": op, "kernel": instance(name), "plan": plan, "kernel_source_sha": sha, "commit": commit,
        "counters_per_dispatch": counters,
        "calibration": cal,
        "fetch_bytes_per_launch": round(fetch) if fetch else None,
        "write_bytes_per_launch": round(write) if write else None,
        "hbm_bytes_per_launch": round(fetch + write) if fetch and write else None,
        "algorithmic_bytes_per_launch": algo,
        "traffic_over_algorithmic": round((fetch + write) / algo, 3) if fetch and write else None,
        "fetch_over_input_bytes": round(fetch / (es * (b * m * k + b * n * k)), 3) if fetch else None,
        "lds_bank_conflict_pct": round(100.0 * counters["SQ_LDS_BANK_CONFLICT"] / counters["SQ_LDS_IDX_ACTIVE"], 3)
        if counters.get("SQ_LDS_IDX_ACTIVE") else None,
        "mfma_busy_pct": round(100.0 * counters["SQ_VALU_MFMA_BUSY_CYCLES"] / (4.0 * busy), 2) if busy else None,
        "mfma_cycles_issued": round(mfma) if mfma else None,
        "mfma_cycles_useful": round(flops / flop_per_simd_clk),
        "mfma_useful_over_issued": round(flops / flop_per_simd_clk / mfma, 4) if mfma else None,
        "cycles_per_launch": round(cycles) if cycles else None,
        "mfma_peak_per_clock_pct": round(100.0 * flops / (cycles * cus * 4 * flop_per_simd_clk), 2)
        if cycles else None,
        "launch_ns_unprofiled": ns,
        "kernel_ns_unprofiled": round(trace_ns) if trace_ns else None,
        "tflops_unprofiled": round(flops / trace_ns / 1e3, 1) if trace_ns else None,
        "clock_ghz": round(cycles / trace_ns, 3) if trace_ns and cycles else None,
        "note": "FETCH_SIZE counts the L2's read requests to the data fabric (Infinity-Cache hits included), "
                "WRITE_SIZE its writes; both scaled by a 1 GiB device copy. cycles_per_launch is GRBM_GUI_ACTIVE "
                "per XCD; launch_ns_unprofiled are the 25 launches of the driver's protocol (5 warmup + 20 timed) "
                "without counters, kernel_ns_unprofiled their timed 20's mean, and the clock is the cycles over "
                "that mean. mfma_cycles_useful = flops / (dense MFMA flops per SIMD per clock): the rest of the "
                "issued MFMA cycles compute padding.",
    }
    return res


def write_markdown(path: str, results, cal, cmdline: str):
    lines = [
        "# rocprofv3 counters per BASELINE config (FETCH_SIZE, WRITE_SIZE, LDS bank conflicts, MFMA busy, clock)",
        "",
        "Made on the MI355X box from the repository root by:",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp",
        f"python3 $R/{cmdline}",
        "```",
        "",
        "(`groupgemm-cktile-optimized_amd/pmc.py` runs rocprofv3 once per counter pass per workload over "
        "`bench.py --workload W --steps 3 --warmup 1 --no-cpu-baseline --power-seconds 0 --baselines \"\"`; "
        "counters are per dispatch of the grouped GEMM, the mean over the dispatches after the first.)",
        "",
        f"Copy calibration (1 GiB device copy): FETCH_SIZE {cal.get('fetch_size_kib')} KiB, WRITE_SIZE "
        f"{cal.get('write_size_kib')} KiB -> {cal.get('bytes_per_fetch_kib')} and {cal.get('bytes_per_write_kib')} "
        "bytes per KiB counted.",
        "",
        "| Workload | Kernel instance | fetch GB | write GB | (fetch+write) / algorithmic | fetch / (x+w) | "
        "LDS bank conflicts | MFMA busy | useful / issued MFMA | Mcycles | % MFMA peak per clock | "
        "kernel ms (timed 20) | TFLOPS | clock GHz |",
        "|---|---|---|---|---|---|---|---|---|---|---|---|---|---|",
    ]
    for r in results:
        f = r["fetch_bytes_per_launch"]
        wr = r["write_bytes_per_launch"]
        lines.append(
            f"| {r['workload']}{'' if r['op'] == 'fwd' else ' ' + r['op']} | `{r['kernel']}` | "
            f"{f / 1e9:.3f} | {wr / 1e9:.3f} | {r['traffic_over_algorithmic']} | {r['fetch_over_input_bytes']} | "
            f"{r['lds_bank_conflict_pct']} % | {r['mfma_busy_pct']} % | {r['mfma_useful_over_issued']} | "
            f"{(r['cycles_per_launch'] or 0) / 1e6:.3f} | {r['mfma_peak_per_clock_pct']} % | "
            f"{(r['kernel_ns_unprofiled'] or 0) / 1e6:.4f} | {r['tflops_unprofiled']} | {r['clock_ghz']} |"
            if f and wr else
            f"| {r['workload']} | `{r['kernel']}` | - | - | - | - | {r['lds_bank_conflict_pct']} % | "
            f"{r['mfma_busy_pct']} % | - | - | - | - | - | - |")
    lines += ["", f"Kernel sources: `{results[0]['kernel_source_sha'] if results else ''}` "
                  f"(commit {results[0]['commit'] if results else ''}).", ""]
    with open(path, "w") as fh:
        fh.write("\n".join(lines))


def main():
    import bench  # the workload table; importing it does not touch the GPU

    import __graft_entry__ as entry

    ap = argparse.ArgumentParser()
    ap.add_argument("--workloads", default="all")
    ap.add_argument("--op", default="fwd", choices=bench.OPS)
    ap.add_argument("--raw", default=os.path.join(ROOT, "gpurun_out", "pmc"))
    ap.add_argument("--profiles", default=os.path.join(ROOT, "gpurun_out", "profiles"))
    ap.add_argument("--commit", default="unknown")
    ap.add_argument("--limit", type=int, default=90, help="seconds per rocprofv3 run")
    args = ap.parse_args()
    # rocprofv3 runs with /tmp as its working directory: every path it is given is absolute
    args.raw = os.path.abspath(args.raw)
    args.profiles = os.path.abspath(args.profiles)
    names = sorted(bench.WORKLOADS) if args.workloads == "all" else args.workloads.split(",")
    sha = entry.load_package().kernel_source_sha()
    os.makedirs(args.profiles, exist_ok=True)
    log(f"kernel sources {sha}, workloads {names}")
    try:
        cal = calibrate(args.raw, args.limit)
        results = []
        for w in names:
            r = profile_workload(w, args.op, args.raw, args.limit, cal, args.commit, sha, bench.WORKLOADS)
            suffix = "" if args.op == "fwd" else f"_{args.op}"
            with open(os.path.join(args.profiles, f"hbm_traffic_{w}{suffix}.json"), "w") as f:
                json.dump(r, f, indent=2)
            log(f"{w}: traffic/algorithmic {r['traffic_over_algorithmic']}, MFMA busy {r['mfma_busy_pct']} %, "
                f"LDS conflicts {r['lds_bank_conflict_pct']} %, clock {r['clock_ghz']} GHz")
            results.append(r)
    except RuntimeError as e:
        log(f"stopped: {e}")
        sys.exit(1)
    cmdline = "groupgemm-cktile-optimized_amd/pmc.py " + " ".join(sys.argv[1:])
    write_markdown(os.path.join(args.profiles, f"pmc_counters_{args.op}_all_configs.md"), results, cal, cmdline)
    log("done")


if __name__ == "__main__":
    main()
