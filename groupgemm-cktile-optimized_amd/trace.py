"""rocprofv3 kernel traces of bench.py's workloads under the driver's protocol, summarised for profiles/.

Run on the GPU box from the repository root (this process starts rocprofv3 as a child per
workload and never touches the GPU itself):

    python3 groupgemm-cktile-optimized_amd/trace.py [--workloads all|W1,W2] [--op fwd]
        [--raw gpurun_out/trace] [--profiles profiles]

Per workload one run of

    rocprofv3 --kernel-trace --stats -- python3 bench.py --workload W --op OP --steps 20 --warmup 5
        --no-cpu-baseline --power-seconds 0 --baselines ""

under `timeout -s KILL`, and a summary profiles/grouped_gemm_kernel_<workload>[_<op>].md: the
command, the plan, rocprofv3's per-kernel statistics, the duration of each of the 25 grouped-GEMM
launches (5 warmup + 20 timed: the clock falls and recovers over them), the timed 20's mean as
TFLOP/s next to bench.py's own HIP-event figure from the same process, and the compiler's
resource report of the kernel instance (lib/resource_usage.txt). Stops at the first run that
fails (exit 1).
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


def log(msg: str) -> None:
    print(f"[trace {time.strftime('%H:%M:%S')}] {msg}", flush=True)


# The GEMM launch of a plan: the persistent kernel, or the small-tile kernel (gg_small.hip).
GEMM_KERNEL = re.compile(r"(grouped_gemm_kernel|small_gemm_kernel)<([^>]*)>")


def mangled_instance(name: str) -> str:
    """Itanium mangling of the kernel instance in a demangled name, for the resource report."""
    m = GEMM_KERNEL.search(name)
    if not m:
        return ""
    parts = []
    for a in (x.strip() for x in m.group(2).split(",")):
        parts.append(("Lb1E" if a == "true" else "Lb0E") if a in ("true", "false") else f"Li{a}E")
    return m.group(1) + "I" + "".join(parts) + "E"


def resource_line(name: str) -> str:
    path = os.path.join(PKG_DIR, "lib", "resource_usage.txt")
    key = mangled_instance(name)
    if not key or not os.path.exists(path):
        return "(no resource report)"
    text = open(path).read().split("\n")
    vals = {}
    for i, line in enumerate(text):
        if "Function Name:" in line and key in line:
            for follow in text[i + 1:i + 12]:
                m = re.search(r"remark: .*?:\s+(TotalSGPRs|VGPRs|AGPRs|SGPRs Spill|VGPRs Spill|ScratchSize \[bytes/lane\]"
                              r"|Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]): (\d+)", follow)
                if m:
                    vals[m.group(1)] = m.group(2)
            break
    if not vals:
        return "(instance not in the resource report)"
    return ", ".join(f"{k} {v}" for k, v in vals.items())


def kernel_label(name: str) -> str:
    """A kernel's demangled name without its namespace qualifiers and argument list."""
    name = name.replace("(anonymous namespace)::", "")
    return re.sub(r"\([^()]*\)$", "", name).replace("void ", "", 1)


def trace_workload(w: str, op: str, raw: str, profiles: str, limit: int, workloads, rerun: bool = True) -> dict:
    tag = w if op == "fwd" else f"{w}_{op}"
    out_dir = os.path.join(raw, tag)
    os.makedirs(out_dir, exist_ok=True)
    bench_args = ["--workload", w, "--op", op, "--steps", "20", "--warmup", "5", "--no-cpu-baseline",
                  "--power-seconds", "0", "--baselines", ""]
    cmd = (["timeout", "-s", "KILL", str(limit), "rocprofv3", "--kernel-trace", "--stats", "-d", out_dir, "-o", tag,
            "--output-format", "csv", "--", sys.executable, os.path.join(ROOT, "bench.py")] + bench_args)
    if rerun:
        p = subprocess.run(cmd, cwd="/tmp", capture_output=True, text=True)
        with open(os.path.join(out_dir, "run.log"), "w") as f:
            f.write(" ".join(cmd) + "\n---- stdout ----\n" + p.stdout + "\n---- stderr ----\n" + p.stderr)
    else:  # summarise an earlier run from its log and CSV files
        text = open(os.path.join(out_dir, "run.log")).read()
        out, err = text.split("\n---- stdout ----\n", 1)[1].split("\n---- stderr ----\n", 1)
        p = subprocess.CompletedProcess(cmd, 0, out, err)
    line = next((x for x in p.stdout.splitlines() if x.startswith("{") and '"metric"' in x), None)
    files = glob.glob(os.path.join(out_dir, "**", "*.csv"), recursive=True)
    # rocprofv3 may end with a segmentation fault after the program finished and wrote its line
    if p.returncode != 0 and not (p.returncode in (139, -11) and line and files):
        raise RuntimeError(f"{tag}: rocprofv3 exited {p.returncode}; see {out_dir}/run.log")
    bench = json.loads(line) if line else {}
    stats, launches, name = [], [], ""
    for path in files:
        base = os.path.basename(path)
        if base.endswith("_kernel_stats.csv"):
            with open(path) as f:
                stats = list(csv.DictReader(f))
        elif base.endswith("_kernel_trace.csv"):
            with open(path) as f:
                rows = [r for r in csv.DictReader(f) if GEMM_KERNEL.search(r.get("Kernel_Name", ""))]
            rows.sort(key=lambda r: int(r["Start_Timestamp"]))
            launches = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows]
            name = rows[0]["Kernel_Name"] if rows else ""
    if len(launches) < 25:
        raise RuntimeError(f"{tag}: {len(launches)} grouped-GEMM launches in the trace, expected 25")
    dtype, b, m, n, k = workloads[w]
    flops = 2.0 * b * m * n * k
    timed = launches[-20:]
    mean_ns = sum(timed) / len(timed)
    plan = re.search(r"\[bench\] \S+ \S+: (.*)", p.stderr)
    short = GEMM_KERNEL.search(name)
    short = short.group(0) if short else name
    lines = [
        f"# rocprofv3 kernel trace: `{short}`, {tag}",
        "",
        "Made on the MI355X box from the repository root `$R` by "
        f"`python3 groupgemm-cktile-optimized_amd/trace.py --workloads {w}{'' if op == 'fwd' else ' --op ' + op}`, "
        "which runs:",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp",
        f"rocprofv3 --kernel-trace --stats -d $R/gpurun_out/trace/{tag} -o {tag} --output-format csv -- \\",
        f"    python3 $R/bench.py {' '.join(a if a else chr(34) * 2 for a in bench_args)}",
        "```",
        "",
        f"Plan: {plan.group(1).strip() if plan else '(not printed)'}",
        "",
        "Kernel statistics (`*_kernel_stats.csv`):",
        "",
        "| Kernel | Calls | Average ns | Min ns | Max ns |",
        "|---|---|---|---|---|",
    ]
    for r in stats:
        nm = kernel_label(r.get("Name", r.get("KernelName", "")))
        lines.append(f"| `{nm[:100]}` | {r.get('Calls')} | {float(r.get('AverageNs', 0)):,.0f} | "
                     f"{float(r.get('MinNs', 0)):,.0f} | {float(r.get('MaxNs', 0)):,.0f} |")
    lines += [
        "",
        "Grouped-GEMM launches in order (µs; 1-5 are bench.py's warmup, 6-25 its timed loop):",
        "",
        "```",
        " ".join(f"{x / 1e3:.1f}" for x in launches[:25]),
        "```",
        "",
        f"Timed 20 (launches 6-25): mean **{mean_ns:,.0f} ns** = {flops / mean_ns / 1e3:.1f} TFLOP/s "
        f"({100.0 * flops / mean_ns / 1e3 / (5000.0 if 'fp8' in op else 2500.0):.1f} % of the dense MFMA peak); "
        f"min {min(timed):,} ns, max {max(timed):,} ns.",
        f"bench.py's HIP-event figure in the same process: {bench.get('ms_per_step')} ms per step, "
        f"{bench.get('value')} TFLOP/s.",
        "",
        f"FLOPs per launch 2 * {b * m} * {n} * {k} = {flops:.4e}.",
        "",
        f"Compiler report of the instance (`lib/resource_usage.txt`): {resource_line(name)}.",
        "",
    ]
    path = os.path.join(profiles, f"grouped_gemm_kernel_{tag}.md")
    with open(path, "w") as f:
        f.write("\n".join(lines))
    return {"workload": tag, "mean_ns": mean_ns, "tflops": flops / mean_ns / 1e3, "bench": bench.get("value"),
            "launches_us": [round(x / 1e3, 1) for x in launches[:25]]}


def main():
    import bench

    ap = argparse.ArgumentParser()
    ap.add_argument("--workloads", default="all")
    ap.add_argument("--op", default="fwd", choices=bench.OPS)
    ap.add_argument("--raw", default=os.path.join(ROOT, "gpurun_out", "trace"))
    ap.add_argument("--profiles", default=os.path.join(ROOT, "profiles"))
    ap.add_argument("--limit", type=int, default=120, help="seconds per rocprofv3 run")
    ap.add_argument("--summarise-only", action="store_true",
                    help="write the summaries from the runs already under --raw (no rocprofv3)")
    ap.add_argument("--fill-resources", action="store_true",
                    help="only rewrite the compiler-report line of the existing summaries (where the build's "
                         "lib/resource_usage.txt is, which GPU runs need not carry)")
    args = ap.parse_args()
    if args.fill_resources:
        for path in glob.glob(os.path.join(os.path.abspath(args.profiles), "grouped_gemm_kernel_*.md")):
            text = open(path).read()
            m = re.search(r"^# rocprofv3 kernel trace: `([^`]*)`", text, re.M)
            if m:
                text = re.sub(r"^Compiler report of the instance .*$",
                              f"Compiler report of the instance (`lib/resource_usage.txt`): {resource_line(m.group(1))}.",
                              text, flags=re.M)
                open(path, "w").write(text)
        return
    args.raw = os.path.abspath(args.raw)  # rocprofv3 runs with /tmp as its working directory
    args.profiles = os.path.abspath(args.profiles)
    os.makedirs(args.profiles, exist_ok=True)
    names = sorted(bench.WORKLOADS) if args.workloads == "all" else args.workloads.split(",")
    for w in names:
        try:
            r = trace_workload(w, args.op, args.raw, args.profiles, args.limit, bench.WORKLOADS,
                               rerun=not args.summarise_only)
        except RuntimeError as e:
            log(f"stopped: {e}")
            sys.exit(1)
        log(f"{r['workload']}: timed mean {r['mean_ns']:,.0f} ns = {r['tflops']:.1f} TFLOP/s (bench {r['bench']}); "
            f"launches {r['launches_us']}")
    log("done")


if __name__ == "__main__":
    main()
