"""Benchmark of the MI355X grouped GEMM on BASELINE.json's headline config.

One "step" = one grouped GEMM launch (Backend::run) over the whole synthetic batch of the
MoE gate+up projection config: B=8 groups x M=4096 tokens, N=4096, K=7168, bf16, balanced
groups, x and w ~ N(0,1) from the seeded generator (x seed 1, w seed 2), inputs resident in
HBM before timing (the reference's protocol, bench/bench_main.cpp:436-501).

--op runs another pass of the same workload instead of the forward GEMM (default: forward, the
headline): dgrad (grad_x = grad_out @ w[g]), wgrad (grad_w[g] = grad_out[g]^T @ x[g]), the
fp8 forward (e4m3 / e5m2 inputs, unit tensor-wise scales, bf16 out), or the fp8 dgrad / wgrad
(e5m2 gradient, e4m3 w / x, unit scales, bf16 out). Same FLOPs, 2 sum(M) N K.

Prints ONE JSON line on stdout. Besides the driver's fields it carries:
  roofline     the kernel against the dense bf16 MFMA peak (2.5 PFLOP/s): achieved = FLOPs
               per launch / mean launch duration from HIP events on the launch stream;
               traffic = fetch + write bytes per launch (rocprofv3 FETCH_SIZE + WRITE_SIZE, scaled
               by a device copy) from profiles/hbm_traffic_<workload>[_<op>].json, but only when
               that file was measured on the kernel sources of this build (kernel_source_sha) and
               the same plan; else null. traffic_profile names the file, its commit, kernel
               instance and why it was or was not used. FETCH_SIZE counts the L2's reads from the
               data fabric, Infinity-Cache hits included, so it bounds the DRAM reads from above.
  baselines    the hipBLASLt comparison backends (default hipblaslt_loop, the Primus-Turbo
               per-group loop on 4 streams the reference compares against, and hipblaslt_seq, the
               same loop on one stream) and the MI355X kernel again, timed right after the timed
               region in one native process (bin/gg_bench, a child of this one) on the same config,
               warmup and steps, each checked on the sampled outputs (forward only); each with its
               TFLOPS, or its N/A reason or error.
  cpu_baseline the CPU oracle (OpenMP fp32, test infrastructure) timed on a bounded sample
               of the same workload on this host; a reported baseline only.
  timed_region_clock
               the effective shader clock of the timed region: the matching profile's GRBM cycles
               per launch over ms_per_step (null, with the reason, when no profile of this build
               and plan exists).
  clock_power  a separate sustained window of the same launches after the timed region
               (--power-seconds, default 1 s; the timed region itself runs without probe or
               sampling thread): its TFLOPS, its effective shader clock from the clock probe (one
               wave beside the GEMM reading s_memtime against s_memrealtime) with the dense peak
               scaled to that clock, and amdsmi's gfx clock and socket power, the two figures the
               reference records (scripts/power.py:1-9); amdsmi's clock is marked inconsistent
               when it is more than 5 % off the probe's.
Human-readable progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402

WORKLOADS = {
    # name: (dtype, B, M per group, N, K)
    "moe_gate_up_b8_m4096_n4096_k7168_bf16": (0, 8, 4096, 4096, 7168),
    "moe_down_b8_m4096_n7168_k2048_bf16": (0, 8, 4096, 7168, 2048),
    "dense_expert_b8_m4096_n14336_k4096_fp16": (1, 8, 4096, 14336, 4096),
    "dense_expert_b8_m4096_n14336_k4096_bf16": (0, 8, 4096, 14336, 4096),
    "tails_b32_m520_n2880_k2880_bf16": (0, 32, 520, 2880, 2880),
    "low_occupancy_b1_m2048_n7168_k2048_bf16": (0, 1, 2048, 7168, 2048),
    "plumbing_b4_m256_n512_k1024_bf16": (0, 4, 256, 512, 1024),
}
HEADLINE = "moe_gate_up_b8_m4096_n4096_k7168_bf16"
MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16/fp16
FP8_PEAK_TFLOPS = 5000.0  # MI355X dense fp8
OPS = ("fwd", "dgrad", "wgrad", "fp8_e4m3", "fp8_e5m2", "dgrad_fp8", "wgrad_fp8")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(oracle, x, w, group_m, dtype, n, k, target_s):
    """Time the CPU oracle on the workload's first R output rows (each row against its own
    group's w, all N columns, full K). R comes from a two-point linear model t(R) = a + b R
    (two short probes on group 0) so that the timed pass takes about target_s seconds."""
    import numpy as np
    import torch

    def bits(t):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)

    def timed(pieces):
        t0 = time.perf_counter()
        for xs, ws in pieces:
            oracle.group_rows(dtype, xs, ws)
        return time.perf_counter() - t0

    w0 = bits(w[0])
    r1, r2 = 32, 128
    t1 = timed([(bits(x[:r1]), w0)])
    t2 = timed([(bits(x[:r2]), w0)])
    per_row = max((t2 - t1) / (r2 - r1), 1e-9)
    fixed = max(t1 - per_row * r1, 0.0)
    total = int(sum(group_m))
    rows = int(min(total, max(r2, (target_s - fixed) / per_row)))
    pieces, row0, left = [], 0, rows
    for g, m in enumerate(group_m):
        take = min(int(m), left)
        if take > 0:
            pieces.append((bits(x[row0:row0 + take]), w0 if g == 0 else bits(w[g])))
        row0 += int(m)
        left -= take
        if left == 0:
            break
    dt = timed(pieces)
    flops = 2.0 * rows * n * k
    return {
        "value": round(flops / dt / 1e12, 6),
        "unit": "TFLOPS",
        "cores": oracle.threads(),
        "kind": "port",
        "sample": f"the first {rows} of {total} output rows (each against its group's w) x all "
                  f"{n} columns x K={k}: {flops / 1e9:.1f} GFLOP in {dt:.1f} s, fp32 OpenMP oracle",
    }


def other_pass(pkg, op, dtype, b, m, n, k, sh, dev):
    """Plan for a non-headline pass over the workload's forward shapes (x [sum(M), K],
    w [B, N, K], grad_out [sum(M), N]). Returns (plan, flops, buffers to keep alive)."""
    import torch

    td = torch.bfloat16 if dtype == 0 else torch.float16
    rows = b * m
    group_m = [m] * b

    def randn(shape, seed):
        t = torch.empty(shape, dtype=td, device=dev)
        pkg.fill_randn(pkg.DType(dtype), t.data_ptr(), t.numel(), seed, sh)
        return t

    if op == "dgrad":  # grad_x [sum(M), K] = grad_out [sum(M), N] @ w[g] [N, K]
        gy, w = randn((rows, n), 3), randn((b, n, k), 2)
        out = torch.zeros((rows, k), dtype=td, device=dev)
        plan = pkg.BackwardPlan("dgrad", pkg.DType(dtype), n, k, group_m, gy.data_ptr(), w.data_ptr(),
                                out.data_ptr(), sh)
        keep = (gy, w, out)
    elif op == "wgrad":  # grad_w [B, N, K] = grad_out[g]^T [N, M] @ x[g] [M, K]
        gy, x = randn((rows, n), 3), randn((rows, k), 1)
        out = torch.zeros((b, n, k), dtype=td, device=dev)
        plan = pkg.BackwardPlan("wgrad", pkg.DType(dtype), n, k, group_m, gy.data_ptr(), x.data_ptr(),
                                out.data_ptr(), sh)
        keep = (gy, x, out)
    elif op in ("dgrad_fp8", "wgrad_fp8"):  # e5m2 gradient, e4m3 other operand, unit scales
        gy = randn((rows, n), 3).to(torch.float8_e5m2)
        other = randn((b, n, k), 2) if op == "dgrad_fp8" else randn((rows, k), 1)
        other = other.to(torch.float8_e4m3fn)
        gs = torch.ones(1, dtype=torch.float32, device=dev)
        os_ = torch.ones(b, dtype=torch.float32, device=dev)
        out = torch.zeros((rows, k) if op == "dgrad_fp8" else (b, n, k), dtype=torch.bfloat16, device=dev)
        plan = pkg.BackwardPlan(op[:5], pkg.DType.FP8_E5M2, n, k, group_m, gy.data_ptr(), other.data_ptr(),
                                out.data_ptr(), sh, other_dtype=pkg.DType.FP8_E4M3, grad_scale=gs.data_ptr(),
                                other_scale=os_.data_ptr())
        keep = (gy, other, gs, os_, out)
    else:  # fp8 forward: N(0,1) inputs rounded to the fp8 format, unit scales, bf16 out
        fdt = torch.float8_e4m3fn if op == "fp8_e4m3" else torch.float8_e5m2
        x = randn((rows, k), 1).to(fdt)
        w = randn((b, n, k), 2).to(fdt)
        xs = torch.ones(1, dtype=torch.float32, device=dev)
        ws = torch.ones(b, dtype=torch.float32, device=dev)
        out = torch.zeros((rows, n), dtype=torch.bfloat16, device=dev)
        fmt = pkg.DType.FP8_E4M3 if op == "fp8_e4m3" else pkg.DType.FP8_E5M2
        plan = pkg.Fp8Plan(fmt, n, k, group_m, x.data_ptr(), w.data_ptr(), xs.data_ptr(), ws.data_ptr(),
                           out.data_ptr(), sh)
        keep = (x, w, xs, ws, out)
    torch.cuda.synchronize(dev)
    return plan, plan.flop, keep


def time_baselines(names, workload, dtype, b, m, n, k, warmup, steps):
    """The MI355X kernel and the named comparators in ONE native process (bin/gg_bench: the same
    buffers, inputs, sampled check, warmup and steps for each, one after the other), started as a
    child of this one. A native process, because torch ships its own libhipblaslt under the ROCm
    library's soname: in this process the comparators would run the wrong build. Returns
    {"source": ..., backend: {"status": "ok", "value": TFLOPS, "ms_per_step", "check", "detail"} or
    {"status": "n/a" | "error", "message"}}."""
    import csv
    import subprocess
    import tempfile

    exe = os.path.join(ROOT, "groupgemm-cktile-optimized_amd", "bin", "gg_bench")
    res = {"source": "bin/gg_bench, one native process: mi355x then " + ", ".join(names) +
                     f" on the same buffers, warmup {warmup}, {steps} timed steps each"}
    with tempfile.TemporaryDirectory() as tmp:
        shapes = os.path.join(tmp, "shapes.csv")
        rows_path = os.path.join(tmp, "rows.csv")
        with open(shapes, "w") as f:
            f.write(f"TestID,Case,B,M,N,K\n1,{workload},{b},{m},{n},{k}\n")
        cmd = [exe, "--shapes", shapes, "--dtype", "bf16" if dtype == 0 else "fp16", "--backends",
               ",".join(["mi355x"] + names), "--warmup", str(warmup), "--iters", str(steps), "--out", rows_path]
        try:
            p = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        except subprocess.TimeoutExpired:
            res["error"] = "gg_bench did not finish in 300 s"
            return res
        if not os.path.exists(rows_path):
            res["error"] = f"gg_bench exited {p.returncode}: {p.stderr.strip()[-500:]}"
            return res
        with open(rows_path) as f:
            for row in csv.DictReader(f):
                if row["Check"] in ("PASS", "SKIP"):
                    rec = {"status": "ok", "value": float(row["TFLOPS"]), "ms_per_step": float(row["Time_ms"]),
                           "check": row["Check"], "detail": row["Detail"]}
                elif row["Check"] == "N/A":
                    rec = {"status": "n/a", "message": row["Detail"]}
                else:
                    rec = {"status": "error", "check": row["Check"], "message": row["Detail"]}
                res[row["Backend"]] = rec
                log(f"[bench] gg_bench {row['Backend']}: {rec.get('value', rec.get('message'))}")
    return res


def traffic_for(pkg, workload, op, plan_detail):
    """(bytes per launch or None, provenance) from profiles/hbm_traffic_<workload>[_<op>].json."""
    suffix = "" if op == "fwd" else f"_{op}"
    rel = os.path.join("profiles", f"hbm_traffic_{workload}{suffix}.json")
    path = os.path.join(ROOT, rel)
    if not os.path.exists(path):
        return None, {"file": None, "status": "no profile for this workload"}
    with open(path) as f:
        data = json.load(f)
    sha = pkg.kernel_source_sha()
    info = {"file": rel, "commit": data.get("commit"), "kernel": data.get("kernel"),
            "kernel_source_sha": data.get("kernel_source_sha"), "plan": data.get("plan"),
            "traffic_over_algorithmic": data.get("traffic_over_algorithmic")}
    if data.get("kernel_source_sha") != sha or data.get("plan") != plan_detail:
        info["status"] = (f"not used: measured on kernel sources {data.get('kernel_source_sha')} with plan "
                          f"{data.get('plan')!r}; this build is {sha} with plan {plan_detail!r}")
        return None, info
    info["status"] = "current: same kernel sources and plan"
    return data.get("hbm_bytes_per_launch"), info


def peak_of(op):
    return FP8_PEAK_TFLOPS if "fp8" in op else MFMA_PEAK_TFLOPS


def sustained_clock_power(pkg, be, sh, stream, flops, ms, seconds, peak):
    """Run the same launch back to back for about `seconds`. The effective shader clock over the
    window comes from the clock probe (gg_clock_probe: one wave on a second stream reading
    s_memtime against s_memrealtime over the first 70 % of the window; it holds a few VGPRs and
    no LDS, so the GEMM's workgroups run beside it). A background thread samples amdsmi's gfx clock
    and socket power meanwhile. Returns the window's TFLOPS, the probe's clock and the dense peak
    scaled to it (peak x MHz / 2400), and the amdsmi readings, whose clock is flagged inconsistent
    when it differs from the probe's by more than 5 %."""
    import torch

    power = entry.load_submodule("power")
    sampler = power.PowerSampler(0)
    n = max(1, int(seconds / max(ms * 1e-3, 1e-6)))
    words = torch.zeros(5, dtype=torch.int64, device=stream.device)
    side = torch.cuda.Stream(device=stream.device)  # default priority
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with sampler:
        # the probe first, so that it is resident before the GEMM's workgroups arrive
        pkg.clock_probe(words.data_ptr(), 0.7 * n * ms * 1e-3, side.cuda_stream)
        t0.record(stream)
        for _ in range(n):
            be.run(sh)
        t1.record(stream)
        torch.cuda.synchronize()
    sampler.close()
    smi = sampler.summary()
    w_ms = t0.elapsed_time(t1)
    mask = (1 << 64) - 1
    mhz = pkg.probe_mhz([int(v) & mask for v in words.cpu().tolist()])
    res = {"steps": n, "seconds": round(w_ms * 1e-3, 3),
           "tflops": round(flops * n / (w_ms * 1e-3) / 1e12, 2),
           "gfx_mhz": round(mhz, 1),
           "gfx_mhz_source": "clock probe: shader clock counter (s_memtime) over the wall clock (s_memrealtime) "
                             "of one wave on a second stream, the window's first 70 %",
           "peak_at_clock_tflops": round(peak * mhz / 2400.0, 1),
           "frac_at_clock": round(flops * n / (w_ms * 1e-3) / 1e12 / (peak * mhz / 2400.0), 4),
           "socket_w": smi.get("socket_w"), "socket_w_max": smi.get("socket_w_max"),
           "power_cap_w": sampler.power_cap_w}
    a_mhz = smi.get("gfx_mhz")
    smi["consistent_with_probe"] = bool(a_mhz) and abs(a_mhz - mhz) <= 0.05 * mhz
    smi["source"] = "amdsmi: clock_info(GFX).clk, power_info.current_socket_power, gpu_metrics current_gfxclks"
    res["amdsmi"] = smi
    return res


def timed_region_clock(ms, traffic_profile_status, workload, op):
    """Effective clock of the timed region: the GRBM cycles per launch of the matching profile
    (same kernel sources and plan) over this run's mean launch time; None with the reason if the
    profile does not match."""
    suffix = "" if op == "fwd" else f"_{op}"
    rel = os.path.join("profiles", f"hbm_traffic_{workload}{suffix}.json")
    if not traffic_profile_status.startswith("current"):
        return {"gfx_mhz": None, "reason": f"{rel} was not measured on this build's kernel sources and plan"}
    with open(os.path.join(ROOT, rel)) as f:
        cycles = json.load(f).get("cycles_per_launch")
    if not cycles:
        return {"gfx_mhz": None, "reason": f"{rel} holds no cycles_per_launch"}
    return {"gfx_mhz": round(cycles / (ms * 1e-3) / 1e6, 1), "cycles_per_launch": cycles,
            "source": f"GRBM_GUI_ACTIVE per XCD from {rel} over this run's ms_per_step"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=HEADLINE, choices=sorted(WORKLOADS))
    ap.add_argument("--op", default="fwd", choices=OPS,
                    help="pass to time (fwd is the headline; the others print no cpu_baseline)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--power-seconds", type=float, default=1.0,
                    help="sustained window sampled for clock and power after the timed region "
                         "(0: skip)")
    ap.add_argument("--baselines", default="hipblaslt_loop,hipblaslt_seq",
                    help="comparison backends timed with the MI355X kernel in bin/gg_bench after the timed "
                         "region (forward only; '' for none)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="BYTES",
                    help="only run 3 device copies of BYTES bytes (reference kernel for the "
                         "FETCH_SIZE / WRITE_SIZE scale factors) and exit")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build measures one MI355X only (asked for --gpus {args.gpus}); "
              "groups shard across GPUs without any exchange, see DESIGN.md", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.calibrate_copy:
        src = torch.ones(args.calibrate_copy, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": args.calibrate_copy, "copies": 3}), flush=True)
        return

    pkg = entry.load_package()
    dtype, b, m, n, k = WORKLOADS[args.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    td = torch.bfloat16 if dtype == 0 else torch.float16
    group_m = [m] * b
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    if args.op == "fwd":
        x = torch.empty((b * m, k), dtype=td, device=dev)
        w = torch.empty((b, n, k), dtype=td, device=dev)
        out = torch.zeros((b * m, n), dtype=td, device=dev)
        pkg.fill_randn(pkg.DType(dtype), x.data_ptr(), x.numel(), 1, sh)
        pkg.fill_randn(pkg.DType(dtype), w.data_ptr(), w.numel(), 2, sh)
        prob = pkg.GroupedGemmProblem(pkg.DType(dtype), b, n, k, group_m, x.data_ptr(), w.data_ptr(),
                                      out.data_ptr())
        be = pkg.make_mi355x_backend()
        why = be.prepare(prob, sh)
        if why:
            raise SystemExit(f"mi355x backend cannot run {args.workload}: {why}")
        flops = prob.flops()
    else:
        be, flops, keep = other_pass(pkg, args.op, dtype, b, m, n, k, sh, dev)
    plan_detail = be.detail()
    log(f"[bench] {args.workload} {args.op}: {plan_detail}")

    for _ in range(args.warmup):
        be.run(sh)
    torch.cuda.synchronize(dev)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        be.run(sh)
    stop.record(stream)
    torch.cuda.synchronize(dev)
    ms = start.elapsed_time(stop) / args.steps
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"[bench] {args.steps} steps, {ms:.4f} ms/step, {tflops:.1f} TFLOPS")

    baselines = None
    names = [b_ for b_ in args.baselines.split(",") if b_]
    if names and args.op == "fwd":
        baselines = time_baselines(names, args.workload, dtype, b, m, n, k, args.warmup, args.steps)
        ours = baselines.get("mi355x", {})
        for name in names:
            rec = baselines.get(name, {})
            if rec.get("status") == "ok" and ours.get("status") == "ok":
                rec["mi355x_speedup_same_process"] = round(ours["value"] / rec["value"], 3)

    clock_power = None
    if args.power_seconds > 0:
        clock_power = sustained_clock_power(pkg, be, sh, stream, flops, ms, args.power_seconds, peak_of(args.op))
        log(f"[bench] sustained {clock_power.get('seconds')} s: {clock_power.get('tflops')} TFLOPS at "
            f"{clock_power.get('gfx_mhz')} MHz (probe; amdsmi {clock_power['amdsmi'].get('gfx_mhz')} MHz), "
            f"{clock_power.get('socket_w')} W")

    traffic, traffic_profile = traffic_for(pkg, args.workload, args.op, plan_detail)
    timed_clock = timed_region_clock(ms, traffic_profile.get("status", ""), args.workload, args.op)

    cpu = None
    if not args.no_cpu_baseline and args.op == "fwd":
        log(f"[bench] cpu baseline (~{args.cpu_seconds:.0f} s of CPU work)...")
        cpu = cpu_baseline(entry.load_oracle(), x, w, group_m, dtype, n, k, args.cpu_seconds)
        log(f"[bench] cpu baseline: {cpu['value']} TFLOPS on {cpu['cores']} threads")
    be.release()

    fp8 = "fp8" in args.op
    peak = peak_of(args.op)
    metric = "grouped-GEMM TFLOPS (bf16) + % of MFMA peak, 1 MI355X, per config"
    if args.op != "fwd":
        metric = f"grouped-GEMM {args.op} TFLOPS + % of MFMA peak, 1 MI355X"
    line = {
        "metric": metric,
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("e5m2 x e4m3" if args.op.endswith("_fp8") else args.op[4:]) if fp8
                 else "bf16" if dtype == 0 else "fp16",
        "data": "synthetic (seeded N(0,1), balanced groups)",
        "config": {"workload": args.workload, "op": args.op, "groups": b, "m_per_group": m, "n": n,
                   "k": k, "layout": "RCR", "parallelism": "single GPU"},
        "pct_of_mfma_peak": round(100.0 * tflops / peak, 2),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(tflops / peak, 4),
                     "traffic": traffic},
        "traffic_profile": traffic_profile,
        "baselines": baselines,
        "cpu_baseline": cpu,
        "timed_region_clock": timed_clock,
        "clock_power": clock_power,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
