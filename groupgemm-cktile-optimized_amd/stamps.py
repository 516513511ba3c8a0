"""Where a cross-tile launch spends its cycles: the kernel's s_memtime stamps, per workgroup and tile.

Needs the instrumented library (GG_STAMPS=1 in csrc/gg_kernel_impl.h), built on the CPU with

    make -C groupgemm-cktile-optimized_amd -j16 stamps      # -> lib_stamps/libgg_mi355x.so

and runs on the GPU box from the repository root:

    python3 groupgemm-cktile-optimized_amd/stamps.py [--shapes '[[b, m, n, k], ...]'] [--fp16]
        [--op fwd|dgrad|wgrad|fp8_e4m3|fp8_e5m2|dgrad_fp8|wgrad_fp8] [--json gpurun_out/stamps.json]

Per shape (balanced groups of m rows in forward terms: x [b m, k], w [b, n, k]; 16-bit forward
through the mi355x backend, or the pass --op names, planned as bench.py plans it): 10 warm
launches, then one launch whose stamps are read back. Lane 0 of wave 0 of every workgroup stamps
the shader clock at kernel start, after the prologue, and for each of its first 7 tiles before
its first K step, after it, after the unchecked K steps, after locating the next tile and after
the tile's last K step, before the final LDS epilogue and at kernel end. The shader clocks of
different CUs are not synchronised (they differ by millions of cycles, also within an XCD), so
only differences of one workgroup's own stamps are used. Printed, averaged over workgroups
(cycles):
  - the launch per workgroup (start to end), the prologue and the final LDS epilogue;
  - per tile: the first K step (which also stores the previous tile's C from registers), the
    unchecked steps (and their cost per step), the next tile's lookup, the checked steps (the
    last ones, whose DMAs fetch the next tile), and the gap to the next tile's first step;
  - the tile's cost beyond its K steps at the unchecked rate ("boundary").
The stamps' own stores count in vmcnt, so an instrumented launch is a little slower than a plain
one; the stamped launch also follows a pause (the host clears the stamps), so its clock and
memory state differ from back-to-back launches, and a shape's first launches in a process run
slower than later ones. Compare segments of one launch, and shapes run in the same order.
"""
from __future__ import annotations

import argparse
import ctypes
import importlib.util
import json
import os
import sys

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
STAMP_LIB = os.path.join(PKG_DIR, "lib_stamps", "libgg_mi355x.so")
SLOTS, WGS, PARTS = 64, 1024, 20


def load_package():
    spec = importlib.util.spec_from_file_location("gg_stamps_pkg", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    pkg = importlib.util.module_from_spec(spec)
    sys.modules["gg_stamps_pkg"] = pkg
    spec.loader.exec_module(pkg)
    if not os.path.exists(STAMP_LIB):
        raise SystemExit(f"{STAMP_LIB} missing: build it with `make -C {PKG_DIR} -j16 stamps`")
    lib = pkg.load_library(STAMP_LIB)
    return pkg, lib


def part_fns(lib):
    fns = []
    for p in range(PARTS):
        rd = getattr(lib, f"gg_stamps_read_p{p}", None)
        clr = getattr(lib, f"gg_stamps_clear_p{p}", None)
        if rd is None or clr is None:
            raise SystemExit("the library has no stamp functions: it is not the GG_STAMPS build")
        rd.argtypes = [ctypes.c_void_p]
        fns.append((rd, clr))
    return fns


def unchecked_steps(T: int, masks: bool) -> int:
    """K steps the kernel's unchecked loop runs: kt = 1, 7, ... while kt + 9 < T (instances with
    tail masks) or kt + 8 < T (without), six per pass."""
    lead = 9 if masks else 8
    passes = max(0, (T - lead - 1 + 5) // 6)
    return 6 * passes


REAL_START, REAL_END = 48, 49  # s_memrealtime at kernel start and end (kStampRealStart / End)


def per_xcd(st: np.ndarray, hz: float, n_xcd: int = 8) -> list:
    """Wall time and shader clock per XCD from the constant-rate stamps (workgroup w runs on XCD
    w % n_xcd). Times in microseconds from the launch's first workgroup start."""
    grid = st.shape[0]
    t0 = st[:, REAL_START].min()
    rows = []
    for x in range(min(n_xcd, grid)):
        w = np.arange(x, grid, n_xcd)
        ticks = (st[w, REAL_END] - st[w, REAL_START]).astype(np.float64)
        cyc = (st[w, 63] - st[w, 0]).astype(np.float64)
        rows.append({
            "xcd": x,
            "start_us_max": float((st[w, REAL_START] - t0).max() / hz * 1e6),
            "end_us_mean": float((st[w, REAL_END] - t0).mean() / hz * 1e6),
            "end_us_max": float((st[w, REAL_END] - t0).max() / hz * 1e6),
            "wall_us_mean": float(ticks.mean() / hz * 1e6),
            "cycles_mean": float(cyc.mean()),
            "mhz": float((cyc / (ticks / hz)).mean() / 1e6),
        })
    return rows


def analyse(st: np.ndarray, T: int, masks: bool) -> dict:
    """st: [grid, 64] stamps of one launch (int64); masks: the instance has tail masks."""
    grid = st.shape[0]
    total = st[:, 63] - st[:, 0]
    tiles = np.array([int(sum(1 for j in range(7) if st[w, 2 + 5 * j] > 0)) for w in range(grid)])
    nun = unchecked_steps(T, masks)
    seg = {"first step": [], "unchecked": [], "next tile lookup": [], "checked": [], "gap to next tile": []}
    for w in range(grid):
        for j in range(tiles[w]):
            s = st[w, 2 + 5 * j: 7 + 5 * j]
            seg["first step"].append(s[1] - s[0])
            seg["unchecked"].append(s[2] - s[1])
            seg["next tile lookup"].append(s[3] - s[2])
            seg["checked"].append(s[4] - s[3])
            if j + 1 < tiles[w]:
                seg["gap to next tile"].append(st[w, 2 + 5 * (j + 1)] - s[4])
    out = {
        "grid": grid, "k_steps": T, "unchecked_steps_per_tile": nun,
        "launch_cycles_mean": float(total.mean()), "launch_cycles_max": float(total.max()),
        "tiles_per_wg_max": int(tiles.max()),
        "prologue": float((st[:, 1] - st[:, 0]).mean()),
        "final_epilogue": float((st[:, 63] - st[:, 62]).mean()) if (st[:, 62] > 0).all() else float("nan"),
    }
    for k, v in seg.items():
        out[k] = float(np.mean(v)) if v else 0.0
    per_step = out["unchecked"] / nun if nun else float("nan")
    out["unchecked_per_step"] = per_step
    if nun:
        tile = out["first step"] + out["unchecked"] + out["next tile lookup"] + out["checked"] + out["gap to next tile"]
        out["tile_cycles"] = tile
        out["boundary"] = tile - T * per_step
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--shapes", default="[[8, 4096, 7168, 2048], [32, 520, 2880, 2880], [8, 4096, 4096, 7168]]")
    ap.add_argument("--fp16", action="store_true")
    ap.add_argument("--op", default="fwd",
                    choices=["fwd", "dgrad", "wgrad", "fp8_e4m3", "fp8_e5m2", "dgrad_fp8", "wgrad_fp8"])
    ap.add_argument("--json", default="")
    args = ap.parse_args()
    import torch

    pkg, lib = load_package()
    fns = part_fns(lib)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    sh = torch.cuda.current_stream(dev).cuda_stream
    words = torch.zeros(5, dtype=torch.int64, device=dev)
    lib.gg_clock_probe(words.data_ptr(), 0.001, sh)  # its fifth word: the constant clock's rate (Hz)
    torch.cuda.synchronize()
    real_hz = float(words[4].item())
    dt = pkg.DType.FP16 if args.fp16 else pkg.DType.BF16
    tdt = torch.float16 if args.fp16 else torch.bfloat16
    results = []
    for b, m, n, k in json.loads(args.shapes):
        print(f"[stamps] {args.op} shape {b} x {m} x {n} x {k}", flush=True)
        keep = None
        if args.op == "fwd":
            x = torch.empty((b * m, k), dtype=tdt, device=dev)
            w = torch.empty((b, n, k), dtype=tdt, device=dev)
            out = torch.zeros((b * m, n), dtype=tdt, device=dev)
            pkg.fill_randn(dt, x.data_ptr(), x.numel(), 1, sh)
            pkg.fill_randn(dt, w.data_ptr(), w.numel(), 2, sh)
            keep = (x, w, out)
            be = pkg.make_mi355x_backend()
            why = be.prepare(pkg.GroupedGemmProblem(dt, b, n, k, [m] * b, x.data_ptr(), w.data_ptr(),
                                                    out.data_ptr()), sh)
            if why:
                raise SystemExit(f"prepare: {why}")
            grid_of = be.grid
        else:
            sys.path.insert(0, os.path.dirname(PKG_DIR))
            import bench  # the other passes' plans and inputs, as the benchmark makes them

            be, _, keep = bench.other_pass(pkg, args.op, 1 if args.fp16 else 0, b, m, n, k, sh, dev)
            grid_of = lambda: lib.gg_plan_grid(be._plan)  # noqa: E731
        detail = be.detail()
        for _ in range(10):
            be.run(sh)
        torch.cuda.synchronize()
        for _, clr in fns:
            if clr() != 0:
                raise SystemExit("stamp clear failed")
        be.run(sh)
        torch.cuda.synchronize()
        grid = grid_of()
        best = None
        for rd, _ in fns:
            buf = np.zeros(WGS * SLOTS, dtype=np.uint64)
            if rd(buf.ctypes.data) != 0:
                raise SystemExit("stamp read failed")
            st = buf.reshape(WGS, SLOTS)[:grid].astype(np.int64)
            if (st[:, 0] > 0).all() and (st[:, 63] > 0).all():
                best = st
                break
        be.release()
        del keep
        if best is None:
            print(f"  {detail}: no part holds a complete set of stamps (per-tile plan?)", flush=True)
            continue
        contraction = {"dgrad": n, "wgrad": m}.get(args.op.split("_")[0], k)
        ks = 128 if "fp8" in args.op else 64
        # the plan's tails flag (KernelArgs::tails), for balanced groups
        kind = args.op.split("_")[0]
        if kind == "dgrad":
            masks = n % ks != 0 or k % 256 != 0
        elif kind == "wgrad":
            masks = m % ks != 0 or m < 4 * ks or n % 256 != 0 or k % 256 != 0
        else:
            masks = k % ks != 0
        r = analyse(best, -(-contraction // ks), masks)
        if real_hz > 0 and (best[:, REAL_START] > 0).all() and (best[:, REAL_END] > 0).all():
            r["per_xcd"] = per_xcd(best, real_hz)
        r.update({"shape": [b, m, n, k], "plan": detail, "stamps": best.tolist()})
        results.append(r)
        print(f"  {detail}", flush=True)
        print(f"  launch per workgroup: mean {r['launch_cycles_mean']:.0f}, max {r['launch_cycles_max']:.0f} cycles; "
              f"{r['tiles_per_wg_max']} tiles stamped (a workgroup's first 7 at most), {r['k_steps']} K steps each", flush=True)
        print(f"  prologue {r['prologue']:.0f}; final epilogue {r['final_epilogue']:.0f}", flush=True)
        print(f"  per tile: first step {r['first step']:.0f} | unchecked {r['unchecked']:.0f} "
              f"({r['unchecked_steps_per_tile']} steps, {r['unchecked_per_step']:.0f} each) | next-tile lookup "
              f"{r['next tile lookup']:.0f} | checked {r['checked']:.0f} | gap {r['gap to next tile']:.0f}", flush=True)
        if "boundary" in r:
            print(f"  tile {r['tile_cycles']:.0f} cycles, of which {r['boundary']:.0f} beyond its K steps at the "
                  f"unchecked rate", flush=True)
        for x in r.get("per_xcd", []):
            print(f"  XCD {x['xcd']}: wall {x['wall_us_mean']:8.1f} us, ends at {x['end_us_mean']:8.1f} "
                  f"(max {x['end_us_max']:8.1f}, last start {x['start_us_max']:6.1f}) us, {x['cycles_mean']:10.0f} "
                  f"cycles, {x['mhz']:7.1f} MHz", flush=True)
    if args.json:
        os.makedirs(os.path.dirname(os.path.abspath(args.json)), exist_ok=True)
        with open(args.json, "w") as f:
            json.dump(results, f, indent=1)


if __name__ == "__main__":
    main()
