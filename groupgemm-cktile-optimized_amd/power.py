"""GPU clock and socket-power sampling around a timed region.

The reference records the socket power and gfx clock of the busiest GPU with `amd-smi metric`
next to its timing runs (scripts/power.py:1-9), because the MI355X is power-capped and the
clock under a sustained GEMM sits well below its 2.4 GHz maximum. This module does the same
in-process through the amdsmi Python library, sampling on a background thread while the GPU
works, so that a TFLOPS figure comes with the clock and power it was measured at.

The device is matched to the HIP device by PCI bus id; if that fails, the busiest GPU (the one
with the highest socket power in a first sample) is taken, as the reference does. Sampling
never raises into the caller: when amdsmi is unavailable the result says why.
"""
from __future__ import annotations

import ctypes
import threading
import time


def _hip_bdf(device: int) -> str | None:
    """PCI bus id (domain:bus:device.function, lower case) of a HIP device."""
    for name in ("libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6"):
        try:
            hip = ctypes.CDLL(name)
            break
        except OSError:
            continue
    else:
        return None
    buf = ctypes.create_string_buffer(64)
    if hip.hipDeviceGetPCIBusId(buf, ctypes.c_int(64), ctypes.c_int(device)) != 0:
        return None
    return buf.value.decode().strip().lower()


def _norm_bdf(s: str) -> str:
    s = s.strip().lower()
    parts = s.split(":")
    if len(parts) == 3:  # dddd:bb:dd.f -> drop leading zeros of the domain
        return f"{int(parts[0], 16):x}:{parts[1]}:{parts[2]}"
    return s


class PowerSampler:
    """Samples gfx clock (MHz) and current socket power (W) every `period_s` while active.

    with PowerSampler(device=0) as ps:
        ... GPU work ...
    ps.summary() -> {"gfx_mhz": mean, "socket_w": mean, "samples": n, ...} or {"error": ...}
    """

    def __init__(self, device: int = 0, period_s: float = 0.002):
        self.device, self.period_s = device, period_s
        self.error: str | None = None
        self._smi = self._handle = None
        self._clk: list[float] = []
        self._pw: list[float] = []
        self._xcd: list[float] = []  # metrics table: mean of the per-XCD current gfx clocks
        self._avg: list[float] = []  # metrics table: the SMU's average gfx clock
        self._thr: dict = {}
        self._metrics_ok = True
        self._t = (0.0, 0.0)
        self._stop = threading.Event()
        self._thread: threading.Thread | None = None
        self.power_cap_w = None
        try:
            import amdsmi

            self._smi = amdsmi
            amdsmi.amdsmi_init()
            handles = amdsmi.amdsmi_get_processor_handles()
            if not handles:
                raise RuntimeError("amdsmi lists no GPU")
            want = _hip_bdf(device)
            pick = None
            if want is not None:
                for h in handles:
                    try:
                        if _norm_bdf(amdsmi.amdsmi_get_gpu_device_bdf(h)) == _norm_bdf(want):
                            pick = h
                            break
                    except Exception:  # noqa: BLE001 - a handle without a bdf is skipped
                        continue
            if pick is None:  # the busiest GPU, as the reference's power.py takes it
                pick = max(handles, key=self._power_of)
            self._handle = pick
            try:
                cap = amdsmi.amdsmi_get_power_cap_info(pick).get("power_cap")
                self.power_cap_w = round(cap / 1e6, 1) if isinstance(cap, (int, float)) and cap > 0 else None
            except Exception:  # noqa: BLE001
                self.power_cap_w = None
        except Exception as e:  # noqa: BLE001 - report, never fail the benchmark
            self.error = f"{type(e).__name__}: {e}"

    def _power_of(self, h) -> float:
        try:
            p = self._smi.amdsmi_get_power_info(h).get("current_socket_power")
            return float(p) if isinstance(p, (int, float)) else -1.0
        except Exception:  # noqa: BLE001
            return -1.0

    def _sample(self):
        smi, h = self._smi, self._handle
        try:
            clk = smi.amdsmi_get_clock_info(h, smi.AmdSmiClkType.GFX).get("clk")
            pw = smi.amdsmi_get_power_info(h).get("current_socket_power")
            if isinstance(clk, (int, float)):
                self._clk.append(float(clk))
            if isinstance(pw, (int, float)):
                self._pw.append(float(pw))
        except Exception as e:  # noqa: BLE001
            self.error = f"{type(e).__name__}: {e}"
            self._stop.set()
            return
        if self._metrics_ok:
            try:
                m = smi.amdsmi_get_gpu_metrics_info(h)
            except Exception:  # noqa: BLE001 - the metrics table is optional
                self._metrics_ok = False
                return
            xcd = [float(v) for v in (m.get("current_gfxclks") or []) if isinstance(v, (int, float)) and v > 0]
            if xcd:
                self._xcd.append(sum(xcd) / len(xcd))
            avg = m.get("average_gfxclk_frequency")
            if isinstance(avg, (int, float)) and avg > 0:
                self._avg.append(float(avg))
            for key in ("throttle_status", "indep_throttle_status"):
                v = m.get(key)
                if v not in (None, "N/A"):
                    self._thr[key] = v

    def _run(self):
        while not self._stop.is_set():
            self._sample()
            self._stop.wait(self.period_s)

    def __enter__(self):
        self._clk, self._pw, self._xcd, self._avg, self._thr = [], [], [], [], {}
        self._t = (time.perf_counter(), 0.0)
        if self.error is None:
            self._stop.clear()
            self._thread = threading.Thread(target=self._run, daemon=True)
            self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self._thread is not None:
            self._thread.join()
            self._thread = None
        self._t = (self._t[0], time.perf_counter())
        return False

    def summary(self) -> dict:
        out = {"window_s": round(self._t[1] - self._t[0], 3)}
        if self.error is not None and not self._clk:
            out["error"] = self.error
            return out
        out["samples"] = len(self._clk)
        out["gfx_mhz"] = round(sum(self._clk) / len(self._clk), 1) if self._clk else None
        out["gfx_mhz_min"] = min(self._clk) if self._clk else None
        out["socket_w"] = round(sum(self._pw) / len(self._pw), 1) if self._pw else None
        out["socket_w_max"] = max(self._pw) if self._pw else None
        mean = lambda v: round(sum(v) / len(v), 1) if v else None  # noqa: E731
        out["xcd_gfx_mhz"] = mean(self._xcd)
        out["avg_gfx_mhz"] = mean(self._avg)
        if self._thr:
            out["throttle"] = self._thr
        return out

    def close(self):
        if self._smi is not None and self.error is None:
            try:
                self._smi.amdsmi_shut_down()
            except Exception:  # noqa: BLE001
                pass
