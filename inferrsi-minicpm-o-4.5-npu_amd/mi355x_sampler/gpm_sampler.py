"""Device activity of one MI355X, sampled on the host clock (diagnostic); the AMD counterpart of the reference's
NVML GPM sampler (``tools/gpm_sampler.py:20-62``).

    python -m mi355x_sampler.gpm_sampler --gpu 0 --out gpm.jsonl [--period 0.5]

Every period it writes one JSON row over the interval since the previous one, with the reference's keys, on
``time.perf_counter`` (CLOCK_MONOTONIC, the clock of an engine stage trace):

``t0``, ``t1``
    the interval on ``time.perf_counter``.
``sm_util``
    GFX engine busy, percent: the mean over the interval's sub-samples of the per-XCC instantaneous busy figures
    (``xcp_stats.gfx_busy_inst``), or of the firmware's ``average_gfx_activity`` where those are absent.
``dram_bw_util``
    memory-controller (UMC) activity, percent (``average_umc_activity``): the share of time the HBM controllers
    were busy, the nearest SMI figure to NVML's DRAM bandwidth utilisation.
``graphics_util``
    ``average_gfx_activity``, percent.
``sm_occupancy``, ``tensor_util``, ``fp16_util``, ``fp32_util``
    ``null``: the SMI exposes no counterpart (wave occupancy and pipe utilisation come from rocprofv3's counters).

AMD-only extras: ``xcc_busy`` (per-XCC busy percent, interval means) and ``samples`` (sub-samples averaged).  The
figures are device-wide: they cover every process on the GPU.  Stops on SIGTERM or SIGINT.  The sampling is
separate from the rows' arithmetic (``interval_row``), which is what the CPU tests check.
"""

from __future__ import annotations

import argparse
import json
import math
import signal
import time

KEYS = ("sm_util", "sm_occupancy", "dram_bw_util", "tensor_util", "fp16_util", "fp32_util", "graphics_util")
NO_COUNTERPART = ("sm_occupancy", "tensor_util", "fp16_util", "fp32_util")
SUBSAMPLES = 5  # readings per period


def _num(v):
    """A finite number from an SMI field, or None ("N/A", out-of-range sentinels, missing)."""
    if isinstance(v, bool) or not isinstance(v, (int, float)):
        return None
    v = float(v)
    if not math.isfinite(v) or v < 0 or v > 100.0 + 1e-9:
        return None
    return v


def reading(metrics: dict) -> dict:
    """The activity figures of one ``amdsmi_get_gpu_metrics_info`` result (percent, or None)."""
    xcc = metrics.get("xcp_stats.gfx_busy_inst")
    busy = []
    if isinstance(xcc, list):
        for part in xcc:
            vals = part if isinstance(part, list) else [part]
            busy.extend(x for x in (_num(v) for v in vals) if x is not None)
    gfx = _num(metrics.get("average_gfx_activity"))
    return {"xcc_busy": busy, "graphics_util": gfx, "dram_bw_util": _num(metrics.get("average_umc_activity"))}


def _mean(xs):
    xs = [x for x in xs if x is not None]
    return round(sum(xs) / len(xs), 3) if xs else None


def interval_row(t0: float, t1: float, readings: list[dict]) -> dict:
    """One output row from the readings taken in [t0, t1] (the reference's keys, null where no counterpart)."""
    row = {"t0": round(t0, 6), "t1": round(t1, 6)}
    nx = max((len(r["xcc_busy"]) for r in readings), default=0)
    xcc = [_mean([r["xcc_busy"][i] for r in readings if i < len(r["xcc_busy"])]) for i in range(nx)]
    gfx = _mean([r["graphics_util"] for r in readings])
    sm = _mean(xcc) if any(v is not None for v in xcc) else gfx
    vals = {"sm_util": sm, "dram_bw_util": _mean([r["dram_bw_util"] for r in readings]), "graphics_util": gfx}
    for k in KEYS:
        row[k] = None if k in NO_COUNTERPART else vals[k]
    row["xcc_busy"] = xcc
    row["samples"] = len(readings)
    return row


class Device:
    """One GPU through amdsmi (imported here: the CPU tests of the row arithmetic do not need it)."""

    def __init__(self, index: int):
        import amdsmi

        self.smi = amdsmi
        amdsmi.amdsmi_init()
        handles = amdsmi.amdsmi_get_processor_handles()
        if not 0 <= index < len(handles):
            amdsmi.amdsmi_shut_down()
            raise SystemExit(f"no GPU {index}: {len(handles)} visible")
        self.handle = handles[index]

    def read(self) -> dict:
        try:
            return reading(self.smi.amdsmi_get_gpu_metrics_info(self.handle))
        except self.smi.AmdSmiException:
            return {"xcc_busy": [], "graphics_util": None, "dram_bw_util": None}

    def close(self) -> None:
        self.smi.amdsmi_shut_down()


def run(dev, out_path: str, period: float, stop: list, max_rows: int | None = None) -> int:
    """Writes rows until ``stop`` is non-empty (or ``max_rows`` rows); returns the number written."""
    n = 0
    t_prev = time.perf_counter()
    with open(out_path, "a") as f:
        while not stop and (max_rows is None or n < max_rows):
            readings = []
            for _ in range(SUBSAMPLES):
                time.sleep(period / SUBSAMPLES)
                readings.append(dev.read())
                if stop:
                    break
            t = time.perf_counter()
            f.write(json.dumps(interval_row(t_prev, t, readings)) + "\n")
            f.flush()
            n += 1
            t_prev = t
    return n


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpu", type=int, required=True)
    ap.add_argument("--out", required=True)
    ap.add_argument("--period", type=float, default=0.5)
    ap.add_argument("--rows", type=int, default=None, help="stop after this many rows (default: run until SIGTERM)")
    a = ap.parse_args(argv)
    if a.period <= 0:
        raise SystemExit("--period must be positive")
    stop: list = []
    signal.signal(signal.SIGTERM, lambda *_: stop.append(1))
    signal.signal(signal.SIGINT, lambda *_: stop.append(1))
    dev = Device(a.gpu)
    try:
        run(dev, a.out, a.period, stop, a.rows)
    finally:
        dev.close()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
