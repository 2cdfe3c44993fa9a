"""The device-activity sampler (``mi355x_sampler.gpm_sampler``), the AMD counterpart of ``tools/gpm_sampler.py``.

CPU tests check the row arithmetic and schema against a fake device; the ``gpu`` test samples the real MI355X
through amdsmi while a sampling kernel runs.
"""

from __future__ import annotations

import json
import subprocess
import sys
import threading

import pytest

from mi355x_sampler import gpm_sampler as gs

# the keys the reference's rows carry (tools/gpm_sampler.py:20-22, :57-59)
REF_KEYS = {"t0", "t1", "sm_util", "sm_occupancy", "dram_bw_util", "tensor_util", "fp16_util", "fp32_util",
            "graphics_util"}


def test_reading_parses_smi_fields_and_sentinels():
    m = {"xcp_stats.gfx_busy_inst": [[10, 30, "N/A", 200], ["N/A"] * 4], "average_gfx_activity": 40,
         "average_umc_activity": "N/A"}
    r = gs.reading(m)
    assert r == {"xcc_busy": [10.0, 30.0], "graphics_util": 40.0, "dram_bw_util": None}
    assert gs.reading({}) == {"xcc_busy": [], "graphics_util": None, "dram_bw_util": None}


def test_interval_row_means_and_nulls():
    rd = [{"xcc_busy": [10.0, 20.0], "graphics_util": 30.0, "dram_bw_util": 5.0},
          {"xcc_busy": [30.0, 40.0], "graphics_util": None, "dram_bw_util": 7.0}]
    row = gs.interval_row(1.0, 1.5, rd)
    assert set(row) >= REF_KEYS
    assert row["t0"] == 1.0 and row["t1"] == 1.5
    assert row["xcc_busy"] == [20.0, 30.0]
    assert row["sm_util"] == 25.0  # mean over XCCs of the interval means
    assert row["graphics_util"] == 30.0 and row["dram_bw_util"] == 6.0
    for k in gs.NO_COUNTERPART:
        assert row[k] is None
    # no per-XCC figures: the engine-wide average stands in
    row = gs.interval_row(0.0, 1.0, [{"xcc_busy": [], "graphics_util": 12.0, "dram_bw_util": None}])
    assert row["sm_util"] == 12.0 and row["dram_bw_util"] is None


class _FakeDevice:
    def __init__(self):
        self.n = 0

    def read(self):
        self.n += 1
        return {"xcc_busy": [float(self.n)] * 8, "graphics_util": 50.0, "dram_bw_util": 25.0}


def test_run_writes_jsonl_on_the_perf_counter_clock(tmp_path):
    out = tmp_path / "gpm.jsonl"
    n = gs.run(_FakeDevice(), str(out), 0.01, [], max_rows=3)
    rows = [json.loads(line) for line in out.read_text().splitlines()]
    assert n == 3 and len(rows) == 3
    for a, b in zip(rows, rows[1:]):
        assert a["t1"] == b["t0"]  # contiguous intervals
    for r in rows:
        assert set(r) >= REF_KEYS and r["t1"] > r["t0"] and r["samples"] == gs.SUBSAMPLES


def test_run_stops_when_signalled(tmp_path):
    stop: list = []
    out = tmp_path / "gpm.jsonl"
    th = threading.Timer(0.05, lambda: stop.append(1))
    th.start()
    n = gs.run(_FakeDevice(), str(out), 0.01, stop)
    th.join()
    assert n >= 1 and len(out.read_text().splitlines()) == n


@pytest.mark.gpu
def test_samples_the_gpu_while_a_kernel_runs(tmp_path, gpu_lib):
    import torch

    from mi355x_sampler import groups, workloads

    out = tmp_path / "gpm.jsonl"
    print("[gpu] gpm sampler: 3 rows at 0.2 s while sampling kernels run", flush=True)
    proc = subprocess.Popen([sys.executable, "-m", "mi355x_sampler.gpm_sampler", "--gpu", "0", "--out", str(out),
                             "--period", "0.2", "--rows", "3"], cwd=str(gs.__file__).rsplit("/mi355x_sampler", 1)[0])
    wl = workloads.thinker_b64().to("cuda:0")
    g = groups.RowGroup(wl.logits, **wl.group_kwargs())
    while proc.poll() is None:
        for _ in range(200):
            groups.launch([g])
        torch.cuda.synchronize()
    assert proc.returncode == 0
    rows = [json.loads(line) for line in out.read_text().splitlines()]
    assert len(rows) >= 2
    for r in rows:
        assert set(r) >= REF_KEYS and r["t1"] > r["t0"]
    assert any(r["sm_util"] is not None or r["dram_bw_util"] is not None for r in rows), rows
    print(f"[gpu] gpm rows: {rows}", flush=True)
