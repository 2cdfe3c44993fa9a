"""Sampled rows/s and HBM-roofline fraction of the fused sampling kernel on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload thinker_b64] [--no-cpu-baseline]
    python bench.py --copy-calibration      # a plain 512 MiB device copy, for scaling rocprof's byte counters

A step is one launch of the fused pipeline + draw over one batch of synthetic
logits resident in HBM (default: the Thinker batch-64 step — vocab 151,748
bf16, heterogeneous top-k / top-p / temperature, repetition 1.1 over
4,096-token histories, a 30%-disallowed bitmask).  The launches rotate over
enough copies of the logits that no copy is still cached (the 256 MB
last-level cache) when it is read again, and are replayed from a HIP graph so
the host never throttles the queue.  Prints one JSON line on stdout.

A step is one launch of the sample kernel (rows whose top-p nucleus is too
large for the published candidates resolve their boundary bin inside it); the
roofline figure divides the step's algorithmic bytes by the step time.  Its
``traffic`` (HBM bytes per step) comes from the rocprof FETCH_SIZE and
WRITE_SIZE counters recorded in profiles/traffic_thinker_b64.json, each scaled
by what the counter reads for the copy of --copy-calibration; it is null when
that file is absent.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "inferrsi-minicpm-o-4.5-npu_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "sampled rows/sec + % HBM roofline, vocab 151,748 bf16, batch 64"
HBM_PEAK_GBS = 8000.0
LLC_BYTES = 256 << 20
COPY_BYTES = 512 << 20
TRAFFIC_FILE = ROOT / "profiles" / "traffic_thinker_b64.json"


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


def cpu_baseline(wl, budget_s: float) -> dict:
    """The oracle (eager torch on the host cores) over whole steps of the same workload, for ~budget_s."""
    import torch

    from oracle import extended_ref
    from tests.parity import oracle_rows

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    rows = oracle_rows(wl)
    done, t0 = 0, time.perf_counter()
    while True:
        extended_ref.sample_rows(rows, with_probs=False)
        done += wl.rows
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {"value": done / el, "unit": "rows/s", "cores": threads, "kind": "port",
            "sample": f"{done // wl.rows} whole {wl.name} step(s) ({done} rows) through the oracle's eager-torch "
                      f"pipeline (processed logits, draw) in {el:.1f} s"}


def copy_calibration() -> int:
    """A device-to-device copy of COPY_BYTES, ten times: reads and writes COPY_BYTES per launch."""
    import torch

    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda:0").random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copied {COPY_BYTES} bytes 10 times")
    return 0


def traffic_per_step(workload: str):
    """HBM bytes per step from the recorded counters (None when there is no record for this workload)."""
    if not TRAFFIC_FILE.exists():
        return None
    rec = json.loads(TRAFFIC_FILE.read_text())
    if rec.get("workload") != workload:
        return None
    fetch = sum(rec["fetch_kib_per_step"].values()) * 1024 * rec["fetch_scale"]
    write = sum(rec["write_kib_per_step"].values()) * 1024 * rec["write_scale"]
    return fetch + write


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4096)
    ap.add_argument("--warmup", type=int, default=256)
    ap.add_argument("--workload", default="thinker_b64")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--copy-calibration", action="store_true")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()
    if args.gpus != 1:
        log(f"bench.py measures one GPU: the sampling path runs on a single MI355X (asked for --gpus {args.gpus}); "
            "rows shard across GPUs without any exchange, so N GPUs would simply run N independent copies")
        return 2

    import torch

    from mi355x_sampler import groups, workloads

    if not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    make = {"thinker_b64": workloads.thinker_b64, "thinker_b8": workloads.thinker_b8,
            "talker_b8": workloads.talker_b8, "talker_b1": workloads.talker_b1}[args.workload]
    wl_cpu = make()
    wl = wl_cpu.to(dev)
    nbytes = wl.algorithmic_bytes()
    rotate = max(2, -(-2 * LLC_BYTES // max(1, wl.logits.numel() * wl.logits.element_size())))
    rotate = min(rotate, 64)
    copies = [wl.logits.clone() for _ in range(rotate)]
    kw = wl.group_kwargs()
    grps = [groups.RowGroup(x, **kw) for x in copies]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for g in grps:  # eager launches: allocate the stream's workspace outside capture
            groups.launch([g])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for g in grps:
                groups.launch([g])
    torch.cuda.synchronize()
    reps_w = max(1, args.warmup // rotate)
    reps = max(1, args.steps // rotate)
    steps = reps * rotate
    log(f"workload {wl.name}: {wl.rows} rows x {wl.vocab} {wl.logits.dtype}, {nbytes} B/step, rotating {rotate} "
        f"copies, {steps} timed launches")
    with torch.cuda.stream(stream):
        for _ in range(reps_w):
            graph.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            graph.replay()
        end.record(stream)
        end.synchronize()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    rows_s = wl.rows / (ms * 1e-3)
    achieved = nbytes / (ms * 1e-3) / 1e9
    tok = grps[0].tokens.cpu().tolist()
    log(f"{ms * 1e3:.2f} us/step  {rows_s / 1e6:.3f} M rows/s  {achieved:.0f} GB/s  ({achieved / HBM_PEAK_GBS:.1%})"
        f"  tokens[0:8]={tok[:8]}")
    out = {
        "metric": METRIC, "value": rows_s, "unit": "rows/s", "n_gpus": 1, "steps": steps, "warmup": reps_w * rotate,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{wl.name}: {wl.rows} rows, vocab {wl.vocab} "
                               f"{str(wl.logits.dtype).replace('torch.', '')} logits, history "
                               f"{wl.history.shape[1]} int32, "
                               f"bitmask {'yes' if wl.allowed is not None else 'no'}, Philox draws",
                   "rows": wl.rows, "vocab": wl.vocab, "bytes_per_step": nbytes, "rotating_copies": rotate,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic_per_step(wl.name)},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(wl_cpu, args.cpu_budget)
        log(f"cpu baseline: {out['cpu_baseline']}")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
