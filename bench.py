"""Sampled rows/s and HBM-roofline fraction of the fused sampling kernel on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload thinker_b64] [--no-cpu-baseline]
    python bench.py --all-configs [--configs-out profiles/bench_configs.jsonl]   # one line per workload
    python bench.py --copy-calibration      # a plain 512 MiB device copy, for scaling rocprof's byte counters

A step is one launch of the fused pipeline + draw over one batch of synthetic inputs resident in HBM (default:
the Thinker batch-64 step — vocab 151,748 bf16, heterogeneous top-k / top-p / temperature, repetition 1.1 over
4,096-token histories, a 30%-disallowed bitmask).  The launches rotate over enough copies of every per-step input
(logits, histories, bitmasks) that no copy is still in the 256 MB last-level cache when it is read again, and are
replayed from HIP graphs so the host never throttles the queue.  Exactly W untimed and K timed steps run; the
timed region is bracketed by device synchronisations and measured with HIP events on the launch stream.  Prints
one JSON line on stdout (the default workload); ``--all-configs`` also writes one line per workload.

The roofline figure divides the step's algorithmic bytes (logits once, the packed bitmask once, the history ids
once) by the step time.  Its ``traffic`` (HBM bytes per step) comes from the rocprof FETCH_SIZE and WRITE_SIZE
counters recorded in profiles/traffic_<workload>.json, each scaled by what the counter reads for the copy of
--copy-calibration; it is null when there is no such record.  The CPU baseline runs the oracle (the reference
pipeline in eager torch, row by row: the reference takes one parameter set per call, and these rows each carry
their own) on the host cores, once with one thread and once with every core.
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
WORKLOADS = ("talker_b1", "talker_b8", "thinker_b8", "thinker_b8_greedy", "thinker_b64", "mixed")


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


def make_workloads(name: str) -> list:
    from mi355x_sampler import workloads as W

    if name == "mixed":
        return list(W.mixed())
    if name == "thinker_b8_greedy":
        return [W.thinker_b8(greedy=True)]
    return [{"talker_b1": W.talker_b1, "talker_b8": W.talker_b8, "thinker_b8": W.thinker_b8,
             "thinker_b64": W.thinker_b64}[name]()]


def describe(name: str, wls: list) -> str:
    parts = []
    for w in wls:
        parts.append(f"{w.rows} rows x vocab {w.vocab} {str(w.logits.dtype).replace('torch.', '')} logits, "
                     f"{w.semantics} order, history {w.history.shape[1]} int32, "
                     f"bitmask {'yes' if w.allowed is not None else 'no'}, {w.rng} draws")
    return f"{name}: " + " + ".join(parts)


def cpu_baseline(wls: list, budget_s: float) -> dict:
    """The oracle over whole steps of the same workload for ~budget_s per leg: one thread, then every core."""
    import torch

    from oracle import extended_ref
    from tests.parity import oracle_rows

    rows = [oracle_rows(w) for w in wls]
    n_rows = sum(w.rows for w in wls)
    legs = {}
    cores = len(os.sched_getaffinity(0))
    for threads in (1, cores):
        torch.set_num_threads(threads)
        done, t0 = 0, time.perf_counter()
        while True:
            for r in rows:
                extended_ref.sample_rows(r, with_probs=False)
            done += n_rows
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
        legs[threads] = (done / el, done, el)
    v1, vn = legs[1], legs[cores]
    return {"value": vn[0], "unit": "rows/s", "cores": cores, "kind": "port", "value_1_thread": v1[0],
            "sample": f"whole steps through the oracle's eager-torch pipeline (processed logits, draw), row by row: "
                      f"{vn[1]} rows in {vn[2]:.1f} s on {cores} threads; {v1[1]} rows in {v1[2]:.1f} s on 1 thread"}


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
    f = ROOT / "profiles" / f"traffic_{workload}.json"
    if not f.exists():
        return None
    rec = json.loads(f.read_text())
    if rec.get("workload") != workload:
        return None
    fetch = sum(rec["fetch_kib_per_step"].values()) * 1024 * rec["fetch_scale"]
    write = sum(rec["write_kib_per_step"].values()) * 1024 * rec["write_scale"]
    return fetch + write


def measure(name: str, steps: int, warmup: int, dev) -> dict:
    """Times exactly `steps` launches after `warmup` untimed ones; returns the step time and workload facts."""
    import torch

    from mi355x_sampler import groups

    wls_cpu = make_workloads(name)
    wls = [w.to(dev) for w in wls_cpu]
    nbytes = sum(w.algorithmic_bytes() for w in wls)
    per_copy = sum(w.logits.numel() * w.logits.element_size() + w.history.numel() * w.history.element_size()
                   + (w.allowed.numel() * 4 if w.allowed is not None else 0) for w in wls)
    rotate = min(64, max(2, -(-2 * LLC_BYTES // per_copy)))
    sets = []
    for _ in range(rotate):
        grs = []
        for w in wls:
            kw = w.group_kwargs()
            kw["history"] = w.history.clone()
            if w.allowed is not None:
                kw["allowed"] = w.allowed.clone()
            grs.append(groups.RowGroup(w.logits.clone(), **kw))
        sets.append(grs)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())

    def capture(n: int):
        if n == 0:
            return None
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n):
                groups.launch(sets[i % rotate])
        return g

    with torch.cuda.stream(stream):
        for grs in sets:  # eager launches: the stream's workspace is allocated outside capture
            groups.launch(grs)
        torch.cuda.synchronize()
        full = capture(rotate)
        tail_t = capture(steps % rotate)
        tail_w = capture(warmup % rotate)
    torch.cuda.synchronize()

    def run(n: int, tail) -> None:
        for _ in range(n // rotate):
            full.replay()
        if tail is not None:
            tail.replay()

    with torch.cuda.stream(stream):
        run(warmup, tail_w)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        run(steps, tail_t)
        end.record(stream)
        end.synchronize()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    rows = sum(w.rows for w in wls)
    return {"name": name, "ms": ms, "rows": rows, "bytes": nbytes, "rotate": rotate, "wls_cpu": wls_cpu,
            "tokens": sets[0][0].tokens.cpu().tolist()[:8]}


def line(m: dict, steps: int, warmup: int) -> dict:
    ms = m["ms"]
    rows_s = m["rows"] / (ms * 1e-3)
    achieved = m["bytes"] / (ms * 1e-3) / 1e9
    wls = m["wls_cpu"]
    return {
        "metric": METRIC, "value": rows_s, "unit": "rows/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": describe(m["name"], wls), "rows": m["rows"], "vocab": max(w.vocab for w in wls),
                   "bytes_per_step": m["bytes"], "rotating_copies": m["rotate"], "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic_per_step(m["name"])},
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2048)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--workload", default="thinker_b64", choices=WORKLOADS)
    ap.add_argument("--all-configs", action="store_true", help="also time every workload and write one line each")
    ap.add_argument("--configs-out", default=str(ROOT / "profiles" / "bench_configs.jsonl"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=8.0, help="seconds per CPU-baseline leg")
    ap.add_argument("--copy-calibration", action="store_true")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()
    if args.gpus != 1:
        log(f"bench.py measures one GPU: the sampling path runs on a single MI355X (asked for --gpus {args.gpus}); "
            "rows shard across GPUs without any exchange, so N GPUs would simply run N independent copies")
        return 2
    if args.steps < 1 or args.warmup < 0:
        log("--steps must be >= 1 and --warmup >= 0")
        return 2

    import torch

    if not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    others = [n for n in WORKLOADS if n != args.workload] if args.all_configs else []
    extra = []
    for name in others:
        m = measure(name, args.steps, args.warmup, dev)
        extra.append(line(m, args.steps, args.warmup))
        log(f"{name}: {m['ms'] * 1e3:.2f} us/step ({extra[-1]['roofline']['frac']:.1%} of HBM peak)")
    m = measure(args.workload, args.steps, args.warmup, dev)
    out = line(m, args.steps, args.warmup)
    log(f"{args.workload}: {m['ms'] * 1e3:.2f} us/step  {out['value'] / 1e6:.3f} M rows/s  "
        f"{out['roofline']['achieved']:.0f} GB/s ({out['roofline']['frac']:.1%})  tokens[0:8]={m['tokens']}")
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(m["wls_cpu"], args.cpu_budget)
        log(f"cpu baseline: {out['cpu_baseline']}")
    if args.all_configs:
        with open(args.configs_out, "w") as f:
            for rec in extra + [out]:
                f.write(json.dumps(rec) + "\n")
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
