"""Write the reference sampler's golden vectors (run once, in the build container only).

This is the one script that imports the reference module
(``engine/talker_sampler.py`` under ``/root/reference``).  It covers the
functions whose exact output bits nothing else pins: the counter uniform
(``:70-76``), ``processed_logits`` and ``draw`` on realistic Talker inputs
(``:136-172``) and whole ``step`` / ``decode_k`` token streams (``:234-254``).
The fixtures are data only (inputs regenerated from recorded torch generator
seeds, plus expected outputs), stored as ``.npz`` next to this script:

    python tests/golden/make_golden.py

The reference never travels with the repository: GPU-side tests read the
``.npz`` files, never the reference.
"""

from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

REF = Path("/root/reference/engine/talker_sampler.py")
OUT = Path(__file__).resolve().parent
V, EOS = 6562, 6561

SEEDS = [0, 1, 11, 1234, 2**31 - 1, 2**31, 2**32 - 1, 2**32, 2**32 + 5, 2**40 + 5, 2**63 - 1, -1, -(2**63)]
STEPS = [0, 1, 2, 3, 49, 50, 2047, 2**31 - 1, 2**31, 2**32 + 3, 2**62]


def load_reference():
    spec = importlib.util.spec_from_file_location("reference_talker_sampler", REF)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod
    spec.loader.exec_module(mod)
    return mod


def talker_inputs(seed: int, b: int, w: int, t: int, spikes: int = 0):
    """Logits N(0, 3^2) (+ spike tokens at +8), history of the last ``w`` frames over a small alphabet."""
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn(b, V, generator=gen) * 3
    for i in range(b):
        if spikes:
            idx = torch.randint(0, V, (spikes,), generator=gen)
            logits[i, idx] += 8
    hist = torch.full((b, w), -1, dtype=torch.int64)
    n = min(t, w)
    if n:
        hist[:, w - n:] = torch.randint(0, 300, (b, n), generator=gen)
    return logits, hist


def main() -> None:
    ts = load_reference()
    meta = dict(torch_version=torch.__version__, numpy_version=np.__version__, reference=str(REF))

    s, t = np.meshgrid(np.array(SEEDS, dtype=np.int64), np.array(STEPS, dtype=np.int64), indexing="ij")
    u = ts.uniform(torch.from_numpy(s.ravel()), torch.from_numpy(t.ravel())).numpy()
    many = ts.uniform(torch.full((4096,), 9), torch.arange(4096)).numpy()
    np.savez_compressed(OUT / "uniform.npz", seeds=s.ravel(), steps=t.ravel(), u=u, many_seed9=many, **meta)

    cases = {}
    # (name, semantics, rows, window, frame, spikes, generator seed, workload params?)
    for name, sem, b, w, t, spikes, seed, workload in [
        ("hf_b1_t0", "hf", 1, 16, 0, 0, 101, False),
        ("hf_b6_t5", "hf", 6, 16, 5, 0, 102, False),
        ("hf_b6_t60", "hf", 6, 16, 60, 0, 103, False),
        ("omni_b1_t0", "omni", 1, 16, 0, 0, 104, False),
        ("omni_b6_t40", "omni", 6, 16, 40, 0, 105, False),
        ("hf_c1_w64", "hf", 1, 64, 64, 0, 1001, True),
        ("omni_c1_w64", "omni", 1, 64, 64, 0, 1001, True),
        ("hf_c2_w256", "hf", 8, 256, 300, 5, 1002, True),
        ("omni_c2_w256", "omni", 8, 256, 300, 5, 1002, True),
    ]:
        logits, hist = talker_inputs(seed, b, w, t, spikes)
        if workload:  # the Talker sample-step parameters: T 0.8, top-k 20, top-p 0.8, repetition 1.05
            cfg = ts.TalkerSampling(semantics=sem, rng="counter", window=w, temperature=0.8, top_k=20, top_p=0.8,
                                    repetition_penalty=1.05)
        else:
            cfg = ts.TalkerSampling(semantics=sem, rng="counter", window=w)
        steps = torch.full((b,), t, dtype=torch.int64)
        seeds = torch.arange(b, dtype=torch.int64) * 7919 + 1234
        x = ts.processed_logits(logits, hist, steps, EOS, cfg)
        tok = ts.draw(x, seeds, steps)
        cases[name] = dict(seed=seed, b=b, w=w, t=t, spikes=spikes, semantics=sem, temperature=cfg.temperature,
                           top_k=cfg.top_k, top_p=cfg.top_p, rep=cfg.repetition_penalty, min_keep=cfg.min_keep,
                           logits=logits.numpy(), history=hist.numpy(), steps=steps.numpy(), seeds=seeds.numpy(),
                           processed=x.numpy(), tokens=tok.numpy())
    flat = {}
    for name, c in cases.items():
        for k, v in c.items():
            flat[f"{name}.{k}"] = np.asarray(v)
    np.savez_compressed(OUT / "processed.npz", names=np.array(list(cases)), **flat, **meta)

    # whole decode streams: 70 frames x 4 rows (hf) and 40 frames x 3 rows (omni counter), one EOS spike
    streams = {}
    for name, sem, frames, rows, gseed in [("hf", "hf", 70, 4, 3), ("omni", "omni", 40, 3, 79)]:
        cfg = ts.TalkerSampling(semantics=sem, rng="counter", min_new_tokens=10 if sem == "omni" else 50)
        gen = torch.Generator().manual_seed(gseed)
        logits = torch.randn(frames, rows, V, generator=gen)
        logits[frames - 10, 1, EOS] = 1e4
        st = ts.DecodeState.new([5 + i for i in range(rows)], cfg)
        toks = ts.decode_k(st, logits, EOS, cfg)
        streams[name] = dict(gseed=gseed, frames=frames, rows=rows, min_new=cfg.min_new_tokens,
                             logits_sum=float(logits.double().sum()), tokens=toks.numpy(),
                             history=st.history.numpy(), steps=st.steps.numpy(), finished=st.finished.numpy())
    flat = {f"{n}.{k}": np.asarray(v) for n, c in streams.items() for k, v in c.items()}
    np.savez_compressed(OUT / "streams.npz", **flat, **meta)
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))


if __name__ == "__main__":
    main()
