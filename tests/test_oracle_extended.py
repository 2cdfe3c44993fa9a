"""The per-row extended oracle pinned against the reference restatement and closed forms."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import extended_ref as ext
from oracle import talker_sampler_ref as ts
from tests.parity import oracle_rows

V, EOS = 6562, 6561


def uniform_rows(sem: str, t: int, b: int = 4, seed: int = 0) -> tuple[ext.Rows, ts.TalkerSampling, torch.Tensor]:
    cfg = ts.TalkerSampling(semantics=sem)
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(b, V, generator=g) * 3
    hist = torch.randint(0, 300, (b, 16), generator=g)
    steps = torch.full((b,), t, dtype=torch.int64)
    full = lambda v, dt: torch.full((b,), v, dtype=dt)  # noqa: E731
    rows = ext.Rows(logits=logits, temperature=full(cfg.temperature, torch.float32),
                    top_k=full(cfg.top_k, torch.int32), top_p=full(cfg.top_p, torch.float32),
                    repetition=full(cfg.repetition_penalty, torch.float32), presence=full(0.0, torch.float32),
                    frequency=full(0.0, torch.float32), history=hist, steps=steps, seeds=torch.arange(b) + 5,
                    eos=EOS, min_new_tokens=cfg.min_new_tokens, max_new_tokens=cfg.max_new_tokens,
                    semantics=sem, min_keep=cfg.min_keep if sem == "hf" else 1, rng="counter",
                    top_k_zero_disables=False, top_p_one_disables=False, alpha="torch")
    return rows, cfg, logits


@pytest.mark.parametrize("sem", ["hf", "omni"])
@pytest.mark.parametrize("t", [0, 1, 30, 60, 2047])
def test_uniform_parameters_reduce_to_the_reference(sem, t):
    rows, cfg, logits = uniform_rows(sem, t, seed=t)
    want = ts.processed_logits(logits, rows.history, rows.steps, EOS, cfg)
    out = ext.sample_rows(rows)
    assert torch.equal(out["processed"], want)
    assert torch.equal(out["tokens"], ts.draw(want, rows.seeds, rows.steps))


def test_presence_frequency_closed_form():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(50, generator=g) * 3
    hist = torch.tensor([3, 3, 3, 7, 9, 9, -1, 60])
    counts = ext.history_counts(hist, 50)
    got = ext.penalties(x, counts, 1.0, 0.5, 0.2, "exact")
    want = x.clone()
    for tok in range(50):
        n = sum(1 for h in hist.tolist() if h == tok)
        if n:
            want[tok] = (want[tok] - np.float32(0.2) * np.float32(n)) - np.float32(0.5)
    assert torch.equal(got, want)
    assert counts[3] == 3 and counts[9] == 2 and counts.sum() == 6  # PAD and ids >= V (60) do not count


def test_exact_alpha_is_correctly_rounded_and_matches_torch_for_small_counts():
    n = torch.arange(0, 28, dtype=torch.float32)
    for rep in (1.05, 1.1, 1.3, 0.9, 2.0):
        a = ext.exact_alpha(rep, n)
        assert torch.equal(a, torch.pow(torch.full_like(n, rep), n))
        big = torch.arange(0, 2000, dtype=torch.float32)
        ex = np.power(np.float64(np.float32(rep)), big.double().numpy())
        with np.errstate(over="ignore"):
            assert np.array_equal(ext.exact_alpha(rep, big).numpy(), ex.astype(np.float32))


def test_mask_packing_round_trip_and_application():
    g = torch.Generator().manual_seed(2)
    allowed = torch.rand(3, 70, generator=g) > 0.4
    words = ext.pack_mask(allowed)
    assert words.shape == (3, 3) and torch.equal(ext.unpack_mask(words, 70), allowed)
    assert int(ext.pack_mask(torch.tensor([[True] + [False] * 31]))[0, 0]) == 1
    assert int(ext.pack_mask(torch.tensor([[False] * 31 + [True]]))[0, 0]) == -(2**31)  # bit 31 set


def test_sentinels():
    g = torch.Generator().manual_seed(3)
    b = 2
    logits = torch.randn(b, 500, generator=g)
    full = lambda v, dt: torch.full((b,), v, dtype=dt)  # noqa: E731
    rows = ext.Rows(logits=logits, temperature=full(1.0, torch.float32), top_k=full(0, torch.int32),
                    top_p=full(1.0, torch.float32), repetition=full(1.0, torch.float32),
                    presence=full(0.0, torch.float32), frequency=full(0.0, torch.float32), seeds=torch.arange(b))
    out = ext.sample_rows(rows)
    assert torch.isfinite(out["processed"]).all()  # top_k 0 and top_p 1 disable both filters
    rows.top_k_zero_disables = False
    out = ext.sample_rows(rows)
    assert (torch.isfinite(out["processed"]).sum(-1) == 1).all()  # reference rule: k = max(0, min_keep) = 1
    rows.temperature = full(0.0, torch.float32)
    assert torch.equal(ext.sample_rows(rows)["tokens"], torch.argmax(logits, -1))


def test_workload_generators_are_deterministic():
    from mi355x_sampler import workloads as W

    a, b = W.thinker_b64(), W.thinker_b64()
    assert torch.equal(a.logits, b.logits) and torch.equal(a.allowed, b.allowed)
    assert a.algorithmic_bytes() == 21_686_528
    allowed = ext.unpack_mask(a.allowed, a.vocab)
    assert allowed.any(dim=1).all() and abs(float((~allowed).float().mean()) - 0.3) < 0.01
    assert W.talker_b8().algorithmic_bytes() == 224_768
    assert W.talker_b1().algorithmic_bytes() == 26_504
    assert W.thinker_b8().algorithmic_bytes() == 2_493_504


def test_oracle_rows_adapter_runs_a_small_workload():
    from mi355x_sampler import workloads as W

    wl = W.talker_b8("omni")
    out = ext.sample_rows(oracle_rows(wl))
    assert out["tokens"].shape == (8,) and (out["tokens"] >= 0).all()
    assert not torch.isfinite(out["processed"][:, V - 2:]).any()  # masked by the bitmask
