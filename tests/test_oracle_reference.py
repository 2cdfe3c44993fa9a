"""The oracle's restatement of ``engine/talker_sampler.py`` pinned against outside checks.

Mirrors the reference's own CPU tests (``tests/engine/test_talker_sampler.py``)
— transformers' warpers and the HF repetition-penalty restatement — and adds
the golden vectors written from the reference module and brute-force checks
on tiny vocabularies.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch
from transformers.generation.logits_process import TopKLogitsWarper, TopPLogitsWarper

from oracle import talker_sampler_ref as ts
from tests.conftest import golden_case

V, EOS = 6562, 6561
CFG = ts.TalkerSampling()


def hf_penalty(ids: torch.Tensor, scores: torch.Tensor, penalty: float, window: int) -> torch.Tensor:
    """The HF processor's logic (one-hot counting over the window), restated in the reference's tests (:13-27)."""
    if ids.size(1) > window:
        ids = ids.narrow(1, -window, window)
    freq = torch.nn.functional.one_hot(ids, scores.size(1)).sum(1)
    alpha = torch.pow(penalty, freq)
    return torch.where(scores < 0, scores.multiply(alpha), scores.divide(alpha))


def hf_processed(logits, prev, t, cfg=CFG, swap=False):
    """``MiniCPMTTS.generate`` order for one row (reference tests :30-41)."""
    x = logits.float().clone()[None] / cfg.temperature
    if t > 0:
        ids = torch.tensor([prev], dtype=torch.long)
        x = hf_penalty(ids, x, cfg.repetition_penalty, 16)
        warpers = [TopPLogitsWarper(cfg.top_p, min_tokens_to_keep=3), TopKLogitsWarper(cfg.top_k, min_tokens_to_keep=3)]
        for w in (reversed(warpers) if swap else warpers):
            x = w(ids, x)
    if t < cfg.min_new_tokens:
        x[:, EOS] = -torch.inf
    return x[0]


def state_rows(b, t, gen):
    prev = [torch.randint(0, 300, (t,), generator=gen).tolist() for _ in range(b)]
    hist = torch.full((b, 16), ts.PAD, dtype=torch.long)
    for i, p in enumerate(prev):
        tail = p[-16:]
        if tail:
            hist[i, 16 - len(tail):] = torch.tensor(tail)
    return prev, hist


@pytest.mark.parametrize("t", [1, 5, 16, 40, 60])
def test_hf_order_matches_transformers_warpers(t):
    gen = torch.Generator().manual_seed(t)
    logits = torch.randn(6, V, generator=gen) * 3
    prev, hist = state_rows(6, t, gen)
    got = ts.processed_logits(logits, hist, torch.full((6,), t), EOS, CFG)
    for i in range(6):
        want = hf_processed(logits[i], prev[i], t)
        assert torch.equal(torch.isinf(got[i]), torch.isinf(want))
        fin = ~torch.isinf(want)
        assert torch.allclose(got[i][fin], want[fin], rtol=1e-6, atol=1e-6)


def test_swapped_order_is_detected():
    gen = torch.Generator().manual_seed(7)
    logits = torch.randn(1, V, generator=gen) * 0.5
    prev, hist = state_rows(1, 20, gen)
    ours = ts.processed_logits(logits, hist, torch.tensor([20]), EOS, CFG)[0]
    assert not torch.equal(torch.isinf(ours), torch.isinf(hf_processed(logits[0], prev[0], 20, swap=True)))


def test_frame_zero_and_eos_rules():
    logits = torch.randn(2, V)
    got = ts.processed_logits(logits, torch.full((2, 16), ts.PAD), torch.zeros(2, dtype=torch.long), EOS, CFG)
    want = logits / CFG.temperature
    want[:, EOS] = -torch.inf
    assert torch.equal(got, want)
    for t, masked in ((49, True), (50, False)):
        x = ts.processed_logits(torch.zeros(1, V).index_fill_(1, torch.tensor([EOS]), 50.0), torch.full((1, 16), 3),
                                torch.tensor([t]), EOS, CFG)
        assert bool(torch.isinf(x[0, EOS])) == masked
    x = ts.processed_logits(torch.randn(1, V), torch.full((1, 16), 3), torch.tensor([CFG.max_new_tokens - 1]), EOS, CFG)
    assert torch.isfinite(x[0, EOS]) and torch.isinf(x[0, :EOS]).all()


def test_top_filters_match_transformers():
    g = torch.Generator().manual_seed(11)
    for scale in (0.3, 1.0, 3.0):
        x = torch.randn(16, 2000, generator=g) * scale
        for p, mk in ((0.85, 3), (0.5, 1), (0.99, 1)):
            assert torch.equal(ts.top_p_filter(x, p, mk), TopPLogitsWarper(p, min_tokens_to_keep=mk)(None, x.clone()))
        for k, mk in ((25, 3), (1, 1), (2, 3)):
            assert torch.equal(ts.top_k_filter(x, k, mk), TopKLogitsWarper(k, min_tokens_to_keep=mk)(None, x.clone()))


def test_fused_filters_equal_two_pass():
    g = torch.Generator().manual_seed(0)
    for scale in (0.3, 1.0, 3.0, 8.0):
        x = torch.randn(64, V, generator=g) * scale
        a = ts.top_k_filter(ts.top_p_filter(x, 0.85, 3), 25, 3)
        b = ts.top_p_top_k_filter(x, 0.85, 25, 3)
        assert torch.equal(torch.isinf(a), torch.isinf(b))
        c = ts.top_p_filter(ts.top_k_filter(x, 25, 1), 0.85, 1)
        d = ts.top_k_top_p_filter(x, 25, 0.85, 1)
        assert torch.equal(torch.isinf(c), torch.isinf(d))


def brute_support(x: np.ndarray, k: int, p: float, min_keep: int, full_norm: bool) -> set:
    """Enumerate ranks in float64: keep rank j while the mass ranked above it is < p (then clamp)."""
    order = np.argsort(-x, kind="stable")
    vals = x[order][:k]
    z = np.exp(x - x.max()).sum() if full_norm else np.exp(vals - vals.max()).sum()
    probs = np.exp(vals - x.max()) / z
    kept = 0
    acc = 0.0
    for pr in probs:
        if acc < p:
            kept += 1
        acc += pr
    kept = min(max(kept, min(min_keep, k)), k)
    thr = vals[kept - 1]
    return set(np.nonzero(x >= thr)[0].tolist())


def test_fused_filters_brute_force_small_vocab():
    rs = np.random.default_rng(3)
    for trial in range(300):
        n = int(rs.integers(2, 12))
        x = (rs.normal(size=n) * rs.choice([0.2, 1.0, 4.0])).astype(np.float32)
        if trial % 5 == 0:
            x[rs.integers(0, n)] = x[rs.integers(0, n)]  # a tie
        k = int(rs.integers(1, n + 1))
        p = float(rs.choice([0.3, 0.5, 0.8, 0.95]))
        xt = torch.from_numpy(x)[None]
        for mk, fn, full in ((1, lambda: ts.top_k_top_p_filter(xt, k, p, 1), False),
                             (3, lambda: ts.top_p_top_k_filter(xt, p, k, 3), True)):
            got = set(torch.nonzero(~torch.isinf(fn()[0])).flatten().tolist())
            assert got == brute_support(x, min(max(k, mk), n), p, mk, full), (x, k, p, mk)


def test_draw_brute_force():
    rs = np.random.default_rng(4)
    for _ in range(300):
        n = int(rs.integers(1, 9))
        x = rs.normal(size=n).astype(np.float32) * 2
        x[rs.random(n) < 0.3] = -np.inf
        if np.isinf(x).all():
            x[0] = 0.0
        u = np.float32(rs.random())
        e = np.exp(x.astype(np.float64) - x.max())
        cdf = np.cumsum(e / e.sum())
        want = min(int(np.searchsorted(cdf, u * cdf[-1], side="right")), n - 1)
        got = int(ts.draw(torch.from_numpy(x)[None], None, None, uniform_values=torch.tensor([u]))[0])
        if got != want:  # only a float-rounding boundary may differ
            assert abs(cdf[min(got, want)] - u * cdf[-1]) < 1e-6
    assert int(ts.draw(torch.tensor([[0.0, -np.inf]]), None, None, uniform_values=torch.tensor([0.99999994]))[0]) == 0


@pytest.mark.parametrize("name", ["hf_b1_t0", "hf_b6_t5", "hf_b6_t60", "omni_b1_t0", "omni_b6_t40", "hf_c1_w64",
                                  "omni_c1_w64", "hf_c2_w256", "omni_c2_w256"])
def test_processed_and_draw_match_reference_golden(golden_processed, name):
    c = golden_case(golden_processed, name)
    cfg = ts.TalkerSampling(temperature=float(c["temperature"]), top_p=float(c["top_p"]), top_k=int(c["top_k"]),
                            repetition_penalty=float(c["rep"]), window=int(c["w"]), semantics=str(c["semantics"]),
                            rng="counter", min_keep=int(c["min_keep"]))
    x = ts.processed_logits(torch.from_numpy(c["logits"]), torch.from_numpy(c["history"]), torch.from_numpy(c["steps"]),
                            EOS, cfg)
    assert np.array_equal(x.numpy().view(np.int32), c["processed"].view(np.int32))
    tok = ts.draw(x, torch.from_numpy(c["seeds"]), torch.from_numpy(c["steps"]))
    assert np.array_equal(tok.numpy(), c["tokens"])


@pytest.mark.parametrize("name,sem", [("hf", "hf"), ("omni", "omni")])
def test_decode_streams_match_reference_golden(golden_streams, name, sem):
    c = golden_case(golden_streams, name)
    cfg = ts.TalkerSampling(semantics=sem, rng="counter", min_new_tokens=int(c["min_new"]))
    gen = torch.Generator().manual_seed(int(c["gseed"]))
    frames, rows = int(c["frames"]), int(c["rows"])
    logits = torch.randn(frames, rows, V, generator=gen)
    logits[frames - 10, 1, EOS] = 1e4
    assert abs(float(logits.double().sum()) - float(c["logits_sum"])) < 1e-9 * abs(float(c["logits_sum"]))
    st = ts.DecodeState.new([5 + i for i in range(rows)], cfg)
    assert np.array_equal(ts.decode_k(st, logits, EOS, cfg).numpy(), c["tokens"])
    assert np.array_equal(st.history.numpy(), c["history"]) and np.array_equal(st.steps.numpy(), c["steps"])
    assert np.array_equal(st.finished.numpy(), c["finished"])


def test_step_invariants():
    """Batch independence, K-step == steps with EOS freeze, padded rows isolated (reference :99-128)."""
    logits = torch.randn(8, V)
    alone = ts.step(ts.DecodeState.new([1234]), logits[3:4], EOS, CFG)
    batch = ts.step(ts.DecodeState.new([1, 2, 3, 1234, 5, 6, 7, 8]), logits, EOS, CFG)
    assert alone[0] == batch[3]
    gen = torch.Generator().manual_seed(4)
    lg = torch.randn(12, 4, V, generator=gen)
    ref_state = ts.DecodeState.new([1, 2, 3, 4])
    want = torch.stack([ts.step(ref_state, lg[i], EOS, CFG) for i in range(12)])
    s = ts.DecodeState.new([1, 2, 3, 4])
    s.active[2] = False
    noisy = lg.clone()
    noisy[:, 2] = torch.randn(12, V, generator=gen) * 100
    got = torch.stack([ts.step(s, noisy[i], EOS, CFG) for i in range(12)])
    assert torch.equal(got[:, [0, 1, 3]], want[:, [0, 1, 3]]) and (got[:, 2] == ts.PAD).all()


def test_unknown_modes_raise():
    with pytest.raises(ValueError):
        ts.processed_logits(torch.zeros(1, 4), torch.full((1, 2), -1), torch.zeros(1, dtype=torch.long), 3,
                            ts.TalkerSampling(semantics="x"))
    with pytest.raises(ValueError):
        _ = ts.TalkerSampling(rng="bad").uses_native_rng


def test_native_multinomial_delegates_to_torch():
    cfg = ts.TalkerSampling(semantics="omni", min_new_tokens=0)
    logits = torch.randn(3, V, generator=torch.Generator().manual_seed(77))
    seeds = [101, 202, 303]
    gens = [torch.Generator().manual_seed(s) for s in seeds]
    want = torch.stack([torch.multinomial(torch.softmax(ts.processed_logits(
        logits[i:i + 1], torch.full((1, 16), ts.PAD), torch.zeros(1, dtype=torch.long), EOS, cfg)[0], -1), 1,
        generator=gens[i]).reshape(()) for i in range(3)])
    state = ts.DecodeState.new(seeds, cfg)
    state.generators = [torch.Generator().manual_seed(s) for s in seeds]
    assert torch.equal(ts.step(state, logits, EOS, cfg), want)


def test_brute_support_helper_itself_on_a_hand_case():
    """Masses 0.5, 0.3, 0.2 (already normalised logs): p=0.6 keeps two ranks, p=0.5 keeps one."""
    x = np.log(np.array([0.5, 0.3, 0.2], dtype=np.float64)).astype(np.float32)
    assert brute_support(x, 3, 0.6, 1, False) == {0, 1}
    assert brute_support(x, 3, 0.5, 1, False) == {0}
    assert brute_support(x, 3, 0.5, 3, True) == {0, 1, 2}
    assert list(itertools.islice(range(3), 1)) == [0]
