"""HIP path vs the oracle (and the reference's golden vectors), through the C-ABI library.

Every test runs the kernel on ``cuda:0`` and checks it against the CPU oracle
on the same seeded inputs: tokens bit-exact (a difference is accepted only
where the float64 CDF or top-p mass sits within the two computations' own
rounding of the decision point, measured per row, see ``tests/parity.py``;
the workload tests allow none), processed logits bit-exact wherever both are
finite, filtered probabilities within 1e-5 relative (fp32) / 2e-3 (bf16).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mi355x_sampler import _lib
from mi355x_sampler import groups as G
from mi355x_sampler import talker_sampler as hs
from mi355x_sampler import workloads as W
from oracle import extended_ref as ext
from oracle import rng_ref
from oracle import talker_sampler_ref as ts
from tests.conftest import golden_case
from tests.parity import compare_group, oracle_rows, token_at_boundary

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
V, EOS = 6562, 6561


@pytest.fixture(scope="module", autouse=True)
def _gpu(gpu_lib):
    torch.cuda.set_device(0)
    yield


def run(wl, **kw):
    d = wl.to(DEV)
    g = G.RowGroup(d.logits, **d.group_kwargs(), processed=True, probs=True, **kw)
    G.launch([g])
    torch.cuda.synchronize()
    return g


WORKLOADS = [
    ("talker_b1_hf", lambda: W.talker_b1("hf")),
    ("talker_b1_omni", lambda: W.talker_b1("omni")),
    ("talker_b8_hf", lambda: W.talker_b8("hf")),
    ("talker_b8_omni", lambda: W.talker_b8("omni")),
    ("thinker_b8", lambda: W.thinker_b8()),
    ("thinker_b8_greedy", lambda: W.thinker_b8(greedy=True)),
    ("thinker_b64", lambda: W.thinker_b64()),
]


@pytest.mark.parametrize("name,make", WORKLOADS, ids=[n for n, _ in WORKLOADS])
def test_workload_matches_oracle(name, make):
    wl = make()
    print(f"[gpu] workload {name}: rows={wl.rows} vocab={wl.vocab} dtype={wl.logits.dtype}", flush=True)
    _lib.reset_path_counters(DEV)
    g = run(wl)
    paths = _lib.path_counters(DEV)
    rows = oracle_rows(wl)
    ref = ext.sample_rows(rows)
    stats = compare_group(name, g.tokens, g.processed, g.probs, ref, rows,
                          prob_rtol=1e-5 if wl.logits.dtype == torch.float32 else 2e-3)
    print(f"[gpu] {name}: {stats} paths {paths}", flush=True)
    # on these seeds no row may need the rounding allowance: every token and support is exact
    assert stats["token_boundary"] == 0 and stats["support_boundary"] == 0, f"{name}: {stats['boundary_rows']}"
    assert paths["stream"] == 0 and sum(paths.values()) == wl.rows


STREAMING = [
    ("talker_b8_hf", lambda: W.talker_b8("hf")),
    ("thinker_b8", lambda: W.thinker_b8()),
    ("thinker_b8_greedy", lambda: W.thinker_b8(greedy=True)),
]


@pytest.mark.parametrize("name,make", STREAMING, ids=[n for n, _ in STREAMING])
def test_streaming_finalise_matches_oracle(name, make):
    """The finaliser a row takes when its slices did not share an XCD: from the logits alone."""
    wl = make()
    print(f"[gpu] streaming finalise {name}", flush=True)
    g = run(wl, finalize_streaming=True)
    rows = oracle_rows(wl)
    ref = ext.sample_rows(rows)
    stats = compare_group(name, g.tokens, g.processed, g.probs, ref, rows,
                          prob_rtol=1e-5 if wl.logits.dtype == torch.float32 else 2e-3)
    print(f"[gpu] streaming {name}: {stats}", flush=True)
    assert stats["token_boundary"] == 0 and stats["support_boundary"] == 0, f"{name}: {stats['boundary_rows']}"


@pytest.mark.parametrize("rows", [1, 3, 5, 9, 13])
def test_row_counts_that_do_not_fill_xcds_evenly(rows):
    """Batches whose slices do not divide evenly over the eight XCDs: every row still sees only its own slices."""
    print(f"[gpu] uneven rows={rows}", flush=True)
    x = torch.randn(rows, W.THINKER_V, generator=torch.Generator().manual_seed(77 + rows)).to(DEV)
    for _ in range(2):  # twice: a stale slot from the first launch must not leak into the second
        got = G.greedy(x)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), torch.argmax(x.cpu(), dim=-1))
    g = G.RowGroup(x, temperature=0.9, top_k=50, top_p=0.9, seeds=torch.full((rows,), 5, device=DEV),
                   steps=torch.zeros(rows, dtype=torch.int64, device=DEV), processed=True, probs=True)
    G.launch([g])
    torch.cuda.synchronize()
    one = lambda v, dt=torch.float32: torch.full((rows,), v, dtype=dt)  # noqa: E731
    ref_rows = ext.Rows(logits=x.cpu(), temperature=one(0.9), top_k=one(50, torch.int32), top_p=one(0.9),
                        repetition=one(1.0), presence=one(0.0), frequency=one(0.0), seeds=one(5, torch.int64),
                        steps=one(0, torch.int64))
    compare_group(f"uneven{rows}", g.tokens, g.processed, g.probs, ext.sample_rows(ref_rows), ref_rows, prob_rtol=1e-5)


@pytest.mark.parametrize("semantics", ["omni", "hf"])
def test_large_nucleus_second_pass(semantics):
    """Top-p rows without top-k whose nucleus is far too large for the first pass's candidates."""
    print(f"[gpu] large nucleus {semantics}", flush=True)
    gen = torch.Generator().manual_seed(91)
    rows, v = 6, W.THINKER_V
    x = (torch.randn(rows, v, generator=gen) * 2.5).to(torch.bfloat16)
    hist = torch.randint(0, v, (rows, 256), generator=gen, dtype=torch.int64).to(torch.int32)
    one = lambda val, dt=torch.float32: torch.full((rows,), val, dtype=dt)  # noqa: E731
    top_p = torch.tensor([0.5, 0.7, 0.9, 0.95, 0.99, 0.8])
    ref_rows = ext.Rows(logits=x, temperature=one(1.0), top_k=one(0, torch.int32), top_p=top_p, repetition=one(1.1),
                        presence=one(0.0), frequency=one(0.0), history=hist, seeds=one(3, torch.int64),
                        steps=one(1, torch.int64), eos=5, min_new_tokens=4, semantics=semantics,
                        min_keep=3 if semantics == "hf" else 1)
    g = G.RowGroup(x.to(DEV), temperature=1.0, top_k=0, top_p=top_p.to(DEV), repetition=1.1, history=hist.to(DEV),
                   seeds=one(3, torch.int64).to(DEV), steps=one(1, torch.int64).to(DEV), eos=5, min_new_tokens=4,
                   semantics=semantics, min_keep=3 if semantics == "hf" else 1, processed=True, probs=True)
    _lib.reset_path_counters(DEV)
    G.launch([g])
    torch.cuda.synchronize()
    paths = _lib.path_counters(DEV)
    print(f"[gpu] large nucleus {semantics} paths {paths}", flush=True)
    compare_group(f"large_nucleus_{semantics}", g.tokens, g.processed, g.probs, ext.sample_rows(ref_rows), ref_rows,
                  prob_rtol=2e-3)
    # the wide rows are settled from the slices' value histograms, none by streaming the row
    assert paths["stream"] == 0 and paths["histogram"] >= 3 and sum(paths.values()) == rows
    assert _lib.wait_failures(DEV) == 0


def test_boundary_bin_and_candidate_rows_across_launches():
    """Launches on one workspace that alternate between top-p rows needing their boundary bin (wide nuclei) and
    rows the first pass's candidates settle (sharp rows): the arrival and decision words must start every launch
    cleared, whichever way the previous launch released its held slices."""
    print("[gpu] boundary bin across launches", flush=True)
    gen = torch.Generator().manual_seed(23)
    rows, v = 5, W.THINKER_V
    wide = (torch.randn(rows, v, generator=gen) * 2.5).to(torch.bfloat16)
    sharp = (torch.randn(rows, v, generator=gen) * 9.0).to(torch.bfloat16)
    hist = torch.randint(0, v, (rows, 128), generator=gen, dtype=torch.int64).to(torch.int32)
    one = lambda val, dt=torch.float32: torch.full((rows,), val, dtype=dt)  # noqa: E731
    x_dev, p_dev = wide.to(DEV), one(0.9).to(DEV)
    steps_dev = one(1, torch.int64).to(DEV)
    g = G.RowGroup(x_dev, temperature=1.0, top_k=0, top_p=p_dev, repetition=1.05, history=hist.to(DEV),
                   seeds=torch.arange(rows, dtype=torch.int64).to(DEV), steps=steps_dev, eos=5, min_new_tokens=2,
                   semantics="hf", min_keep=3, processed=True, probs=True)
    plan = [(wide, 0.95), (sharp, 0.5), (wide, 0.9), (wide, 0.99), (sharp, 0.8), (wide, 0.7)]
    for it, (x, tp) in enumerate(plan):
        x_dev.copy_(x.to(DEV))
        p_dev.fill_(tp)
        steps_dev.fill_(it + 1)
        G.launch([g])
        torch.cuda.synchronize()
        ref_rows = ext.Rows(logits=x, temperature=one(1.0), top_k=one(0, torch.int32), top_p=one(tp),
                            repetition=one(1.05), presence=one(0.0), frequency=one(0.0), history=hist,
                            seeds=torch.arange(rows, dtype=torch.int64), steps=one(it + 1, torch.int64), eos=5,
                            min_new_tokens=2, semantics="hf", min_keep=3)
        compare_group(f"across_launches_{it}", g.tokens, g.processed, g.probs, ext.sample_rows(ref_rows), ref_rows,
                      prob_rtol=2e-3)


@pytest.mark.parametrize("case", ["tiny_values", "mostly_tiny", "one_slice"])
def test_histogram_rows_with_values_at_zero(case):
    """Top-p rows without top-k settled from value counts, with values crowding zero: exact +0 and -0, magnitudes
    below 2^-15 (weighed one by one by the slices), rows whose values are mostly in the lumps next to zero (a cut
    inside a lump is streamed instead), and a vocabulary of one slice (the finaliser draws itself)."""
    print(f"[gpu] histogram rows at zero {case}", flush=True)
    gen = torch.Generator().manual_seed(47)
    rows = 6
    v = 20000 if case == "one_slice" else W.THINKER_V
    x = torch.randn(rows, v, generator=gen) * (0.008 if case == "mostly_tiny" else 0.3)
    x[torch.rand(rows, v, generator=gen) < 0.01] = 0.0
    x[:, 1::997] = -0.0
    x[:, 3::1009] = 1e-6
    x[:, 5::1013] = -2e-6
    x = x.to(torch.bfloat16)
    hist = torch.randint(0, v, (rows, 256), generator=gen, dtype=torch.int64).to(torch.int32)
    one = lambda val, dt=torch.float32: torch.full((rows,), val, dtype=dt)  # noqa: E731
    temps = torch.tensor([0.05, 0.1, 0.3, 1.0, 0.02, 0.5])
    top_p = torch.tensor([0.9, 0.5, 0.95, 0.8, 0.7, 0.99])
    ref_rows = ext.Rows(logits=x, temperature=temps, top_k=one(0, torch.int32), top_p=top_p, repetition=one(1.1),
                        presence=one(0.0), frequency=one(0.0), history=hist, seeds=one(7, torch.int64),
                        steps=one(2, torch.int64))
    g = G.RowGroup(x.to(DEV), temperature=temps.to(DEV), top_k=0, top_p=top_p.to(DEV), repetition=1.1,
                   history=hist.to(DEV), seeds=one(7, torch.int64).to(DEV), steps=one(2, torch.int64).to(DEV),
                   processed=True, probs=True)
    _lib.reset_path_counters(DEV)
    G.launch([g])
    torch.cuda.synchronize()
    paths = _lib.path_counters(DEV)
    print(f"[gpu] histogram rows at zero {case} paths {paths}", flush=True)
    compare_group(f"at_zero_{case}", g.tokens, g.processed, g.probs, ext.sample_rows(ref_rows), ref_rows,
                  prob_rtol=2e-3)
    assert _lib.wait_failures(DEV) == 0
    if case == "mostly_tiny":
        assert paths["histogram"] + paths["stream"] == rows
    else:
        assert paths["histogram"] == rows and paths["stream"] == 0


def test_histories_with_more_distinct_ids_than_a_slice_lists():
    """A 60,000-id history holding 40% of the vocabulary: every slice meets more distinct history ids than its list
    of penalised values holds (2,048), for a greedy row, an unfiltered row, a top-k row and a top-p row.  The history
    ids carry the largest logits, so a value left unpenalised would win; every such row is streamed instead."""
    print("[gpu] overflowing specials", flush=True)
    gen = torch.Generator().manual_seed(61)
    rows, v = 4, W.THINKER_V
    hist = torch.randperm(v, generator=gen)[:60000].to(torch.int32).repeat(rows, 1)
    x = torch.randn(rows, v, generator=gen) * 2.0
    x[:, hist[0].long()] += 6.0
    x = x.to(torch.bfloat16)
    temps = torch.tensor([0.0, 1.0, 1.0, 1.0])
    top_k = torch.tensor([0, 0, 50, 0], dtype=torch.int32)
    top_p = torch.tensor([1.0, 1.0, 1.0, 0.9])
    one = lambda val, dt=torch.float32: torch.full((rows,), val, dtype=dt)  # noqa: E731
    ref_rows = ext.Rows(logits=x, temperature=temps, top_k=top_k, top_p=top_p, repetition=one(1.5),
                        presence=one(1.0), frequency=one(0.25), history=hist, seeds=one(11, torch.int64),
                        steps=one(3, torch.int64))
    g = G.RowGroup(x.to(DEV), temperature=temps.to(DEV), top_k=top_k.to(DEV), top_p=top_p.to(DEV), repetition=1.5,
                   presence=1.0, frequency=0.25, history=hist.to(DEV), seeds=one(11, torch.int64).to(DEV),
                   steps=one(3, torch.int64).to(DEV), processed=True, probs=True)
    _lib.reset_path_counters(DEV)
    G.launch([g])
    torch.cuda.synchronize()
    paths = _lib.path_counters(DEV)
    print(f"[gpu] overflowing specials paths {paths}", flush=True)
    compare_group("overflowing_specials", g.tokens, g.processed, g.probs, ext.sample_rows(ref_rows), ref_rows,
                  prob_rtol=2e-3)
    assert paths["stream"] == rows


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_greedy_ties_take_the_first_index(dtype):
    """Greedy rows whose maximum is tied: inside one 16-byte chunk, across chunks and slices, against a masked
    element, and between a penalised history id and a plain element (either one first); the first index wins."""
    print(f"[gpu] greedy ties {dtype}", flush=True)
    v = W.THINKER_V if dtype == "bf16" else V
    rows = 7
    gen = torch.Generator().manual_seed(83)
    x = torch.randn(rows, v, generator=gen) * 0.5
    p, q = 4096, v - 9
    x[0] = 0.0
    x[1, [p, p + 3, q]] = 5.0
    x[2, [p, p + 1]] = 5.0
    x[3, [q, p + 8]] = 5.0
    x[4, [v - 1, q]] = 5.0
    x[5, p], x[5, p + 2] = 6.25, 5.0  # 6.25 / 1.25 = 5 exactly: the history id ties with the later plain element
    x[6, p], x[6, p + 2] = 5.0, 6.25  # ... and with the earlier one
    x = x.to(torch.bfloat16) if dtype == "bf16" else x
    allowed = torch.ones(rows, v, dtype=torch.bool)
    allowed[2, p] = False
    hist = torch.full((rows, 4), -1, dtype=torch.int32)
    hist[5, 0], hist[6, 0] = p, p + 2
    one = lambda val, dt=torch.float32: torch.full((rows,), val, dtype=dt)  # noqa: E731
    words = W.pack_allowed(allowed)
    ref_rows = ext.Rows(logits=x, temperature=one(0.0), top_k=one(0, torch.int32), top_p=one(1.0),
                        repetition=one(1.25), presence=one(0.0), frequency=one(0.0), history=hist, mask=words,
                        seeds=one(1, torch.int64), steps=one(1, torch.int64))
    g = G.RowGroup(x.to(DEV), temperature=0.0, repetition=1.25, history=hist.to(DEV), allowed=words.to(DEV),
                   seeds=one(1, torch.int64).to(DEV), steps=one(1, torch.int64).to(DEV), processed=True, probs=True)
    G.launch([g])
    torch.cuda.synchronize()
    ref = ext.sample_rows(ref_rows)
    compare_group(f"greedy_ties_{dtype}", g.tokens, g.processed, g.probs, ref, ref_rows, prob_rtol=2e-3)
    assert g.tokens.cpu().tolist() == [0, p, p + 1, p + 8, q, p, p]


def test_thinker_greedy_is_first_argmax_at_full_size():
    wl = W.thinker_b64().to(DEV)
    x = wl.logits.clone()
    x[3, 100] = x[3].max()  # a tie: the first index wins
    x[3, 7] = x[3].max()
    got = G.greedy(x)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.argmax(x.float().cpu(), dim=-1))
    x32 = torch.randn(5, W.THINKER_V, device=DEV)
    assert torch.equal(G.greedy(x32).cpu(), torch.argmax(x32.cpu(), dim=-1))


def test_counter_uniform_matches_reference_golden(golden_uniform):
    g = golden_uniform
    u = hs.uniform(torch.from_numpy(g["seeds"]).to(DEV), torch.from_numpy(g["steps"]).to(DEV)).cpu().numpy()
    assert np.array_equal(u.view(np.int32), g["u"].view(np.int32))
    many = hs.uniform(torch.full((4096,), 9, device=DEV), torch.arange(4096, device=DEV)).cpu().numpy()
    assert np.array_equal(many, g["many_seed9"])


def test_philox_uniform_matches_oracle():
    rs = np.random.default_rng(2)
    s = rs.integers(-(2**63), 2**63 - 1, size=2048, dtype=np.int64)
    t = rs.integers(0, 2**40, size=2048, dtype=np.int64)
    r = rs.integers(0, 2**20, size=2048, dtype=np.int64)
    got = hs.philox_uniform(torch.from_numpy(s).to(DEV), torch.from_numpy(t).to(DEV), torch.from_numpy(r).to(DEV))
    assert np.array_equal(got.cpu().numpy(), rng_ref.philox_uniform(s, t, r))


@pytest.mark.parametrize("name", ["hf_b1_t0", "hf_b6_t5", "hf_b6_t60", "omni_b1_t0", "omni_b6_t40", "hf_c1_w64",
                                  "omni_c1_w64", "hf_c2_w256", "omni_c2_w256"])
def test_processed_and_draw_match_reference_golden(golden_processed, name):
    c = golden_case(golden_processed, name)
    cfg = hs.TalkerSampling(temperature=float(c["temperature"]), top_p=float(c["top_p"]), top_k=int(c["top_k"]),
                            repetition_penalty=float(c["rep"]), window=int(c["w"]), semantics=str(c["semantics"]),
                            rng="counter", min_keep=int(c["min_keep"]))
    logits = torch.from_numpy(c["logits"]).to(DEV)
    hist = torch.from_numpy(c["history"]).to(DEV)
    steps = torch.from_numpy(c["steps"]).to(DEV)
    x = hs.processed_logits(logits, hist, steps, EOS, cfg).cpu()
    want = torch.from_numpy(c["processed"])
    if not torch.equal(torch.isinf(x), torch.isinf(want)):
        pytest.fail(f"{name}: support differs from the reference")  # no boundary case in these fixtures
    assert np.array_equal(x.numpy().view(np.int32), c["processed"].view(np.int32))
    tok = hs.draw(torch.from_numpy(c["processed"]).to(DEV), torch.from_numpy(c["seeds"]).to(DEV), steps).cpu()
    u = rng_ref.counter_uniform(c["seeds"], c["steps"])
    for i, (a, b) in enumerate(zip(tok.tolist(), c["tokens"].tolist())):
        assert a == b or token_at_boundary(want[i], float(u[i]), a, b), (name, i, a, b)


@pytest.mark.parametrize("name,sem", [("hf", "hf"), ("omni", "omni")])
def test_decode_streams_match_reference_golden(golden_streams, name, sem):
    c = golden_case(golden_streams, name)
    cfg = hs.TalkerSampling(semantics=sem, rng="counter", min_new_tokens=int(c["min_new"]))
    gen = torch.Generator().manual_seed(int(c["gseed"]))
    frames, rows = int(c["frames"]), int(c["rows"])
    logits = torch.randn(frames, rows, V, generator=gen)
    logits[frames - 10, 1, EOS] = 1e4
    assert abs(float(logits.double().sum()) - float(c["logits_sum"])) < 1e-9 * abs(float(c["logits_sum"]))
    st = hs.DecodeState.new([5 + i for i in range(rows)], cfg, device=DEV)
    toks = hs.decode_k(st, logits.to(DEV), EOS, cfg).cpu().numpy()
    assert np.array_equal(toks, c["tokens"])
    assert np.array_equal(st.history.cpu().numpy(), c["history"])
    assert np.array_equal(st.steps.cpu().numpy(), c["steps"])
    assert np.array_equal(st.finished.cpu().numpy(), c["finished"])


def _boundary_ok(xr, got, want, p, k, full):
    from tests.parity import support_at_boundary
    return support_at_boundary(xr, got, want, p, k, full)


@pytest.mark.parametrize("scale", [0.3, 1.0, 3.0, 8.0])
def test_mirror_filters_match_oracle(scale):
    g = torch.Generator().manual_seed(int(scale * 10))
    x = torch.randn(16, V, generator=g) * scale
    xd = x.to(DEV)
    assert torch.equal(hs.top_k_filter(xd, 25, 3).cpu(), ts.top_k_filter(x, 25, 3))
    assert torch.equal(hs.top_k_filter(xd, 0, 1).cpu(), ts.top_k_filter(x, 0, 1))
    for got, want, p, k, full in (
            (hs.top_k_top_p_filter(xd, 25, 0.85, 1).cpu(), ts.top_k_top_p_filter(x, 25, 0.85, 1), 0.85, 25, False),
            (hs.top_p_top_k_filter(xd, 0.85, 25, 3).cpu(), ts.top_p_top_k_filter(x, 0.85, 25, 3), 0.85, 25, True),
            (hs.top_p_filter(xd, 0.9, 1).cpu(), ts.top_p_filter(x, 0.9, 1), 0.9, V, True)):
        for i in range(x.shape[0]):
            fin = torch.isfinite(got[i]) & torch.isfinite(want[i])
            assert torch.equal(got[i][fin], want[i][fin])
            assert torch.equal(torch.isfinite(got[i]), torch.isfinite(want[i])) or _boundary_ok(
                x[i], got[i], want[i], p, k, full), (i, scale)
    hist = torch.randint(0, 300, (16, 64), generator=g)
    hist[:, :5] = -1
    assert torch.equal(hs.repetition_penalty(xd, hist.to(DEV), 1.3).cpu(), ts.repetition_penalty(x, hist, 1.3))


def test_step_invariants():
    cfg = hs.TalkerSampling()
    logits = torch.randn(8, V, device=DEV)
    alone = hs.step(hs.DecodeState.new([1234], device=DEV), logits[3:4], EOS, cfg)
    batch = hs.step(hs.DecodeState.new([1, 2, 3, 1234, 5, 6, 7, 8], device=DEV), logits, EOS, cfg)
    assert int(alone[0]) == int(batch[3])
    gen = torch.Generator().manual_seed(4)
    lg = torch.randn(30, 4, V, generator=gen)
    ref_state = hs.DecodeState.new([1, 2, 3, 4], device=DEV)
    want = torch.stack([hs.step(ref_state, lg[i].to(DEV), EOS, cfg) for i in range(30)])
    s = hs.DecodeState.new([1, 2, 3, 4], device=DEV)
    s.active[2] = False
    noisy = lg.clone()
    noisy[:, 2] = torch.randn(30, V, generator=gen) * 100
    got = torch.stack([hs.step(s, noisy[i].to(DEV), EOS, cfg) for i in range(30)])
    assert torch.equal(got[:, [0, 1, 3]], want[:, [0, 1, 3]]) and (got[:, 2] == hs.PAD).all()
    assert int(s.steps[2]) == 0 and (s.history[2] == hs.PAD).all()


def test_in_place_step_with_injected_uniforms_equals_step():
    cfg = hs.TalkerSampling(semantics="omni", rng="counter", min_new_tokens=3)
    gen = torch.Generator().manual_seed(9)
    lg = torch.randn(12, 5, V, generator=gen).to(DEV)
    a = hs.DecodeState.new([11, 12, 13, 14, 15], cfg, device=DEV)
    b = hs.DecodeState.new([11, 12, 13, 14, 15], cfg, device=DEV)
    for i in range(12):
        u = hs.uniform(b.seeds, b.steps)
        ta = hs.step(a, lg[i], EOS, cfg)
        tb = hs.step_(b, lg[i], EOS, cfg, uniform_values=u)
        assert torch.equal(ta, tb)
    assert torch.equal(a.history, b.history) and torch.equal(a.steps, b.steps)


def test_mixed_launch_equals_separate_launches():
    big, small = W.mixed()
    bd, sd = big.to(DEV), small.to(DEV)
    g1 = G.RowGroup(bd.logits, **bd.group_kwargs())
    g2 = G.RowGroup(sd.logits, **sd.group_kwargs())
    G.launch([g1, g2])
    h1 = G.sample(bd.logits, **bd.group_kwargs())
    h2 = G.sample(sd.logits, **sd.group_kwargs())
    torch.cuda.synchronize()
    assert torch.equal(g1.tokens, h1.tokens) and torch.equal(g2.tokens, h2.tokens)


@pytest.mark.parametrize("mode", ["window", "ring"])
def test_state_update_matches_oracle(mode):
    wl = W.talker_b8("omni", step=0)
    wl.history[:, :100] = -1
    rows = oracle_rows(wl)
    d = wl.to(DEV)
    hist = d.history.clone()
    steps = d.steps.clone()
    finished = torch.zeros(wl.rows, dtype=torch.bool, device=DEV)
    finished[5] = True
    rows.finished = finished.cpu().clone()
    head = torch.arange(wl.rows, dtype=torch.int32, device=DEV) * 7 if mode == "ring" else None
    head_cpu = head.cpu().to(torch.int64).clone() if head is not None else None
    kw = d.group_kwargs()
    kw.update(history=hist, steps=steps, finished=finished, update_state=True, history_head=head)
    for it in range(5):
        g = G.sample(d.logits, **kw)
        ref = ext.sample_rows(rows, update_state=True, history_mode=mode, history_head=head_cpu)
        torch.cuda.synchronize()
        assert torch.equal(g.tokens.cpu(), ref["tokens"]), it
        assert torch.equal(hist.cpu().to(torch.int64), rows.history.to(torch.int64)), it
        assert torch.equal(steps.cpu(), rows.steps), it
        if head is not None:
            assert torch.equal(head.cpu().to(torch.int64), head_cpu % wl.history.shape[1]), it


def test_fallback_path_on_clustered_logits():
    """Top values packed into one slice: the candidates cannot prove the top-k and the row is re-streamed."""
    wl = W.thinker_b8()
    x = wl.logits.float()
    x, _ = torch.sort(x, dim=-1)  # ascending: every top value sits in the last slice
    wl.logits = x.to(torch.bfloat16)
    wl.params["top_k"][:] = torch.tensor([1000, 100, 20, 5, 1000, 1, 300, 2], dtype=torch.int32)
    g = run(wl)
    rows = oracle_rows(wl)
    ref = ext.sample_rows(rows)
    compare_group("fallback", g.tokens, g.processed, g.probs, ref, rows, prob_rtol=2e-3)


def test_graph_replay_equals_eager():
    wl = W.talker_b8("hf").to(DEV)
    kw = wl.group_kwargs()
    eager = G.sample(wl.logits, **kw).tokens.clone()
    torch.cuda.synchronize()
    grp = G.RowGroup(wl.logits, **kw)
    G.launch([grp])  # warm the workspace outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        G.launch([grp])  # workspace for this stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            G.launch([grp])
    torch.cuda.synchronize()
    for _ in range(4):
        grp.tokens.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(grp.tokens, eager)


def test_graph_replay_after_the_stream_workspace_is_outgrown():
    """A graph captured on a stream keeps its workspace: a later, larger launch on that stream takes a new one and the
    graph's replays still match the eager tokens (the outgrown buffer stays alive for the graph)."""
    print("[gpu] graph replay after workspace growth", flush=True)
    small = W.talker_b8("hf").to(DEV)
    big = W.thinker_b64().to(DEV)
    eager_small = G.sample(small.logits, **small.group_kwargs()).tokens.clone()
    eager_big = G.sample(big.logits, **big.group_kwargs()).tokens.clone()
    torch.cuda.synchronize()
    grp = G.RowGroup(small.logits, **small.group_kwargs())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        G.launch([grp])  # the stream's workspace, sized for the small launch
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            G.launch([grp])
        torch.cuda.synchronize()
        for _ in range(3):
            gb = G.RowGroup(big.logits, **big.group_kwargs())
            G.launch([gb])  # outgrows the stream's workspace
            grp.tokens.fill_(-7)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(gb.tokens, eager_big)
            assert torch.equal(grp.tokens, eager_small)


def test_errors_are_loud():
    with pytest.raises(ValueError):
        G.RowGroup(torch.zeros(2, 8))  # CPU tensor: no CPU path
    with pytest.raises(ValueError):
        hs.processed_logits(torch.zeros(1, 8, device=DEV), torch.full((1, 2), -1, device=DEV),
                            torch.zeros(1, dtype=torch.long, device=DEV), 3, hs.TalkerSampling(semantics="x"))
    with pytest.raises(ValueError):
        G.sample(torch.zeros(2, 8, device=DEV), eos=9)  # eos outside the vocabulary


@pytest.mark.parametrize("semantics", ["hf", "omni"])
def test_censored_eos_as_row_max_greedy_and_sampled(semantics):
    """EOS is the row maximum (by far) while step < min_new_tokens: greedy rows (T = 0) and sampled rows must never
    return it, and a sampled row's draw must renormalise over the other survivors (no underflow against the
    censored maximum), in both pipeline orders."""
    print(f"[gpu] censored EOS as the row max, {semantics}", flush=True)
    gen = torch.Generator().manual_seed(404)
    rows = 6
    x = torch.randn(rows, V, generator=gen)
    x[:, EOS] = torch.tensor([150.0, 150.0, 40.0, 200.0, 150.0, 1e4])
    temps = torch.tensor([0.0, 0.8, 0.8, 1.0, 0.0, 0.7])
    one = lambda val, dt=torch.float32: torch.full((rows,), val, dtype=dt)  # noqa: E731
    hist = torch.randint(0, V, (rows, 16), generator=gen, dtype=torch.int64)
    steps = torch.tensor([1, 2, 3, 4, 5, 6], dtype=torch.int64)
    mk = 3 if semantics == "hf" else 1
    ref_rows = ext.Rows(logits=x, temperature=temps, top_k=torch.tensor([25, 25, 0, 25, 0, 0], dtype=torch.int32),
                        top_p=torch.tensor([0.85, 0.85, 0.9, 1.0, 1.0, 1.0]), repetition=one(1.05),
                        presence=one(0.0), frequency=one(0.0), history=hist, seeds=one(9, torch.int64),
                        steps=steps, eos=EOS, min_new_tokens=50, semantics=semantics, min_keep=mk)
    g = G.RowGroup(x.to(DEV), temperature=temps.to(DEV), top_k=ref_rows.top_k.to(DEV), top_p=ref_rows.top_p.to(DEV),
                   repetition=1.05, history=hist.to(DEV), seeds=one(9, torch.int64).to(DEV), steps=steps.to(DEV),
                   eos=EOS, min_new_tokens=50, semantics=semantics, min_keep=mk, processed=True, probs=True)
    G.launch([g])
    torch.cuda.synchronize()
    ref = ext.sample_rows(ref_rows)
    stats = compare_group(f"eos_censor_{semantics}", g.tokens, g.processed, g.probs, ref, ref_rows, prob_rtol=1e-5)
    assert stats["token_boundary"] == 0, stats["boundary_rows"]
    assert (g.tokens.cpu() != EOS).all()


def test_mirror_max_new_tokens_zero_forces_eos_every_frame():
    """engine/talker_sampler.py:157: steps >= max_new_tokens - 1 holds for every frame when max_new_tokens <= 0."""
    gen = torch.Generator().manual_seed(405)
    x = torch.randn(3, V, generator=gen)
    hist = torch.full((3, 16), -1, dtype=torch.int64)
    steps = torch.tensor([0, 7, 60], dtype=torch.int64)
    for max_new in (0, -3):
        for sem in ("hf", "omni"):
            cfg = hs.TalkerSampling(semantics=sem, rng="counter", max_new_tokens=max_new, min_new_tokens=0)
            rcfg = ts.TalkerSampling(semantics=sem, rng="counter", max_new_tokens=max_new, min_new_tokens=0)
            got = hs.processed_logits(x.to(DEV), hist.to(DEV), steps.to(DEV), EOS, cfg).cpu()
            want = ts.processed_logits(x, hist, steps, EOS, rcfg)
            assert torch.equal(got, want), (max_new, sem)
