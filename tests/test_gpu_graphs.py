"""Captured decode bodies: the Talker post graph (replay == eager == oracle) and K-frame sample blocks, including
the mixed 64 Thinker + 64 Talker step advanced over 128 consecutive steps in captured 16-step blocks.

Mirrors the reference's replay regression (``tests/engine/test_talker_post_graph_npu.py:23-81``): edge seeds
(2^63 - 1, 2^32, 2^32 - 1), two blocks of 16 frames per row count, a forced EOS in the middle of a block and an
inactive row in a padded bucket.  Every frame is also checked against the CPU oracle on the same logits.
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch
import torch.nn.functional as F

from mi355x_sampler import graphs
from mi355x_sampler import groups as G
from mi355x_sampler import talker_sampler as ts
from mi355x_sampler import workloads as W
from oracle import extended_ref as ext
from oracle import talker_sampler_ref as ref
from tests.parity import oracle_rows, token_at_boundary

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
SEEDS = [0, 42, (1 << 63) - 1, (1 << 60) + 1234567, 1 << 32, 1, 2035223770, (1 << 32) - 1]
CFG = ts.TalkerSampling(semantics="omni", rng="counter")
VOCAB, WIDTH = 6563, 256
EOS = VOCAB - 1


@pytest.fixture(scope="module", autouse=True)
def _gpu(gpu_lib):
    torch.cuda.set_device(0)
    yield


def _ref_cfg(cfg: ts.TalkerSampling) -> ref.TalkerSampling:
    return ref.TalkerSampling(**{f: getattr(cfg, f) for f in ref.TalkerSampling.__dataclass_fields__})


def _ref_state(seeds, cfg) -> ref.DecodeState:
    return ref.DecodeState.new(seeds, _ref_cfg(cfg))


def _oracle_step(state: ref.DecodeState, logits: torch.Tensor, cfg, got: torch.Tensor) -> int:
    """One oracle step on the CPU; a token that differs from the GPU's only at a CDF step is adopted (the row's
    state then follows the GPU).  Returns the number of such rows."""
    rcfg = _ref_cfg(cfg)
    x = logits.cpu()
    prepared = ref.processed_logits(x, state.history, state.steps, EOS, rcfg)
    u = ref.uniform(state.seeds, state.steps)
    want = ref.step(state, x, EOS, rcfg)
    got = got.cpu()
    nb = 0
    for i in torch.nonzero(want != got).flatten().tolist():
        assert int(want[i]) >= 0 and int(got[i]) >= 0, (i, int(want[i]), int(got[i]))
        assert token_at_boundary(prepared[i], float(u[i]), int(got[i]), int(want[i])), (i, int(got[i]), int(want[i]))
        state.history[i, -1] = got[i]
        state.finished[i] = bool(got[i] == EOS)
        nb += 1
    return nb


def _states_equal(a, b) -> None:
    for f in ("seeds", "steps", "history", "finished", "active"):
        assert torch.equal(getattr(a, f).cpu(), getattr(b, f).cpu()), f


@pytest.mark.parametrize("rows", [1, 3, 4, 8])
def test_post_graph_replay_matches_eager_and_oracle(rows):
    print(f"[gpu] post graph rows={rows}", flush=True)
    gen = torch.Generator().manual_seed(172 + rows)
    head = (torch.randn(VOCAB, WIDTH, generator=gen) * .02).bfloat16().to(DEV)
    eager, captured = [ts.DecodeState.new(SEEDS[:rows], CFG, DEV) for _ in range(2)]
    oracle = _ref_state(SEEDS[:rows], CFG)
    for s in (eager, captured, oracle):
        s.steps.fill_(60)
    post = graphs.TalkerPostGraphs(head, EOS, CFG)
    nb = 0
    for _ in range(2):  # the second block rebinds with the advanced frame indices
        assert post.begin(captured, frames=16), post.failures
        for frame in range(16):
            hidden = (torch.randn(rows, WIDTH, generator=gen) * .25).bfloat16().to(DEV)
            logits = F.linear(hidden, head).float()
            expected = ts.step(eager, logits, EOS, CFG)
            observed, feed = post.step(hidden)
            assert torch.equal(expected.cpu(), observed.cpu()), (rows, frame, expected.cpu(), observed.cpu())
            assert torch.equal(feed.cpu(), observed.clamp_min(0).cpu())
            nb += _oracle_step(oracle, logits, CFG, observed)
        with pytest.raises(RuntimeError, match="exhausted"):
            post.step(hidden)
        post.finish()
        _states_equal(eager, captured)
        _states_equal(eager, oracle)
    assert post.replays == {post._bucket(rows): 32}
    assert nb == 0, f"{nb} oracle rows decided only at a CDF step"
    with pytest.raises(RuntimeError, match="not bound"):
        post.step(hidden)


def test_post_graph_eos_and_inactive_rows_freeze_in_padded_bucket():
    print("[gpu] post graph mid-block EOS, inactive row", flush=True)
    cfg = replace(CFG, min_new_tokens=0, max_new_tokens=69)
    gen = torch.Generator().manual_seed(173)
    head = (torch.randn(VOCAB, WIDTH, generator=gen) * .02).bfloat16()
    head[:, -1] = 0
    head[EOS, -1] = 20
    head = head.to(DEV)
    eager, captured = [ts.DecodeState.new(SEEDS[:3], cfg, DEV) for _ in range(2)]
    oracle = _ref_state(SEEDS[:3], cfg)
    for s in (eager, captured, oracle):
        s.steps.fill_(60)
        s.active[1] = False
    post = graphs.TalkerPostGraphs(head, EOS, cfg)
    assert post.begin(captured, frames=16), post.failures
    outputs = []
    for frame in range(16):
        hidden = (torch.randn(3, WIDTH, generator=gen) * .25).bfloat16()
        hidden[:, -1] = 0
        if frame == 2:
            hidden[0, -1] = 10  # EOS dominates row 0 in the middle of the block
        hidden = hidden.to(DEV)
        logits = F.linear(hidden, head).float()
        expected = ts.step(eager, logits, EOS, cfg)
        observed, _ = post.step(hidden)
        assert torch.equal(expected.cpu(), observed.cpu()), frame
        assert _oracle_step(oracle, logits, cfg, observed) == 0
        outputs.append(observed.cpu())
    post.finish()
    _states_equal(eager, captured)
    _states_equal(eager, oracle)
    out = torch.stack(outputs)
    assert out[2, 0] == EOS and (out[3:, 0] == ts.PAD).all()
    assert (out[:, 1] == ts.PAD).all()
    assert int(captured.steps[0]) == 63 and int(captured.steps[1]) == 60
    assert int(captured.steps[2]) == 69 and bool(captured.finished[2])  # EOS forced at step 68
    with pytest.raises(ValueError, match="at least one"):
        post.begin(captured, frames=0)


def _frame_logits(base: torch.Tensor, step: int) -> torch.Tensor:
    """A different logits matrix per step from one seeded base (rows rotated along the vocabulary)."""
    return torch.roll(base, shifts=(37 * step) % base.shape[1], dims=1)


@pytest.mark.timeout(600)
def test_mixed_step_128_steps_in_captured_blocks_matches_oracle():
    """64 Thinker rows (vocab 151,748 bf16, heterogeneous params, repetition 1.1 over 4,096-token histories, 30%
    masked) plus 64 Talker rows (vocab 6,562 fp32, HF order) sampled in one launch per step, 128 consecutive steps
    captured as 8 blocks of 16, histories appended and steps advanced in place inside the graph; every step's
    tokens and the final state against the oracle for both groups."""
    big, small = W.mixed()
    K, blocks = 16, 8
    wls = [big, small]
    dev = [w.to(DEV) for w in wls]
    state = []
    specs = []
    for d in dev:
        st = {"history": d.history.clone(), "steps": d.steps.clone(),
              "finished": torch.zeros(d.rows, dtype=torch.bool, device=DEV)}
        state.append(st)
        kw = d.group_kwargs()
        kw.update(st)
        kw["logits"] = d.logits
        specs.append(kw)
    rows = [oracle_rows(w) for w in wls]
    for r in rows:
        r.finished = torch.zeros(r.rows, dtype=torch.bool)
    block = graphs.SampleBlockGraph(specs, K)
    for b in range(blocks):
        print(f"[gpu] mixed 128-step run: block {b}", flush=True)
        frames = [torch.stack([_frame_logits(w.logits, b * K + f) for f in range(K)]) for w in wls]
        unis = [graphs.block_uniforms(d.seeds, st["steps"], K, d.rng, d.row_ids) for d, st in zip(dev, state)]
        toks = block.run([fr.to(DEV) for fr in frames], unis)
        for f in range(K):
            for gi in range(2):
                r = rows[gi]
                r.logits = frames[gi][f]
                r.uniforms = unis[gi][f].cpu()
                want = ext.sample_rows(r, update_state=True, with_probs=False)
                got = toks[gi][f].cpu()
                bad = torch.nonzero(got != want["tokens"]).flatten().tolist()
                assert not bad, f"group {gi} step {b * K + f} rows {bad}: {got[bad].tolist()} vs oracle " \
                                f"{want['tokens'][bad].tolist()}"
        for gi in range(2):
            assert torch.equal(state[gi]["history"].cpu().to(torch.int64), rows[gi].history.to(torch.int64)), (b, gi)
            assert torch.equal(state[gi]["steps"].cpu(), rows[gi].steps), (b, gi)
            assert torch.equal(state[gi]["finished"].cpu(), rows[gi].finished), (b, gi)
    assert int(state[0]["steps"][0]) == 128 and int(state[1]["steps"][0]) == 128
    print("[gpu] mixed 128 steps: every token exact", flush=True)


def test_block_graph_replays_equal_eager_steps():
    """A captured 16-step Talker block (HF order, counter RNG, mid-block EOS, an inactive and a finished row)
    equals 16 eager launches on the same inputs, over two consecutive blocks."""
    print("[gpu] block graph == eager", flush=True)
    gen = torch.Generator().manual_seed(5)
    rows, v, K = 6, 6562, 16
    base = torch.randn(rows, v, generator=gen) * 3
    seeds = torch.tensor(SEEDS[2:8], dtype=torch.int64, device=DEV)

    def fresh():
        return {"history": torch.full((rows, 16), -1, dtype=torch.int64, device=DEV),
                "steps": torch.full((rows,), 45, dtype=torch.int64, device=DEV),
                "finished": torch.tensor([0, 0, 0, 1, 0, 0], dtype=torch.bool, device=DEV),
                "active": torch.tensor([1, 1, 0, 1, 1, 1], dtype=torch.bool, device=DEV)}

    def kw(st):
        return dict(temperature=0.8, top_k=25, top_p=0.85, repetition=1.05, semantics="hf", min_keep=3,
                    eos=v - 1, min_new_tokens=50, max_new_tokens=2048, rng="counter", **st)

    cap, eag = fresh(), fresh()
    block = graphs.SampleBlockGraph([dict(logits=base.to(DEV), **kw(cap))], K)
    for b in range(2):
        frames = torch.stack([_frame_logits(base, b * K + f) for f in range(K)])
        frames[5, 1, v - 1] = 60.0  # row 1 ends in the middle of the first block (after its censor)
        u = graphs.block_uniforms(seeds, eag["steps"], K, "counter")
        got = block.run([frames.to(DEV)], [u])[0]
        for f in range(K):
            g = G.sample(frames[f].to(DEV), uniforms=u[f], update_state=True, **kw(eag))
            assert torch.equal(g.tokens, got[f]), (b, f)
        for k in ("history", "steps", "finished"):
            assert torch.equal(cap[k], eag[k]), (b, k)
    assert bool(cap["finished"][1]) and (got[:, 2] == -1).all() and (got[:, 3] == -1).all()
