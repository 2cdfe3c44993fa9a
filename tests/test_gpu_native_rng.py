"""Native-RNG mode of the mirror on the device (``engine/talker_sampler.py:175-212``; the reference pins it in
``tests/engine/test_talker_sampler.py:175-222``): per-request ``torch.multinomial`` generators drive the draw, the
counter mode leaves them untouched, and a K block's speculative draws after a row's first PAD are rewound.

The processed logits come from the HIP kernel; they equal the oracle's bit for bit, so per-row
``torch.multinomial`` with identically seeded device generators over the oracle's logits gives the same tokens.
"""

from __future__ import annotations

import pytest
import torch

from mi355x_sampler import talker_sampler as ts
from oracle import talker_sampler_ref as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
V, EOS = 6562, 6561


@pytest.fixture(scope="module", autouse=True)
def _gpu(gpu_lib):
    torch.cuda.set_device(0)
    yield


def _ref_cfg(cfg: ts.TalkerSampling) -> ref.TalkerSampling:
    return ref.TalkerSampling(**{f: getattr(cfg, f) for f in ref.TalkerSampling.__dataclass_fields__})


def _gens(seeds):
    return [torch.Generator(device=DEV).manual_seed(s) for s in seeds]


def test_native_step_is_per_request_multinomial_over_steps():
    print("[gpu] native RNG: 12 omni steps with device generators", flush=True)
    cfg = ts.TalkerSampling(semantics="omni", min_new_tokens=4)
    assert cfg.uses_native_rng
    rcfg = _ref_cfg(cfg)
    seeds = [101, 202, 303, 404]
    gen = torch.Generator().manual_seed(77)
    state = ts.DecodeState.new(seeds, cfg, DEV)
    state.generators = _gens(seeds)
    oracle = ref.DecodeState.new(seeds, rcfg)
    expected_gens = _gens(seeds)
    for t in range(12):
        logits = torch.randn(len(seeds), V, generator=gen) * 2
        prepared = ref.processed_logits(logits, oracle.history, oracle.steps, EOS, rcfg)
        got_prepared = ts.processed_logits(logits.to(DEV), state.history, state.steps, EOS, cfg).cpu()
        assert torch.equal(got_prepared, prepared), t
        probs = torch.softmax(prepared.to(DEV), dim=-1)
        want = torch.stack([torch.multinomial(probs[i], 1, generator=g).reshape(())
                            for i, g in enumerate(expected_gens)]).cpu()
        got = ts.step(state, logits.to(DEV), EOS, cfg).cpu()
        assert torch.equal(got, want), (t, got, want)
        # the oracle's state advances with the same tokens (the reference's step body, draw aside)
        live = oracle.active & ~oracle.finished
        tok = torch.where(live, want, torch.full_like(want, ref.PAD))
        oracle.history = torch.where(live[:, None], torch.cat([oracle.history[:, 1:], tok[:, None]], 1),
                                     oracle.history)
        oracle.steps = oracle.steps + live.to(torch.int64)
        oracle.finished = oracle.finished | (live & (tok == EOS))
    for f in ("steps", "history", "finished"):
        assert torch.equal(getattr(state, f).cpu(), getattr(oracle, f)), f
    with pytest.raises(ValueError, match="one generator per row"):
        ts.step(ts.DecodeState.new(seeds, cfg, DEV), torch.zeros(4, V, device=DEV), EOS, cfg)


def test_draw_multinomial_on_device_generators():
    cfg = ts.TalkerSampling(semantics="omni", min_new_tokens=0)
    logits = torch.randn(3, V, generator=torch.Generator().manual_seed(78)).to(DEV)
    x = ts.processed_logits(logits, torch.full((3, 16), ts.PAD, device=DEV), torch.zeros(3, dtype=torch.long,
                            device=DEV), EOS, cfg)
    got = ts.draw_multinomial(x, _gens([1, 2, 3]))
    probs = torch.softmax(x, dim=-1)
    want = torch.stack([torch.multinomial(probs[i], 1, generator=g).reshape(()) for i, g in enumerate(_gens([1, 2, 3]))])
    assert torch.equal(got.cpu(), want.cpu())
    with pytest.raises(ValueError, match="expected 3 generators"):
        ts.draw_multinomial(x, _gens([1, 2]))


def test_counter_mode_does_not_advance_native_generators():
    cfg = ts.TalkerSampling(semantics="omni", rng="counter", min_new_tokens=0)
    assert not cfg.uses_native_rng
    logits = torch.randn(3, V, generator=torch.Generator().manual_seed(79))
    seeds = [101, 202, 303]
    state = ts.DecodeState.new(seeds, cfg, DEV)
    state.generators = _gens(seeds)
    before = [g.get_state().clone() for g in state.generators]
    rcfg = _ref_cfg(cfg)
    o = ref.DecodeState.new(seeds, rcfg)
    want = ref.draw(ref.processed_logits(logits, o.history, o.steps, EOS, rcfg), o.seeds, o.steps)
    assert torch.equal(ts.step(state, logits.to(DEV), EOS, cfg).cpu(), want)
    assert all(torch.equal(g.get_state(), s) for g, s in zip(state.generators, before))


def test_block_rewind_restores_device_generators_after_pad():
    probs = torch.tensor([0.1, 0.2, 0.3, 0.4], device=DEV)
    reference = torch.Generator(device=DEV).manual_seed(987)
    expected = [int(torch.multinomial(probs, 1, generator=reference)) for _ in range(3)]
    expected_next = int(torch.multinomial(probs, 1, generator=reference))
    g = torch.Generator(device=DEV).manual_seed(987)
    states = []
    for _ in range(6):
        torch.multinomial(probs, 1, generator=g)
        states.append([g.get_state().clone()])
    host = torch.tensor([[expected[0]], [expected[1]], [expected[2]], [ts.PAD], [ts.PAD], [ts.PAD]])
    ts.restore_multinomial_states_after_block([g], states, host)
    assert int(torch.multinomial(probs, 1, generator=g)) == expected_next
    with pytest.raises(ValueError, match="mismatch"):
        ts.restore_multinomial_states_after_block([g, g], states, host)
