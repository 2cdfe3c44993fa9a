"""Drop-in for ``engine/talker_sampler.py``: the same names and signatures, computed by the MI355X HIP kernel.

Every tensor argument must live on the GPU; there is no CPU path.  The
functions keep the reference's semantics (pipeline order, ``min_keep`` rules,
EOS censor / forcing, counter RNG, ``draw``'s clamp to ``V - 1``) with the
reference's scalar conventions (``top_k = 0`` keeps ``min_keep`` tokens, the
top-p formula is evaluated even at ``top_p = 1``).  Deliberate differences:

* ``temperature <= 0`` selects greedily (the reference divides by zero).
* ``top_p_filter`` keeps rank j when the probability mass ranked above it is
  below ``top_p`` — the descending form of the reference's ascending-sort rule,
  identical except where the two sums round across the boundary
  (``engine/talker_sampler.py:106-108`` notes the same of its fused filters).
* ``step`` / ``decode_k`` update fresh copies of the state tensors in one launch
  and rebind them, as the reference does (``:245-248``); ``step_`` updates the
  caller's tensors in place (the graph-body contract of
  ``engine/runtime/talker_post_graph.py:67-76``).
* ``draw_multinomial`` / ``restore_multinomial_states_after_block`` (the
  native-RNG mode) stay with torch's generators, as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

import torch

from . import _lib
from .groups import RowGroup, launch

PAD = -1
M32 = 0xFFFFFFFF


@dataclass(frozen=True)
class TalkerSampling:
    """``engine/talker_sampler.py:34-57``."""

    temperature: float = 0.8
    top_p: float = 0.85
    top_k: int = 25
    repetition_penalty: float = 1.05
    window: int = 16
    min_new_tokens: int = 50
    max_new_tokens: int = 2048
    min_keep: int = 3
    semantics: str = "hf"
    rng: str = "auto"

    @property
    def uses_native_rng(self) -> bool:
        if self.rng not in ("auto", "native", "counter"):
            raise ValueError(f"unknown Talker RNG mode: {self.rng!r}")
        return self.rng == "native" or (self.rng == "auto" and self.semantics == "omni")


@dataclass
class DecodeState:
    """``engine/talker_sampler.py:215-231``."""

    seeds: torch.Tensor     # [B] int64
    steps: torch.Tensor     # [B] int64, next frame index
    history: torch.Tensor   # [B, W] int64, PAD where empty
    finished: torch.Tensor  # [B] bool
    active: torch.Tensor    # [B] bool
    generators: list[torch.Generator] | None = None

    @classmethod
    def new(cls, seeds: list[int], cfg: TalkerSampling = TalkerSampling(), device="cuda") -> "DecodeState":
        b = len(seeds)
        return cls(seeds=torch.tensor(seeds, dtype=torch.int64, device=device),
                   steps=torch.zeros(b, dtype=torch.int64, device=device),
                   history=torch.full((b, cfg.window), PAD, dtype=torch.int64, device=device),
                   finished=torch.zeros(b, dtype=torch.bool, device=device),
                   active=torch.ones(b, dtype=torch.bool, device=device))


@lru_cache(maxsize=64)
def _alpha_table_cpu(penalty: float) -> torch.Tensor:
    """``torch.pow(penalty, n)`` for n < 256, as the reference computes alpha (``:83``)."""
    return torch.pow(torch.full((256,), penalty, dtype=torch.float32), torch.arange(256, dtype=torch.float32))


_alpha_dev: dict[tuple[float, torch.device], torch.Tensor] = {}


def _alpha_table(penalty: float, device: torch.device) -> torch.Tensor:
    key = (float(penalty), device)
    t = _alpha_dev.get(key)
    if t is None:
        t = _alpha_table_cpu(float(penalty)).to(device)
        _alpha_dev[key] = t
    return t


def _check_semantics(cfg: TalkerSampling) -> None:
    if cfg.semantics not in ("hf", "omni"):
        raise ValueError(f"unknown Talker sampling semantics: {cfg.semantics!r}")


def _as_i64(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    t = torch.as_tensor(t, device=device)
    return t.to(torch.int64).contiguous()


def uniform(seeds: torch.Tensor, steps: torch.Tensor) -> torch.Tensor:
    """Counter uniform keyed by (seed, frame) (``engine/talker_sampler.py:70-76``); broadcasts like the reference."""
    if seeds.device.type != "cuda":
        raise ValueError("uniform: seeds must be on the GPU")
    s, t = torch.broadcast_tensors(seeds.to(torch.int64), steps.to(device=seeds.device, dtype=torch.int64))
    return _lib.uniform(s.contiguous(), t.contiguous(), None, _lib.MIS_RNG_COUNTER)


def philox_uniform(seeds: torch.Tensor, steps: torch.Tensor, row_ids: torch.Tensor) -> torch.Tensor:
    """Philox4x32-10 uniforms keyed by (seed, request id, step); no reference counterpart."""
    s, t, r = torch.broadcast_tensors(seeds.to(torch.int64), steps.to(seeds.device, torch.int64),
                                      row_ids.to(seeds.device, torch.int64))
    return _lib.uniform(s.contiguous(), t.contiguous(), r.contiguous(), _lib.MIS_RNG_PHILOX)


def _filter(x: torch.Tensor, **kw) -> torch.Tensor:
    """Processed logits of a filter-only launch: T = 1 (an exact division), no draw."""
    args = dict(temperature=1.0, tokens=False, processed=True, top_k_zero_disables=False, top_p_one_disables=False)
    args.update(kw)
    g = RowGroup(x, **args)
    launch([g])
    return g.processed


def repetition_penalty(x: torch.Tensor, history: torch.Tensor, penalty: float) -> torch.Tensor:
    """``engine/talker_sampler.py:79-84``: a token seen n times in the window is scaled by ``penalty**n``."""
    return _filter(x.float(), history=history, repetition=float(penalty), alpha_lut=_alpha_table(penalty, x.device),
                   top_k=x.shape[-1], top_p=1.0, top_p_one_disables=True)


def top_p_filter(x: torch.Tensor, top_p: float, min_keep: int) -> torch.Tensor:
    """``engine/talker_sampler.py:87-92`` (nucleus over the whole vocabulary)."""
    return _filter(x.float(), top_k=x.shape[-1], top_p=float(top_p), min_keep=int(min_keep))


def top_k_filter(x: torch.Tensor, top_k: int, min_keep: int) -> torch.Tensor:
    """``engine/talker_sampler.py:95-98``: ties at the k-th value are kept."""
    return _filter(x.float(), top_k=int(top_k), min_keep=int(min_keep), top_p=1.0, top_p_one_disables=True)


def top_p_top_k_filter(x: torch.Tensor, top_p: float, top_k: int, min_keep: int) -> torch.Tensor:
    """``engine/talker_sampler.py:101-116``: full-vocabulary normaliser (the HF order)."""
    later = torch.ones(x.shape[0], dtype=torch.int64, device=x.device)
    return _filter(x.float(), top_k=int(top_k), top_p=float(top_p), min_keep=int(min_keep), semantics="hf",
                   steps=later)


def top_k_top_p_filter(x: torch.Tensor, top_k: int, top_p: float, min_keep: int = 1) -> torch.Tensor:
    """``engine/talker_sampler.py:119-133``: normaliser over the top-k only (the vLLM order)."""
    return _filter(x.float(), top_k=int(top_k), top_p=float(top_p), min_keep=int(min_keep))


def _cfg_group(logits: torch.Tensor, history: torch.Tensor, steps: torch.Tensor, eos: int, cfg: TalkerSampling,
               **kw) -> RowGroup:
    _check_semantics(cfg)
    dev = logits.device
    # The reference forces EOS at steps >= max_new_tokens - 1 (:157), so max_new_tokens <= 0 forces it on every
    # frame (frame indices are >= 0); the kernel reads 0 as "never", so such a budget is passed as 1.
    max_new = int(cfg.max_new_tokens) if int(cfg.max_new_tokens) > 0 else 1
    return RowGroup(logits, temperature=float(cfg.temperature), top_k=int(cfg.top_k), top_p=float(cfg.top_p),
                    repetition=float(cfg.repetition_penalty), alpha_lut=_alpha_table(cfg.repetition_penalty, dev),
                    history=history, eos=int(eos), min_new_tokens=int(cfg.min_new_tokens),
                    max_new_tokens=max_new, semantics=cfg.semantics,
                    min_keep=int(cfg.min_keep) if cfg.semantics == "hf" else 1, top_k_zero_disables=False,
                    top_p_one_disables=False, steps=steps, **kw)


def processed_logits(logits: torch.Tensor, history: torch.Tensor, steps: torch.Tensor, eos: int,
                     cfg: TalkerSampling) -> torch.Tensor:
    """``engine/talker_sampler.py:136-158``."""
    g = _cfg_group(logits, history, _as_i64(steps, logits.device), eos, cfg, tokens=False, processed=True)
    launch([g])
    return g.processed


def draw(x: torch.Tensor, seeds: torch.Tensor, steps: torch.Tensor, *, uniform_values: torch.Tensor | None = None
         ) -> torch.Tensor:
    """``engine/talker_sampler.py:161-172``: softmax, cumulative sum in vocabulary order, first entry above
    ``u * total`` (``searchsorted(right=True)``), clamped to ``V - 1``."""
    dev = x.device
    kw = {}
    if uniform_values is not None:
        kw["uniforms"] = uniform_values.to(device=dev, dtype=torch.float32)
    else:
        kw["seeds"] = _as_i64(seeds, dev)
        kw["steps"] = _as_i64(steps, dev)
    g = RowGroup(x.float(), temperature=1.0, top_k=0, top_p=1.0, **kw)
    launch([g])
    return g.tokens


def draw_multinomial(x: torch.Tensor, generators: list[torch.Generator]) -> torch.Tensor:
    """``engine/talker_sampler.py:175-188``: torch's per-request generators (native-RNG mode)."""
    if len(generators) != x.size(0):
        raise ValueError(f"expected {x.size(0)} generators, got {len(generators)}")
    probs = torch.softmax(x, dim=-1)
    return torch.stack([torch.multinomial(probs[i], 1, generator=g).reshape(()) for i, g in enumerate(generators)])


def restore_multinomial_states_after_block(generators: list[torch.Generator],
                                           states_after_step: list[list[torch.Tensor]],
                                           host_tokens: torch.Tensor) -> None:
    """``engine/talker_sampler.py:191-212``: rewind each generator to its last non-PAD draw of a K block."""
    if not states_after_step:
        return
    if len(generators) != host_tokens.size(1):
        raise ValueError("generator/token row mismatch")
    for row, generator in enumerate(generators):
        pads = (host_tokens[:, row] == PAD).nonzero()
        draws = int(pads[0]) if pads.numel() else host_tokens.size(0)
        if 0 < draws < len(states_after_step):
            generator.set_state(states_after_step[draws - 1][row])


def step_(state: DecodeState, logits: torch.Tensor, eos: int, cfg: TalkerSampling = TalkerSampling(),
          uniform_values: torch.Tensor | None = None) -> torch.Tensor:
    """``step`` updating ``state.history`` / ``steps`` / ``finished`` in place (one launch, graph-capturable).

    ``uniform_values`` injects the draws, as ``engine/runtime/talker_post_graph.py:60-65`` does."""
    if cfg.uses_native_rng:
        raise ValueError("step_ needs the counter RNG; native generators are host-driven (use step)")
    dev = logits.device
    kw = {"uniforms": uniform_values} if uniform_values is not None else {"seeds": state.seeds}
    g = _cfg_group(logits, state.history, state.steps, eos, cfg, active=state.active, finished=state.finished,
                   update_state=True, **kw)
    launch([g])
    return g.tokens


def step(state: DecodeState, logits: torch.Tensor, eos: int, cfg: TalkerSampling = TalkerSampling()) -> torch.Tensor:
    """``engine/talker_sampler.py:234-249``: one frame per row; inactive / finished rows return ``PAD`` and keep
    their state.  The state's history, steps and finished tensors are rebound to updated copies."""
    live = state.active & ~state.finished
    if cfg.uses_native_rng:
        if state.generators is None:
            raise ValueError("native Talker RNG requires one generator per row")
        tok = draw_multinomial(processed_logits(logits, state.history, state.steps, eos, cfg), state.generators)
        tok = torch.where(live, tok, torch.full_like(tok, PAD))
        shifted = torch.cat([state.history[:, 1:], tok[:, None]], dim=1)
        state.history = torch.where(live[:, None], shifted, state.history)
        state.steps = state.steps + live.to(torch.int64)
        state.finished = state.finished | (live & (tok == eos))
        return tok
    state.history = state.history.to(torch.int64).clone()
    state.steps = state.steps.to(torch.int64).clone()
    state.finished = state.finished.to(torch.bool).clone()
    return step_(state, logits, eos, cfg)


def decode_k(state: DecodeState, logits_k: torch.Tensor, eos: int, cfg: TalkerSampling = TalkerSampling()
             ) -> torch.Tensor:
    """``engine/talker_sampler.py:252-254``: K frames from precomputed logits [K, B, V]."""
    return torch.stack([step(state, logits_k[i], eos, cfg) for i in range(logits_k.size(0))])
