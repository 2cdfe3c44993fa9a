"""Eager-torch CPU restatement of the reference sampler (oracle; test infrastructure only).

Follows ``engine/talker_sampler.py`` function by function.  Every function
takes and returns CPU tensors and reproduces the reference's arithmetic order
(same torch operations, same dtypes), so on the same torch build it returns
the same bits as the reference.

Pins (see ``tests/test_oracle_reference.py``):

* ``uniform`` — golden vectors written by ``tests/golden/make_golden.py`` from
  the reference module itself; the published lowbias32 finalizer
  (``rng_ref.lowbias32``, numpy and C restatements, a bijection test); the
  reference's own invariants (``tests/engine/test_talker_sampler.py:92-98``).
* ``repetition_penalty`` — the HF processor logic restated in the reference's
  tests (``tests/engine/test_talker_sampler.py:13-27``): one-hot counting.
* ``top_p_filter`` / ``top_k_filter`` — transformers' ``TopPLogitsWarper`` and
  ``TopKLogitsWarper`` (the library routines the reference's tests pin against).
* ``top_p_top_k_filter`` / ``top_k_top_p_filter`` — equal support to the
  two-pass compositions (``tests/engine/test_talker_sampler.py:131-155``) and a
  brute-force enumeration over sorted ranks on small vocabularies.
* ``processed_logits`` — the HF order of ``tests/engine/test_talker_sampler.py:30-64``
  (transformers warpers), frame-0 / EOS rules (``:76-89``), golden vectors.
* ``draw`` — brute-force inverse CDF in float64 on small inputs and golden
  vectors; ``step`` / ``decode_k`` — golden token streams and the reference's
  invariants (batch independence, K-step equivalence, padded rows).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

PAD = -1
M32 = 0xFFFFFFFF


@dataclass(frozen=True)
class TalkerSampling:
    """``engine/talker_sampler.py:34-57`` (defaults and the ``uses_native_rng`` rule)."""

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


def _mix32(v: torch.Tensor) -> torch.Tensor:
    """lowbias32 on int64 lanes (``engine/talker_sampler.py:60-67``)."""
    v = v & M32
    v = v ^ (v >> 16)
    v = (v * 0x7FEB352D) & M32
    v = v ^ (v >> 15)
    v = (v * 0x846CA68B) & M32
    return v ^ (v >> 16)


def uniform(seeds: torch.Tensor, steps: torch.Tensor) -> torch.Tensor:
    """Counter uniform keyed by (seed, frame) (``engine/talker_sampler.py:70-76``)."""
    s = seeds.to(torch.int64)
    h = _mix32(s & M32)
    h = _mix32(h ^ ((s >> 32) & M32) ^ 0x9E3779B9)
    h = _mix32(h ^ (steps.to(torch.int64) & M32) ^ 0x632BE5AB)
    return (h >> 8).to(torch.float32) * (1.0 / (1 << 24))


def token_counts(history: torch.Tensor, vocab: int, dtype=torch.float32) -> torch.Tensor:
    """Per-row occurrence counts of the history ids; ``PAD`` (negative) slots count zero.

    The counting step of ``engine/talker_sampler.py:81-82``.
    """
    valid = history >= 0
    out = torch.zeros(history.shape[0], vocab, dtype=dtype)
    return out.scatter_add_(1, history.clamp(min=0).to(torch.int64), valid.to(dtype))


def repetition_penalty(x: torch.Tensor, history: torch.Tensor, penalty: float) -> torch.Tensor:
    """Count-powered penalty (``engine/talker_sampler.py:79-84``): ``alpha = penalty**n``."""
    n = token_counts(history, x.shape[-1], x.dtype)
    alpha = torch.pow(torch.full_like(x, penalty), n)
    return torch.where(x < 0, x * alpha, x / alpha)


def top_p_filter(x: torch.Tensor, top_p: float, min_keep: int) -> torch.Tensor:
    """HF top-p by ascending sort (``engine/talker_sampler.py:87-92``)."""
    asc, order = torch.sort(x, dim=-1, descending=False)
    cum = asc.softmax(dim=-1).cumsum(dim=-1)
    drop = cum <= (1 - top_p)
    drop[..., -min_keep:] = False
    return x.masked_fill(drop.scatter(1, order, drop), float("-inf"))


def top_k_filter(x: torch.Tensor, top_k: int, min_keep: int) -> torch.Tensor:
    """``engine/talker_sampler.py:95-98``: ties at the k-th value are kept."""
    k = min(max(top_k, min_keep), x.size(-1))
    kth = torch.topk(x, k, dim=-1).values[..., -1:]
    return x.masked_fill(x < kth, float("-inf"))


def _kept_threshold(vals: torch.Tensor, probs: torch.Tensor, top_p: float, min_keep: int, k: int) -> torch.Tensor:
    """Last kept rank from the exclusive descending mass (``engine/talker_sampler.py:113-115,130-132``)."""
    above = probs.cumsum(dim=-1) - probs
    kept = (above < top_p).sum(dim=-1).clamp(min=min(min_keep, k), max=k)
    return vals.gather(1, (kept - 1)[:, None])


def top_p_top_k_filter(x: torch.Tensor, top_p: float, top_k: int, min_keep: int) -> torch.Tensor:
    """HF fused form, full-vocabulary normaliser (``engine/talker_sampler.py:101-116``)."""
    k = min(max(top_k, min_keep), x.size(-1))
    vals = torch.topk(x, k, dim=-1).values
    probs = torch.exp(vals - torch.logsumexp(x, dim=-1, keepdim=True))
    thr = _kept_threshold(vals, probs, top_p, min_keep, k)
    return x.masked_fill(x < thr, float("-inf"))


def top_k_top_p_filter(x: torch.Tensor, top_k: int, top_p: float, min_keep: int = 1) -> torch.Tensor:
    """vLLM order, normaliser over the top-k only (``engine/talker_sampler.py:119-133``)."""
    k = min(max(int(top_k), int(min_keep)), x.size(-1))
    vals = torch.topk(x, k, dim=-1).values
    probs = torch.softmax(vals, dim=-1)
    thr = _kept_threshold(vals, probs, top_p, min_keep, k)
    return x.masked_fill(x < thr, float("-inf"))


def processed_logits(logits: torch.Tensor, history: torch.Tensor, steps: torch.Tensor, eos: int,
                     cfg: TalkerSampling) -> torch.Tensor:
    """``engine/talker_sampler.py:136-158`` (both orders, EOS censor and forced EOS)."""
    if cfg.semantics not in ("hf", "omni"):
        raise ValueError(f"unknown Talker sampling semantics: {cfg.semantics!r}")
    x = logits.float()
    is_eos = torch.arange(x.size(-1))[None, :] == eos
    censor = is_eos & (steps < cfg.min_new_tokens)[:, None]
    if cfg.semantics == "omni":
        x = x.masked_fill(censor, float("-inf"))
        x = repetition_penalty(x, history, cfg.repetition_penalty) / cfg.temperature
        x = top_k_top_p_filter(x, cfg.top_k, cfg.top_p, min_keep=1)
    else:
        x = x / cfg.temperature
        filtered = top_p_top_k_filter(repetition_penalty(x, history, cfg.repetition_penalty), cfg.top_p, cfg.top_k,
                                      cfg.min_keep)
        x = torch.where((steps > 0)[:, None], filtered, x)
        x = x.masked_fill(censor, float("-inf"))
    forced = (steps >= cfg.max_new_tokens - 1)[:, None]
    neg = torch.full_like(x, float("-inf"))
    return torch.where(forced & ~is_eos, neg, torch.where(forced & is_eos, torch.zeros_like(x), x))


def draw(x: torch.Tensor, seeds: torch.Tensor, steps: torch.Tensor, *, uniform_values: torch.Tensor | None = None
         ) -> torch.Tensor:
    """Inverse-CDF draw in vocabulary order (``engine/talker_sampler.py:161-172``)."""
    cdf = torch.softmax(x, dim=-1).cumsum(dim=-1)
    u = uniform(seeds, steps) if uniform_values is None else uniform_values
    target = u.to(cdf.dtype)[:, None] * cdf[:, -1:]
    return torch.searchsorted(cdf, target, right=True).squeeze(-1).clamp_(max=x.size(-1) - 1)


def draw_multinomial(x: torch.Tensor, generators: list[torch.Generator]) -> torch.Tensor:
    """``engine/talker_sampler.py:175-188``."""
    if len(generators) != x.size(0):
        raise ValueError(f"expected {x.size(0)} generators, got {len(generators)}")
    probs = torch.softmax(x, dim=-1)
    return torch.stack([torch.multinomial(probs[i], 1, generator=g).reshape(()) for i, g in enumerate(generators)])


@dataclass
class DecodeState:
    """``engine/talker_sampler.py:215-231``."""

    seeds: torch.Tensor
    steps: torch.Tensor
    history: torch.Tensor
    finished: torch.Tensor
    active: torch.Tensor
    generators: list[torch.Generator] | None = None

    @classmethod
    def new(cls, seeds: list[int], cfg: TalkerSampling = TalkerSampling(), device="cpu") -> "DecodeState":
        b = len(seeds)
        return cls(seeds=torch.tensor(seeds, dtype=torch.int64, device=device),
                   steps=torch.zeros(b, dtype=torch.int64, device=device),
                   history=torch.full((b, cfg.window), PAD, dtype=torch.int64, device=device),
                   finished=torch.zeros(b, dtype=torch.bool, device=device),
                   active=torch.ones(b, dtype=torch.bool, device=device))


def step(state: DecodeState, logits: torch.Tensor, eos: int, cfg: TalkerSampling = TalkerSampling(),
         uniform_values: torch.Tensor | None = None) -> torch.Tensor:
    """``engine/talker_sampler.py:234-249``; ``uniform_values`` injects the draw's uniforms
    (as ``engine/runtime/talker_post_graph.py:60-65`` does)."""
    live = state.active & ~state.finished
    x = processed_logits(logits, state.history, state.steps, eos, cfg)
    if cfg.uses_native_rng:
        if state.generators is None:
            raise ValueError("native Talker RNG requires one generator per row")
        tok = draw_multinomial(x, state.generators)
    else:
        tok = draw(x, state.seeds, state.steps, uniform_values=uniform_values)
    tok = torch.where(live, tok, torch.full_like(tok, PAD))
    shifted = torch.cat([state.history[:, 1:], tok[:, None]], dim=1)
    state.history = torch.where(live[:, None], shifted, state.history)
    state.steps = state.steps + live.to(torch.int64)
    state.finished = state.finished | (live & (tok == eos))
    return tok


def decode_k(state: DecodeState, logits_k: torch.Tensor, eos: int, cfg: TalkerSampling = TalkerSampling()
             ) -> torch.Tensor:
    """``engine/talker_sampler.py:252-254``."""
    return torch.stack([step(state, logits_k[i], eos, cfg) for i in range(logits_k.size(0))])
