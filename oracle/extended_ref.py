"""Per-row extended sampling pipeline on the CPU (oracle; test infrastructure only).

The reference (``engine/talker_sampler.py``) takes one ``TalkerSampling`` per
call.  The decode loops this path serves batch rows with their own
parameters, so the build defines a per-row pipeline that reduces to the
reference's exactly when every row carries the same parameters.  This module
restates it one row at a time on top of ``talker_sampler_ref``.

Row semantics (build-defined where the reference is silent, vLLM conventions):

``omni`` order (``engine/talker_sampler.py:142-147`` extended):
    x = float(logits); EOS censored (-inf) while ``step < min_new``;
    repetition penalty ``alpha = rep**n`` (``x<0 ? x*alpha : x/alpha``);
    then ``x -= frequency*n``; then ``x -= presence*(n>0)`` (vLLM's order);
    then the allowed-token bitmask (bit j of word w is token 32w+j, 1 =
    allowed); then ``x / T``; then the reference's fused top-k → top-p filter
    with the top-k softmax normaliser.
``hf`` order (``engine/talker_sampler.py:148-156`` extended):
    x = float(logits) / T; rows with ``step > 0`` get the penalties as above;
    the bitmask applies to every row; rows with ``step > 0`` get the
    reference's fused top-p → top-k filter with the full-vocabulary
    normaliser; then the EOS censor.
Both: forced EOS at ``step >= max_new - 1`` (``engine/talker_sampler.py:157-158``).

Sentinels: ``T <= 0`` ⇒ greedy (first index of the maximum of the penalised,
masked logits; no temperature, no filters).  With ``top_k_zero_disables``,
``top_k <= 0`` ⇒ k = V (no top-k); otherwise ``k = min(max(top_k,
min_keep), V)`` as in the reference.  With ``top_p_one_disables``,
``top_p >= 1`` ⇒ no top-p (the reference instead evaluates its formula at
p = 1).  ``alpha`` is ``torch.pow`` as in the reference (``alpha="torch"``)
or the correctly rounded ``rep**n`` (``alpha="exact"``, float64 power rounded
to float32 — the GPU's default).

Pins: with uniform parameters every row equals ``talker_sampler_ref``'s
``processed_logits`` (tested); presence/frequency are closed forms checked
against a loop over the history; the bitmask is checked against a boolean
mask; Philox against Random123 / rocRAND (``tests/test_oracle_*.py``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import rng_ref
from . import talker_sampler_ref as ref

PAD = ref.PAD


@dataclass
class Rows:
    """One group of rows sharing a vocabulary, dtype and semantics (all CPU tensors)."""

    logits: torch.Tensor                      # [B, V] float32 / bfloat16
    temperature: torch.Tensor                 # [B] float32
    top_k: torch.Tensor                       # [B] int
    top_p: torch.Tensor                       # [B] float32
    repetition: torch.Tensor                  # [B] float32
    presence: torch.Tensor                    # [B] float32
    frequency: torch.Tensor                   # [B] float32
    history: torch.Tensor | None = None       # [B, W] int, PAD (<0) where empty
    mask: torch.Tensor | None = None          # [B, ceil(V/32)] int32 words (uint32 bit patterns)
    seeds: torch.Tensor | None = None         # [B] int64
    steps: torch.Tensor | None = None         # [B] int64
    row_ids: torch.Tensor | None = None       # [B] int64 (Philox counter words 2-3)
    uniforms: torch.Tensor | None = None      # [B] float32 injected draws
    active: torch.Tensor | None = None        # [B] bool
    finished: torch.Tensor | None = None      # [B] bool
    eos: int = -1
    min_new_tokens: int = 0
    max_new_tokens: int = 0                   # 0 = no forced EOS
    semantics: str = "omni"
    min_keep: int = 1
    rng: str = "counter"                      # "counter" | "philox"
    top_k_zero_disables: bool = True
    top_p_one_disables: bool = True
    alpha: str = "exact"                      # "exact" | "torch"
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return int(self.logits.shape[0])

    @property
    def vocab(self) -> int:
        return int(self.logits.shape[1])


def resolve_k(top_k: int, min_keep: int, vocab: int, zero_disables: bool) -> int:
    if zero_disables and top_k <= 0:
        return vocab
    return min(max(int(top_k), int(min_keep)), vocab)


def unpack_mask(words: torch.Tensor, vocab: int) -> torch.Tensor:
    """[B, ceil(V/32)] int32 words → [B, V] bool (bit j of word w ↔ token 32w + j, LSB first)."""
    w = words.to(torch.int64) & 0xFFFFFFFF
    bits = (w[:, :, None] >> torch.arange(32, dtype=torch.int64)) & 1
    return bits.reshape(words.shape[0], -1)[:, :vocab].bool()


def pack_mask(allowed: torch.Tensor) -> torch.Tensor:
    """[B, V] bool → [B, ceil(V/32)] int32 (inverse of ``unpack_mask``)."""
    b, v = allowed.shape
    nw = (v + 31) // 32
    padded = torch.zeros(b, nw * 32, dtype=torch.int64)
    padded[:, :v] = allowed.to(torch.int64)
    words = (padded.reshape(b, nw, 32) << torch.arange(32, dtype=torch.int64)).sum(-1)
    return torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)


def history_counts(hist_row: torch.Tensor, vocab: int) -> torch.Tensor:
    """[W] ids → [V] float32 counts; PAD (< 0) and ids >= V are empty slots."""
    h = hist_row[None].to(torch.int64)
    h = torch.where(h < vocab, h, torch.full_like(h, PAD))
    return ref.token_counts(h, vocab)[0]


def exact_alpha(rep: float, counts: torch.Tensor) -> torch.Tensor:
    """Correctly rounded ``fp32(rep) ** n`` (float64 power, one rounding to float32)."""
    with np.errstate(over="ignore", under="ignore"):
        a = np.power(np.float64(np.float32(rep)), counts.double().numpy())
    return torch.from_numpy(a.astype(np.float32))


def penalties(x: torch.Tensor, counts: torch.Tensor, rep: float, presence: float, frequency: float,
              alpha: str) -> torch.Tensor:
    """One row: count-powered repetition penalty, then frequency, then presence (float32 throughout)."""
    if alpha == "torch":
        a = torch.pow(torch.full_like(x, rep), counts)
    else:
        a = exact_alpha(rep, counts)
    x = torch.where(x < 0, x * a, x / a)
    f = torch.tensor(frequency, dtype=torch.float32)
    x = x - f * counts
    p = torch.tensor(presence, dtype=torch.float32)
    return x - p * (counts > 0).to(torch.float32)


def _filter_row(x: torch.Tensor, k: int, top_p: float, min_keep: int, skip_p: bool, semantics: str) -> torch.Tensor:
    xr = x[None]
    if skip_p:
        kth = torch.topk(xr, k, dim=-1).values[..., -1:]
        return xr.masked_fill(xr < kth, float("-inf"))[0]
    if semantics == "omni":
        return ref.top_k_top_p_filter(xr, k, top_p, min_keep)[0]
    return ref.top_p_top_k_filter(xr, top_p, k, min_keep)[0]


def row_uniform(g: Rows, i: int) -> float:
    if g.uniforms is not None:
        return float(g.uniforms[i])
    seed = int(g.seeds[i]) if g.seeds is not None else 0
    st = int(g.steps[i]) if g.steps is not None else 0
    if g.rng == "philox":
        rid = int(g.row_ids[i]) if g.row_ids is not None else 0
        return float(rng_ref.philox_uniform(seed, st, rid))
    return float(rng_ref.counter_uniform(seed, st))


def process_row(g: Rows, i: int) -> tuple[torch.Tensor, bool]:
    """Processed (filtered) logits of row ``i`` and whether the row is greedy."""
    v = g.vocab
    x = g.logits[i].float().clone()
    step = int(g.steps[i]) if g.steps is not None else 0
    temp = float(g.temperature[i])
    greedy = temp <= 0
    k = resolve_k(int(g.top_k[i]), g.min_keep, v, g.top_k_zero_disables)
    top_p = float(np.float32(g.top_p[i]))
    skip_p = g.top_p_one_disables and top_p >= 1.0
    if g.history is not None:
        counts = history_counts(g.history[i], v)
    else:
        counts = torch.zeros(v)
    allowed = unpack_mask(g.mask[i:i + 1], v)[0] if g.mask is not None else None
    is_eos = torch.arange(v) == g.eos
    censor = g.eos >= 0 and step < g.min_new_tokens
    pen = (float(g.repetition[i]), float(g.presence[i]), float(g.frequency[i]))
    tdiv = torch.tensor(1.0 if greedy else temp, dtype=torch.float32)
    if g.semantics == "omni":
        if censor:
            x = x.masked_fill(is_eos, float("-inf"))
        x = penalties(x, counts, *pen, g.alpha)
        if allowed is not None:
            x = x.masked_fill(~allowed, float("-inf"))
        x = x / tdiv
        if not greedy:
            x = _filter_row(x, k, top_p, g.min_keep, skip_p, "omni")
    elif g.semantics == "hf":
        x = x / tdiv
        later = step > 0
        if later:
            x = penalties(x, counts, *pen, g.alpha)
        if allowed is not None:
            x = x.masked_fill(~allowed, float("-inf"))
        if later and not greedy:
            x = _filter_row(x, k, top_p, g.min_keep, skip_p, "hf")
        if censor:
            x = x.masked_fill(is_eos, float("-inf"))
    else:
        raise ValueError(f"unknown semantics {g.semantics!r}")
    if g.eos >= 0 and g.max_new_tokens > 0 and step >= g.max_new_tokens - 1:
        x = torch.where(is_eos, torch.zeros_like(x), torch.full_like(x, float("-inf")))
    return x, greedy


def sample_rows(g: Rows, *, update_state: bool = False, history_mode: str = "window",
                history_head: torch.Tensor | None = None, with_probs: bool = True) -> dict:
    """Processed logits, filtered probabilities and tokens of every row of ``g``.

    ``update_state`` advances the decode state in place like
    ``engine/talker_sampler.py:244-248`` (history shift-append, or ring write at
    ``history_head`` for ``history_mode="ring"``; steps; finished).
    """
    b, v = g.rows, g.vocab
    processed = torch.empty(b, v)
    probs = torch.empty(b, v)
    tokens = torch.empty(b, dtype=torch.int64)
    uniforms = torch.empty(b)
    for i in range(b):
        x, greedy = process_row(g, i)
        processed[i] = x
        if with_probs:
            probs[i] = torch.softmax(x, dim=-1)
        u = row_uniform(g, i)
        uniforms[i] = u
        if greedy:
            tokens[i] = int(torch.argmax(x))
        else:
            tokens[i] = int(ref.draw(x[None], None, None, uniform_values=torch.tensor([u], dtype=torch.float32))[0])
    live = torch.ones(b, dtype=torch.bool)
    if g.active is not None:
        live &= g.active.bool()
    if g.finished is not None:
        live &= ~g.finished.bool()
    tokens = torch.where(live, tokens, torch.full_like(tokens, PAD))
    if update_state:
        for i in range(b):
            if not live[i]:
                continue
            if g.history is not None:
                if history_mode == "ring":
                    w = g.history.shape[1]
                    g.history[i, int(history_head[i]) % w] = tokens[i]
                    history_head[i] += 1
                else:
                    g.history[i, :-1] = g.history[i, 1:].clone()
                    g.history[i, -1] = tokens[i]
            if g.steps is not None:
                g.steps[i] += 1
            if g.finished is not None and int(tokens[i]) == g.eos:
                g.finished[i] = True
    return {"processed": processed, "probs": probs, "tokens": tokens, "uniforms": uniforms, "live": live}


def greedy_argmax(logits: torch.Tensor) -> torch.Tensor:
    """Thinker greedy (``engine/runtime/thinker_decode.py:107``; ``backend_npu.py:890``): first index of the max."""
    return torch.argmax(logits.float(), dim=-1)
