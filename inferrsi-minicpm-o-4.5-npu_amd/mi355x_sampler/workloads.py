"""Synthetic sampling workloads (seeded, CPU-generated): the Talker and Thinker sample steps.

* ``talker_b1``  — Talker audio-token step: batch 1, vocab 6,562 fp32 logits ~N(0, 3^2); T 0.8, top-k 20,
  top-p 0.8, repetition 1.05 over a 64-token history of uniform ids; Philox seed 1234, step 0.
* ``talker_b8``  — batch 8, vocab 6,562 fp32 ~N(0, 3^2) with 5 spike tokens per row at +8; T in [0.6, 1.0],
  top-k 20, top-p 0.8, repetition 1.05 over 256-token histories; bitmask disallowing the last 2 ids.
* ``thinker_b8`` — Thinker text step: batch 8, vocab 151,748 bf16 ~N(0, 2.5^2) plus a Zipf(s = 1.1) rank bias;
  T 0.7, top-p 0.8, top-k 100; presence 0.5 and frequency 0.2 over 2,048-token histories (and a greedy variant).
* ``thinker_b64`` — batch 64, vocab 151,748 bf16, per-row top-k in {0, 20, 100, 1000}, top-p in
  {0.5, 0.8, 0.95, 1.0}, T in [0.3, 1.2]; repetition 1.1 over 4,096-token histories; bitmask with 30% of ids
  disallowed (at least one allowed per row).
* ``mixed`` — 64 ``thinker_b64`` rows + 64 ``talker_b8``-style rows in one launch, advanced over many steps with
  the histories appended in place.

Generators: ``torch.Generator().manual_seed(1000 + n)`` for logits, histories, spikes and masks.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

TALKER_V, TALKER_EOS = 6562, 6561
THINKER_V = 151748
PHILOX_SEED = 1234


@dataclass
class Workload:
    """One group of rows, on the CPU; ``to(device)`` moves every tensor."""

    name: str
    logits: torch.Tensor
    params: dict                      # temperature / top_k / top_p / repetition / presence / frequency tensors [B]
    history: torch.Tensor             # [B, W] int32 (ids; PAD = -1)
    allowed: torch.Tensor | None      # [B, ceil(V/32)] int32 words or None
    seeds: torch.Tensor
    steps: torch.Tensor
    row_ids: torch.Tensor
    semantics: str = "omni"
    min_keep: int = 1
    eos: int = -1
    rng: str = "philox"
    extra: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return int(self.logits.shape[0])

    @property
    def vocab(self) -> int:
        return int(self.logits.shape[1])

    def algorithmic_bytes(self) -> int:
        """Logits once + packed mask once + history ids as int32, per step."""
        per_row = self.vocab * self.logits.element_size() + 4 * self.history.shape[1]
        if self.allowed is not None:
            per_row += 4 * ((self.vocab + 31) // 32)
        return per_row * self.rows

    def to(self, device) -> "Workload":
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        return Workload(self.name, mv(self.logits), {k: mv(v) for k, v in self.params.items()}, mv(self.history),
                        mv(self.allowed), mv(self.seeds), mv(self.steps), mv(self.row_ids), self.semantics,
                        self.min_keep, self.eos, self.rng, dict(self.extra))

    def group_kwargs(self) -> dict:
        """Keyword arguments of ``groups.RowGroup`` (everything but the logits)."""
        return dict(**self.params, history=self.history, allowed=self.allowed, seeds=self.seeds, steps=self.steps,
                    row_ids=self.row_ids, semantics=self.semantics, min_keep=self.min_keep, eos=self.eos,
                    rng=self.rng)


def pack_allowed(allowed: torch.Tensor) -> torch.Tensor:
    """[B, V] bool → [B, ceil(V/32)] int32 words (bit j of word w = token 32w + j)."""
    b, v = allowed.shape
    nw = (v + 31) // 32
    padded = torch.zeros(b, nw * 32, dtype=torch.int64)
    padded[:, :v] = allowed.to(torch.int64)
    words = (padded.reshape(b, nw, 32) << torch.arange(32, dtype=torch.int64)).sum(-1)
    return torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)


def _params(b, temperature, top_k, top_p, repetition=1.0, presence=0.0, frequency=0.0) -> dict:
    full = lambda v, dt: v.to(dt) if isinstance(v, torch.Tensor) else torch.full((b,), v, dtype=dt)  # noqa: E731
    return dict(temperature=full(temperature, torch.float32), top_k=full(top_k, torch.int32),
                top_p=full(top_p, torch.float32), repetition=full(repetition, torch.float32),
                presence=full(presence, torch.float32), frequency=full(frequency, torch.float32))


def _rng_keys(b: int, step: int = 0):
    return (torch.full((b,), PHILOX_SEED, dtype=torch.int64), torch.full((b,), step, dtype=torch.int64),
            torch.arange(b, dtype=torch.int64))


def talker_b1(semantics: str = "hf") -> Workload:
    g = torch.Generator().manual_seed(1001)
    logits = torch.randn(1, TALKER_V, generator=g) * 3
    hist = torch.randint(0, TALKER_V, (1, 64), generator=g, dtype=torch.int64).to(torch.int32)
    seeds, steps, rids = _rng_keys(1)
    return Workload("talker_b1", logits, _params(1, 0.8, 20, 0.8, 1.05), hist, None, seeds, steps, rids,
                    semantics=semantics, min_keep=3 if semantics == "hf" else 1, eos=TALKER_EOS)


def talker_b8(semantics: str = "hf", step: int = 1) -> Workload:
    g = torch.Generator().manual_seed(1002)
    b = 8
    logits = torch.randn(b, TALKER_V, generator=g) * 3
    for i in range(b):
        logits[i, torch.randint(0, TALKER_V, (5,), generator=g)] += 8
    hist = torch.randint(0, TALKER_V, (b, 256), generator=g, dtype=torch.int64).to(torch.int32)
    allowed = torch.ones(b, TALKER_V, dtype=torch.bool)
    allowed[:, TALKER_V - 2:] = False
    seeds, steps, rids = _rng_keys(b, step)
    temps = torch.linspace(0.6, 1.0, b)
    return Workload("talker_b8", logits, _params(b, temps, 20, 0.8, 1.05), hist, pack_allowed(allowed), seeds,
                    steps, rids, semantics=semantics, min_keep=3 if semantics == "hf" else 1, eos=TALKER_EOS)


def _thinker_logits(b: int, g: torch.Generator) -> torch.Tensor:
    logits = torch.randn(b, THINKER_V, generator=g) * 2.5
    perm = torch.randperm(THINKER_V, generator=g)
    bias = torch.empty(THINKER_V)
    bias[perm] = -1.1 * torch.log(torch.arange(1, THINKER_V + 1, dtype=torch.float32))
    return (logits + bias).to(torch.bfloat16)


def thinker_b8(greedy: bool = False) -> Workload:
    g = torch.Generator().manual_seed(1003)
    b = 8
    logits = _thinker_logits(b, g)
    hist = torch.randint(0, THINKER_V, (b, 2048), generator=g, dtype=torch.int64).to(torch.int32)
    seeds, steps, rids = _rng_keys(b)
    t = 0.0 if greedy else 0.7
    return Workload("thinker_b8_greedy" if greedy else "thinker_b8", logits,
                    _params(b, t, 100, 0.8, 1.0, 0.5, 0.2), hist, None, seeds, steps, rids)


def thinker_b64() -> Workload:
    g = torch.Generator().manual_seed(1004)
    b = 64
    logits = _thinker_logits(b, g)
    hist = torch.randint(0, THINKER_V, (b, 4096), generator=g, dtype=torch.int64).to(torch.int32)
    allowed = torch.rand(b, THINKER_V, generator=g) >= 0.3
    allowed[:, 0] |= ~allowed.any(dim=1)
    i = torch.arange(b)
    top_k = torch.tensor([0, 20, 100, 1000], dtype=torch.int32)[i % 4]
    top_p = torch.tensor([0.5, 0.8, 0.95, 1.0], dtype=torch.float32)[(i // 4) % 4]
    temps = (0.3 + 0.9 * i.to(torch.float64) / 63).to(torch.float32)
    seeds, steps, rids = _rng_keys(b)
    return Workload("thinker_b64", logits, _params(b, temps, top_k, top_p, 1.1), hist, pack_allowed(allowed), seeds,
                    steps, rids)


def mixed() -> tuple[Workload, Workload]:
    """The Thinker batch-64 group and a 64-row Talker group (talker_b8's parameters, tiled), in one launch."""
    big = thinker_b64()
    g = torch.Generator().manual_seed(1005)
    b = 64
    logits = torch.randn(b, TALKER_V, generator=g) * 3
    for r in range(b):
        logits[r, torch.randint(0, TALKER_V, (5,), generator=g)] += 8
    hist = torch.randint(0, TALKER_V, (b, 256), generator=g, dtype=torch.int64).to(torch.int32)
    allowed = torch.ones(b, TALKER_V, dtype=torch.bool)
    allowed[:, TALKER_V - 2:] = False
    seeds, steps, rids = _rng_keys(b)
    rids = rids + 64
    temps = torch.linspace(0.6, 1.0, 8).repeat(8)
    small = Workload("talker_b64", logits, _params(b, temps, 20, 0.8, 1.05), hist, pack_allowed(allowed), seeds,
                     steps, rids, semantics="hf", min_keep=3, eos=TALKER_EOS)
    return big, small


CONFIGS = {
    "talker_b1": talker_b1,
    "talker_b8": talker_b8,
    "thinker_b8": thinker_b8,
    "thinker_b64": thinker_b64,
}


def zipf_check() -> float:
    """Sum of the Zipf bias weights (a sanity figure for the generator; e^bias = r^-1.1)."""
    return sum(math.exp(-1.1 * math.log(r)) for r in range(1, 1000))
