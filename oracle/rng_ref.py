"""Counter-based uniforms restated in numpy uint32 arithmetic (oracle; test infrastructure only).

* ``lowbias32`` — C. Wellons' 32-bit integer finalizer ("hash-prospector",
  the ``lowbias32`` entry: shifts 16/15/16, multipliers 0x7feb352d and
  0x846ca68b), as used by ``engine/talker_sampler.py:60-67``.
* ``counter_uniform`` — the reference's (seed, step) chain
  (``engine/talker_sampler.py:70-76``): three finalizer rounds folding in the
  seed's low word, its high word ^ 0x9E3779B9, and the step's low word
  ^ 0x632BE5AB; the top 24 bits become a float in [0, 1).
* ``philox4x32_10`` — Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
  easy as 1, 2, 3" (SC'11): multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key
  increments 0x9E3779B9 / 0xBB67AE85, ten rounds.  Pinned by the Random123
  known-answer vectors and by rocRAND's open-source header
  (``tests/test_oracle_rng.py``).
* ``philox_uniform`` — the build's draw key for the Philox mode: key = the
  64-bit seed (low word, high word), counter = (step low, step high, row id
  low, row id high); output word 0's top 24 bits become the uniform.  There is
  no reference counterpart (the reference has only the counter hash).
"""

from __future__ import annotations

import numpy as np

_U32 = np.uint32
_U64 = np.uint64


def lowbias32(x) -> np.ndarray:
    x = np.asarray(x, dtype=_U64) & _U64(0xFFFFFFFF)
    x ^= x >> _U64(16)
    x = (x * _U64(0x7FEB352D)) & _U64(0xFFFFFFFF)
    x ^= x >> _U64(15)
    x = (x * _U64(0x846CA68B)) & _U64(0xFFFFFFFF)
    x ^= x >> _U64(16)
    return x.astype(_U32)


def _split(v) -> tuple[np.ndarray, np.ndarray]:
    u = np.asarray(v, dtype=np.int64).astype(_U64)
    return (u & _U64(0xFFFFFFFF)).astype(_U32), (u >> _U64(32)).astype(_U32)


def _to_unit(word: np.ndarray) -> np.ndarray:
    return (np.asarray(word, dtype=_U32) >> _U32(8)).astype(np.float32) * np.float32(1.0 / (1 << 24))


def counter_hash(seeds, steps) -> np.ndarray:
    s_lo, s_hi = _split(seeds)
    t_lo, _ = _split(steps)
    h = lowbias32(s_lo)
    h = lowbias32(h ^ s_hi ^ _U32(0x9E3779B9))
    return lowbias32(h ^ t_lo ^ _U32(0x632BE5AB))


def counter_uniform(seeds, steps) -> np.ndarray:
    return _to_unit(counter_hash(*np.broadcast_arrays(np.asarray(seeds), np.asarray(steps))))


_PH_M0, _PH_M1 = 0xD2511F53, 0xCD9E8D57
_PH_W0, _PH_W1 = 0x9E3779B9, 0xBB67AE85


def philox4x32_10(ctr, key) -> np.ndarray:
    """Vectorised over leading axes: ``ctr`` [..., 4], ``key`` [..., 2] uint32 → [..., 4] uint32."""
    c = [np.asarray(ctr, dtype=_U64)[..., i] for i in range(4)]
    k0, k1 = (np.asarray(key, dtype=_U64)[..., i] for i in range(2))
    m = _U64(0xFFFFFFFF)
    for rnd in range(10):
        if rnd:
            k0 = (k0 + _U64(_PH_W0)) & m
            k1 = (k1 + _U64(_PH_W1)) & m
        p0 = _U64(_PH_M0) * c[0]
        p1 = _U64(_PH_M1) * c[2]
        c = [(p1 >> _U64(32)) ^ c[1] ^ k0, p1 & m, (p0 >> _U64(32)) ^ c[3] ^ k1, p0 & m]
    return np.stack(c, axis=-1).astype(_U32)


def philox_uniform(seeds, steps, row_ids) -> np.ndarray:
    seeds, steps, row_ids = np.broadcast_arrays(np.asarray(seeds), np.asarray(steps), np.asarray(row_ids))
    s_lo, s_hi = _split(seeds)
    t_lo, t_hi = _split(steps)
    r_lo, r_hi = _split(row_ids)
    out = philox4x32_10(np.stack([t_lo, t_hi, r_lo, r_hi], axis=-1), np.stack([s_lo, s_hi], axis=-1))
    return _to_unit(out[..., 0])
