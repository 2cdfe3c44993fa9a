"""CPU oracle for the token-sampling path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference sampler
(``engine/talker_sampler.py``) and the build-defined extensions of the same
pipeline (per-row parameters, presence/frequency penalties, the packed
allowed-token bitmask, Philox4x32-10 draws, ``top_k = 0`` / ``top_p = 1``
sentinels).  It is the checker that the HIP path is compared with, and the
CPU baseline that the benchmark times beside the GPU.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from here.  The shipped sampler never calls
into this package: it has no CPU fallback and fails loudly when its HIP
library is missing.

Modules:

* ``talker_sampler_ref`` — eager-torch restatement of the reference module,
  name for name (``uniform``, ``repetition_penalty``, the four filters,
  ``processed_logits``, ``draw``, ``step``, ``decode_k`` …).
* ``rng_ref`` — numpy-uint32 restatements of the lowbias32 counter hash and of
  Philox4x32-10, plus ``rng.c`` (the same two generators in plain C, built by
  ``oracle/Makefile`` into ``oracle/_build/liboracle_rng.so``).
* ``extended_ref`` — the per-row extended pipeline (one row at a time, built
  from the functions of ``talker_sampler_ref``).

Pins (how each function is checked against something other than itself) are
listed in the module docstrings and exercised by ``tests/test_oracle_*.py``.
"""
