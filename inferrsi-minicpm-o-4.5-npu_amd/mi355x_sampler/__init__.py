"""MI355X-native token sampler for the MiniCPM-o 4.5 Thinker / Talker decode loops.

* ``talker_sampler`` — drop-in for the reference module ``engine/talker_sampler.py``.
* ``groups`` — per-row parameters, several vocabularies in one launch (``RowGroup``, ``launch``, ``greedy``).
* ``_lib`` — the ctypes binding of ``libmi355x_sampler.so`` (C-ABI: ``include/mi355x_sampler.h``).

Everything runs on the GPU through the HIP library; importing works without a
GPU, calling does not.
"""

from . import groups, talker_sampler  # noqa: F401
from .groups import RowGroup, greedy, launch, sample  # noqa: F401
