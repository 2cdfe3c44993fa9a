"""Shared test set-up: import paths, the ``gpu`` marker, golden fixture loaders.

``-m "not gpu"`` tests run anywhere (oracle, golden vectors, host logic, the
C-ABI library's exports).  ``-m gpu`` tests need an MI355X and call the HIP
path through the C-ABI library.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "inferrsi-minicpm-o-4.5-npu_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"

for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)

os.environ.setdefault("OMP_NUM_THREADS", "8")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP path through the C-ABI library)")


def load_npz(name: str) -> dict:
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_case(store: dict, name: str) -> dict:
    pre = name + "."
    return {k[len(pre):]: v for k, v in store.items() if k.startswith(pre)}


@pytest.fixture(scope="session")
def golden_uniform() -> dict:
    return load_npz("uniform.npz")


@pytest.fixture(scope="session")
def golden_processed() -> dict:
    return load_npz("processed.npz")


@pytest.fixture(scope="session")
def golden_streams() -> dict:
    return load_npz("streams.npz")


@pytest.fixture(scope="session")
def gpu_lib():
    """The HIP library, loaded; skips when there is no GPU (these tests carry the ``gpu`` marker)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from mi355x_sampler import _lib

    return _lib.lib()
