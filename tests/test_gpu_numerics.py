"""The kernel's division (``div_rn`` in ``csrc/elem.h``: one double product, IEEE division below 2^-125) against
IEEE float division, on the device, over every divisor mantissa of two binades and numerators at the range edges;
the device's IEEE quotients are themselves checked against numpy's float32 division.

Divisors in [1, 2) cover the temperatures and repetition factors of practice; divisors in [4, 8) include the even
integers 4 and 6, for which a subnormal quotient can fall exactly on a rounding midpoint (x = 3 * 2^-149, d = 6
gives 2^-150).  Numerators: subnormal, at the normal edge, mid-range and near the top of the float range.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
PROBE = Path(__file__).resolve().parent / "native" / "libdivprobe.so"


@pytest.fixture(scope="module")
def probe(gpu_lib):
    if not PROBE.exists():
        pytest.fail(f"{PROBE} is missing: run __graft_entry__.build()")
    h = ctypes.CDLL(str(PROBE))
    h.divprobe_run.restype = ctypes.c_int
    h.divprobe_run.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                               ctypes.c_void_p]
    return h


def _run(h, x: np.ndarray, d: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    xt, dt = torch.from_numpy(x).to(DEV), torch.from_numpy(d).to(DEV)
    a, b = torch.empty_like(xt), torch.empty_like(xt)
    assert h.divprobe_run(xt.data_ptr(), dt.data_ptr(), xt.numel(), a.data_ptr(), b.data_ptr(),
                          torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    return a.cpu().numpy(), b.cpu().numpy()


def _numerators(rs, n: int) -> list[np.ndarray]:
    sub = (rs.integers(1, 1 << 23, size=n, dtype=np.uint32)).view(np.float32)          # subnormal
    edge = ((rs.integers(1, 3, size=n, dtype=np.uint32) << 23)
            | rs.integers(0, 1 << 23, size=n, dtype=np.uint32)).view(np.float32)        # [2^-126, 2^-124)
    mid = ((rs.integers(107, 147, size=n, dtype=np.uint32) << 23)
           | rs.integers(0, 1 << 23, size=n, dtype=np.uint32)).view(np.float32)         # [2^-20, 2^20)
    top = ((rs.integers(253, 255, size=n, dtype=np.uint32) << 23)
           | rs.integers(0, 1 << 23, size=n, dtype=np.uint32)).view(np.float32)         # [2^126, 2^128)
    sign = np.where(rs.integers(0, 2, size=n) == 1, np.float32(-1), np.float32(1))
    return [v * sign for v in (sub, edge, mid, top)]


@pytest.mark.parametrize("exponent", [127, 129])  # divisors in [1, 2) and [4, 8)
def test_division_equals_ieee_for_every_divisor_mantissa(probe, exponent):
    print(f"[gpu] div_rn sweep, divisor exponent {exponent - 127}", flush=True)
    d = ((np.uint32(exponent) << np.uint32(23)) | np.arange(1 << 23, dtype=np.uint32)).view(np.float32)
    rs = np.random.default_rng(exponent)
    for band, x in zip(("subnormal", "edge", "mid", "top"), _numerators(rs, d.size)):
        rn, ieee = _run(probe, x, d)
        bad = np.nonzero(rn.view(np.uint32) != ieee.view(np.uint32))[0]
        assert bad.size == 0, (band, [(float(x[i]), float(d[i]), float(rn[i]), float(ieee[i])) for i in bad[:5]])
        with np.errstate(all="ignore"):
            host = x / d  # numpy float32 division: IEEE, round to nearest even, subnormals kept
        assert np.array_equal(ieee.view(np.uint32), host.view(np.uint32)), band


def test_subnormal_midpoint_ties_and_specials(probe):
    """Quotients exactly on a subnormal rounding midpoint (x = (d / 2) * (2 j + 1) * 2^-149 for even integer d),
    signed zeros, infinities and NaN."""
    xs, ds = [], []
    for dv in (4.0, 6.0, 10.0, 12.0, 14.0, 6.0 * 1024, 2.0 ** 20 * 3):
        for j in range(0, 40):
            m = int(dv // 2) * (2 * j + 1)
            if m < (1 << 23):
                xs.append(np.uint32(m).view(np.float32))
                ds.append(dv)
    x = np.array(xs, dtype=np.float32)
    d = np.array(ds, dtype=np.float32)
    x = np.concatenate([x, -x, np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0], dtype=np.float32)])
    d = np.concatenate([d, d, np.array([0.7, 0.7, 0.7, 1.3, 0.9, np.float32(3e38)], dtype=np.float32)])
    rn, ieee = _run(probe, x, d)
    with np.errstate(all="ignore"):
        host = x / d
    nan = np.isnan(host)
    assert np.array_equal(np.isnan(rn), nan) and np.array_equal(np.isnan(ieee), nan)
    assert np.array_equal(rn[~nan].view(np.uint32), host[~nan].view(np.uint32))
    assert np.array_equal(ieee[~nan].view(np.uint32), host[~nan].view(np.uint32))
