"""Counter hash and Philox restatements (numpy, C, torch) pinned against outside vectors."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import rng_ref
from oracle import talker_sampler_ref as ref

ORACLE = Path(__file__).resolve().parents[1] / "oracle"

# Random123 known-answer vectors for philox4x32-10 (kat_vectors: ctr[4], key[2] -> out[4]).
PHILOX_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.fixture(scope="module")
def crng():
    subprocess.run(["make", "-s", "-C", str(ORACLE)], check=True)
    lib = ctypes.CDLL(str(ORACLE / "_build" / "liboracle_rng.so"))
    lib.oracle_counter_uniform.restype = ctypes.c_float
    lib.oracle_counter_uniform.argtypes = [ctypes.c_int64, ctypes.c_int64]
    lib.oracle_philox_uniform.restype = ctypes.c_float
    lib.oracle_philox_uniform.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
    lib.oracle_philox4x32_10.argtypes = [ctypes.POINTER(ctypes.c_uint32)] * 3
    lib.oracle_lowbias32.restype = ctypes.c_uint32
    lib.oracle_lowbias32.argtypes = [ctypes.c_uint32]
    return lib


def test_counter_uniform_matches_reference_golden(golden_uniform):
    g = golden_uniform
    got = rng_ref.counter_uniform(g["seeds"], g["steps"])
    assert np.array_equal(got.view(np.int32), g["u"].view(np.int32))
    torch_got = ref.uniform(torch.from_numpy(g["seeds"]), torch.from_numpy(g["steps"])).numpy()
    assert np.array_equal(torch_got.view(np.int32), g["u"].view(np.int32))
    many = rng_ref.counter_uniform(np.full(4096, 9), np.arange(4096))
    assert np.array_equal(many, g["many_seed9"])


def test_counter_uniform_c_equals_numpy(crng, golden_uniform):
    g = golden_uniform
    for s, t, u in zip(g["seeds"], g["steps"], g["u"]):
        assert np.float32(crng.oracle_counter_uniform(int(s), int(t))) == u


def test_lowbias32_is_a_bijection_with_the_published_inverse():
    """lowbias32's inverse (modular inverses of the multipliers, xorshift inverses) recovers the input."""
    x = np.random.default_rng(0).integers(0, 2**32, size=4096, dtype=np.uint64)
    h = rng_ref.lowbias32(x).astype(np.uint64)

    def unxorshift(v, s):
        r = v.copy()
        for _ in range(32 // s + 1):
            r = v ^ (r >> np.uint64(s))
        return r & np.uint64(0xFFFFFFFF)

    inv1 = np.uint64(pow(0x7FEB352D, -1, 2**32))
    inv2 = np.uint64(pow(0x846CA68B, -1, 2**32))
    v = unxorshift(h, 16)
    v = (v * inv2) & np.uint64(0xFFFFFFFF)
    v = unxorshift(v, 15)
    v = (v * inv1) & np.uint64(0xFFFFFFFF)
    v = unxorshift(v, 16)
    assert np.array_equal(v, x)


def test_counter_uniform_reference_invariants():
    """``tests/engine/test_talker_sampler.py:92-98`` of the reference, on the restatement."""
    seeds = np.array([11, 12, 13, 2**40 + 5])
    u1 = rng_ref.counter_uniform(seeds, np.array([0, 1, 2, 3]))
    assert np.array_equal(u1, rng_ref.counter_uniform(seeds, np.array([0, 1, 2, 3])))
    assert u1.min() >= 0 and u1.max() < 1 and len(set(u1.tolist())) == 4
    many = rng_ref.counter_uniform(np.full(20000, 9), np.arange(20000))
    assert abs(float(many.mean()) - 0.5) < 0.01


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(ctr, key, want, crng):
    got = rng_ref.philox4x32_10(np.array(ctr, dtype=np.uint32), np.array(key, dtype=np.uint32))
    assert [int(v) for v in got] == want
    c = (ctypes.c_uint32 * 4)(*ctr)
    k = (ctypes.c_uint32 * 2)(*key)
    o = (ctypes.c_uint32 * 4)()
    crng.oracle_philox4x32_10(c, k, o)
    assert list(o) == want


def test_philox_matches_rocrand_header():
    """rocRAND's open-source philox4x32-10 (host side of its header) agrees on random counters and keys."""
    exe = ORACLE / "_build" / "rocrand_philox_kat"
    subprocess.run(["make", "-s", "-C", str(ORACLE), "rocrand"], check=True)
    rs = np.random.default_rng(5)
    ctr = rs.integers(0, 2**32, size=(64, 4), dtype=np.uint64).astype(np.uint32)
    key = rs.integers(0, 2**32, size=(64, 2), dtype=np.uint64).astype(np.uint32)
    lines = "\n".join(" ".join(str(int(v)) for v in list(c) + list(k)) for c, k in zip(ctr, key))
    out = subprocess.run([str(exe)], input=lines, capture_output=True, text=True, check=True).stdout.split()
    theirs = np.array([int(v) for v in out], dtype=np.uint64).reshape(64, 4).astype(np.uint32)
    ours = rng_ref.philox4x32_10(ctr, key)
    assert np.array_equal(ours, theirs)


def test_philox_uniform_c_equals_numpy(crng):
    rs = np.random.default_rng(9)
    for _ in range(200):
        s, t, r = (int(v) for v in rs.integers(-(2**63), 2**63 - 1, size=3))
        assert np.float32(crng.oracle_philox_uniform(s, t, r)) == rng_ref.philox_uniform(s, t, r)
