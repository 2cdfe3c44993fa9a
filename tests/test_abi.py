"""The C-ABI library: loads without a GPU, exports every declared entry point, validates arguments on the host."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from mi355x_sampler import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "mi355x_sampler.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(mis_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_declares_the_bound_entry_points():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_and_struct_layout(lib):
    assert lib.mis_version() == _lib.MIS_ABI_VERSION
    assert lib.mis_sizeof_group() == ctypes.sizeof(_lib.MisGroup)


def _group(**kw) -> _lib.MisGroup:
    g = _lib.MisGroup()
    g.logits = 0x1000
    g.logits_row_stride = 8
    g.dtype = _lib.MIS_F32
    g.vocab = 8
    g.rows = 2
    g.min_keep = 1
    for k, v in kw.items():
        setattr(g, k, v)
    return g


@pytest.mark.parametrize("field,value,needle", [
    ("dtype", 7, "dtype"), ("vocab", 0, "vocab"), ("semantics", 5, "semantics"), ("min_keep", 0, "min_keep"),
    ("rng", 9, "RNG"), ("eos", 8, "eos"), ("logits_row_stride", 4, "stride"), ("history_len", 70000, "history_len"),
])
def test_invalid_arguments_are_rejected_before_launch(lib, field, value, needle):
    g = _group(**{field: value})
    rc = lib.mis_sample(ctypes.byref(g), 1, None, 0, None)
    assert rc == _lib.MIS_E_ARG
    assert needle in lib.mis_last_error().decode()
    assert lib.mis_workspace_bytes(ctypes.byref(g), 1) == 0


def test_workspace_too_small_is_rejected(lib):
    g = _group()
    need = lib.mis_workspace_bytes(ctypes.byref(g), 1)
    assert need > 0
    assert lib.mis_sample(ctypes.byref(g), 1, 0x2000, need - 1, None) == _lib.MIS_E_WORKSPACE
    assert lib.mis_sample(ctypes.byref(g), 0, None, 0, None) == _lib.MIS_E_ARG


def test_unsupported_vocabulary_is_reported(lib):
    g = _group(vocab=10_000_000, logits_row_stride=10_000_000)
    assert lib.mis_sample(ctypes.byref(g), 1, None, 0, None) == _lib.MIS_E_UNSUPPORTED


def test_uniform_rejects_bad_mode(lib):
    assert lib.mis_uniform(None, None, None, 4, 3, 0x1000, None) == _lib.MIS_E_ARG
    assert lib.mis_uniform(None, None, None, 0, 0, None, None) == 0


def test_python_layer_refuses_cpu_tensors():
    import torch

    from mi355x_sampler import groups

    with pytest.raises(ValueError, match="GPU"):
        groups.RowGroup(torch.zeros(2, 8))
