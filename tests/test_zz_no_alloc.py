"""The allocation-free entry point (``mis_sample_static``): the library's own device workspace instead of the
caller's, called through the C-ABI and checked against ``mis_sample`` bit for bit on two calls in a row (the second
smaller), and its size limit reported as an error."""

from __future__ import annotations

import pytest
import torch

from mi355x_sampler import _lib
from mi355x_sampler import groups as G
from mi355x_sampler import workloads as W

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _gpu(gpu_lib):
    torch.cuda.set_device(0)
    yield


def _pair(wl):
    d = wl.to(DEV)
    kw = d.group_kwargs()
    a = G.RowGroup(d.logits, **kw, processed=True, probs=True)
    b = G.RowGroup(d.logits, **kw, processed=True, probs=True)
    return a, b


def test_static_workspace_matches_caller_workspace_twice():
    for name, make in (("thinker_b64", W.thinker_b64), ("talker_b8", lambda: W.talker_b8("hf"))):
        print(f"[gpu] static workspace: {name}", flush=True)
        wl = make()
        need = _lib.lib().mis_workspace_bytes((_lib.MisGroup * 1)(G.RowGroup(wl.to(DEV).logits,
                                                                               **wl.to(DEV).group_kwargs()).struct), 1)
        assert 0 < need <= _lib.MIS_STATIC_WORKSPACE_BYTES
        ref, got = _pair(wl)
        G.launch([ref])
        G.launch_static([got])
        torch.cuda.synchronize()
        assert torch.equal(got.tokens, ref.tokens), name
        assert torch.equal(got.processed, ref.processed), name
        assert torch.equal(got.probs, ref.probs), name


def test_static_workspace_rejects_what_does_not_fit():
    x = torch.zeros(1, 8, device=DEV)
    g = _lib.MisGroup()
    g.logits, g.logits_row_stride, g.dtype, g.vocab, g.rows = x.data_ptr(), W.THINKER_V, _lib.MIS_BF16, W.THINKER_V, 2000
    g.min_keep, g.temperature_value, g.top_p_value, g.repetition_value, g.top_k_value = 1, 1.0, 1.0, 1.0, 0
    need = _lib.lib().mis_workspace_bytes((_lib.MisGroup * 1)(g), 1)
    assert need > _lib.MIS_STATIC_WORKSPACE_BYTES
    with pytest.raises(_lib.SamplerError, match="static workspace"):
        _lib.sample_static([g], DEV)
