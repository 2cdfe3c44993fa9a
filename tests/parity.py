"""Parity helpers shared by the GPU tests: oracle adapters and float-boundary classification.

A token or support difference between the HIP path and the oracle is accepted
only when the oracle's own float64 arithmetic puts the decision within a
relative 1e-5 of its boundary (the inverse-CDF target lands on a CDF step, or
a rank's exclusive mass is at top_p); every other difference fails.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import extended_ref as ext

BOUNDARY_TOL = 1e-5


def oracle_rows(wl, *, zero_disables=True, one_disables=True, alpha="exact", **over) -> ext.Rows:
    """The workload (CPU tensors) as an oracle group."""
    p = wl.params
    kw = dict(logits=wl.logits, temperature=p["temperature"], top_k=p["top_k"], top_p=p["top_p"],
              repetition=p["repetition"], presence=p["presence"], frequency=p["frequency"],
              history=None if wl.history is None else wl.history.clone(), mask=wl.allowed,
              seeds=wl.seeds, steps=wl.steps.clone(), row_ids=wl.row_ids, eos=wl.eos, semantics=wl.semantics,
              min_keep=wl.min_keep, rng=wl.rng, top_k_zero_disables=zero_disables,
              top_p_one_disables=one_disables, alpha=alpha)
    kw.update(over)
    return ext.Rows(**kw)


def token_at_boundary(x: torch.Tensor, u: float, a: int, b: int, tol: float = BOUNDARY_TOL) -> bool:
    """Tokens a != b from the same processed row differ only by where u * total falls on a CDF step."""
    x64 = x.double()
    p = torch.softmax(x64, dim=-1)
    cdf = torch.cumsum(p, dim=-1)
    t = u * float(cdf[-1])
    lo, hi = min(a, b), max(a, b)
    return abs(float(cdf[lo]) - t) < tol and abs(float(cdf[hi - 1]) - t) < tol


def support_at_boundary(pre: torch.Tensor, got: torch.Tensor, want: torch.Tensor, top_p: float, k: int,
                        full_norm: bool, tol: float = BOUNDARY_TOL) -> bool:
    """Supports (finite entries) differ only in ranks whose exclusive mass sits at top_p (float64)."""
    diff = torch.nonzero(torch.isfinite(got) != torch.isfinite(want)).flatten()
    if diff.numel() == 0:
        return True
    x64 = pre.double()
    order = torch.argsort(-x64, stable=True)
    vals = x64[order][:k]
    z = torch.logsumexp(x64, 0) if full_norm else torch.logsumexp(vals, 0)
    probs = torch.exp(vals - z)
    above = torch.cumsum(probs, 0) - probs
    rank = torch.empty_like(order)
    rank[order] = torch.arange(order.numel())
    for j in diff.tolist():
        r = int(rank[j])
        v = float(x64[j])
        # every rank holding this value (ties) is a candidate position of the boundary
        tied = torch.nonzero(vals == v).flatten()
        cands = tied.tolist() if tied.numel() else [r]
        if not any(abs(float(above[c]) - top_p) < tol for c in cands if c < k):
            return False
    return True


def compare_group(name, got_tokens, got_proc, got_probs, ref: dict, rows: ext.Rows, prob_rtol: float) -> dict:
    """Asserts parity of one group; returns counts of exact and boundary-classified rows."""
    n_exact = n_tok_boundary = n_sup_boundary = 0
    toks = got_tokens.cpu()
    for i in range(rows.rows):
        want_x = ref["processed"][i]
        want_t = int(ref["tokens"][i])
        got_t = int(toks[i])
        sup_ok = True
        if got_proc is not None:
            gx = got_proc[i].cpu()
            same_support = torch.equal(torch.isfinite(gx), torch.isfinite(want_x))
            if not same_support:
                pre = _prefilter(rows, i)
                k = ext.resolve_k(int(rows.top_k[i]), rows.min_keep, rows.vocab, rows.top_k_zero_disables)
                sup_ok = support_at_boundary(pre, gx, want_x, float(rows.top_p[i]), k, rows.semantics == "hf")
                assert sup_ok, f"{name} row {i}: support differs away from the top-p boundary"
                n_sup_boundary += 1
            both = torch.isfinite(gx) & torch.isfinite(want_x)
            assert torch.equal(gx[both], want_x[both]), f"{name} row {i}: processed values differ"
        if got_probs is not None and got_proc is not None and torch.equal(torch.isfinite(got_proc[i].cpu()),
                                                                          torch.isfinite(want_x)):
            gp = got_probs[i].cpu().double()
            wp = ref["probs"][i].double()
            np.testing.assert_allclose(gp.numpy(), wp.numpy(), rtol=prob_rtol, atol=1e-9,
                                       err_msg=f"{name} row {i}: probabilities")
        if got_t != want_t:
            x = got_proc[i].cpu() if got_proc is not None else want_x
            assert got_t >= 0 and want_t >= 0, f"{name} row {i}: PAD mismatch {got_t} vs {want_t}"
            assert token_at_boundary(x, float(ref["uniforms"][i]), got_t, want_t), \
                f"{name} row {i}: token {got_t} vs oracle {want_t} away from a CDF boundary"
            n_tok_boundary += 1
        else:
            n_exact += 1
    return {"exact": n_exact, "token_boundary": n_tok_boundary, "support_boundary": n_sup_boundary}


def _prefilter(rows: ext.Rows, i: int) -> torch.Tensor:
    """Row i before the top-k / top-p filter (same penalties, mask, temperature)."""
    import copy

    r = copy.copy(rows)
    r.top_k = torch.zeros_like(rows.top_k)
    r.top_p = torch.ones_like(rows.top_p)
    r.top_k_zero_disables = True
    r.top_p_one_disables = True
    x, _ = ext.process_row(r, i)
    return x
