"""Parity helpers shared by the GPU tests: oracle adapters and float-boundary classification.

A token or support difference between the HIP path and the oracle is accepted only where the two computations'
own rounding can move the decision, and the tolerance is derived per row, not fixed:

* the oracle (the reference's arithmetic) forms its CDF, its draw target and its top-p exclusive masses in float32;
  the classifier recomputes them exactly as the oracle does and measures their deviation from the float64 values
  on that row (``oracle_dev``);
* the HIP path forms each element's mass as exp(q - max) with the device ``expf`` (within 1 ulp) rounded to
  2^-42 fixed point and sums exactly, so its CDF deviates from float64 by at most 2^-23 of the total
  (``GPU_BOUND``).

A difference passes only when the float64 CDF at every step between the two tokens (or the exclusive mass at the
cut) lies within ``oracle_dev + GPU_BOUND`` of the decision point.  The workload tests additionally require that
no row needs this allowance on their seeds.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import extended_ref as ext

GPU_BOUND = 2.0 ** -23  # relative to the row's total mass


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


def draw_margin(x: torch.Tensor, u: float, a: int, b: int) -> tuple[float, float]:
    """(distance, tolerance) of the decision between tokens a != b drawn from processed row x with uniform u:
    the largest |cdf64[j] - u * total64| over the CDF steps j in [min(a, b), max(a, b)), relative to the total,
    and the tolerance the two computations' rounding allows on this row."""
    x64 = x.double()
    cdf64 = torch.cumsum(torch.softmax(x64, dim=-1), dim=-1)
    tot64 = float(cdf64[-1])
    t64 = u * tot64
    cdf32 = torch.softmax(x.float()[None], dim=-1).cumsum(dim=-1)[0]  # the oracle's own arithmetic
    t32 = float(torch.tensor(u, dtype=torch.float32) * cdf32[-1])
    lo, hi = min(a, b), max(a, b)
    dist = float((cdf64[lo:hi] - t64).abs().max()) / tot64
    finite = torch.isfinite(x64)
    oracle_dev = (float((cdf32.double() - cdf64)[finite].abs().max()) + abs(t32 - t64)) / tot64
    return dist, oracle_dev + GPU_BOUND


def token_at_boundary(x: torch.Tensor, u: float, a: int, b: int) -> bool:
    """Tokens a != b from the same processed row differ only by where u * total falls on a CDF step."""
    dist, tol = draw_margin(x, u, a, b)
    return dist <= tol


def support_at_boundary(pre: torch.Tensor, got: torch.Tensor, want: torch.Tensor, top_p: float, k: int,
                        full_norm: bool) -> bool:
    """Supports (finite entries) differ only in ranks whose exclusive mass sits at top_p within the rounding of
    the oracle's float32 masses (measured on this row) plus ``GPU_BOUND``."""
    diff = torch.nonzero(torch.isfinite(got) != torch.isfinite(want)).flatten()
    if diff.numel() == 0:
        return True
    x64 = pre.double()
    order = torch.argsort(-x64, stable=True)
    vals = x64[order][:k]
    z = torch.logsumexp(x64, 0) if full_norm else torch.logsumexp(vals, 0)
    probs = torch.exp(vals - z)
    above = torch.cumsum(probs, 0) - probs
    # the oracle's float32 exclusive masses (engine/talker_sampler.py:111-115, :127-132)
    v32 = pre.float()[order][:k]
    p32 = torch.exp(v32 - torch.logsumexp(pre.float(), 0)) if full_norm else torch.softmax(v32, 0)
    a32 = torch.cumsum(p32, 0) - p32
    fin = torch.isfinite(above) & torch.isfinite(a32.double())
    tol = float((a32.double() - above)[fin].abs().max()) + GPU_BOUND if bool(fin.any()) else GPU_BOUND
    rank = torch.empty_like(order)
    rank[order] = torch.arange(order.numel())
    for j in diff.tolist():
        r = int(rank[j])
        v = float(x64[j])
        # every rank holding this value (ties) is a candidate position of the boundary
        tied = torch.nonzero(vals == v).flatten()
        cands = tied.tolist() if tied.numel() else [r]
        if not any(abs(float(above[c]) - top_p) <= tol for c in cands if c < k):
            return False
    return True


def compare_group(name, got_tokens, got_proc, got_probs, ref: dict, rows: ext.Rows, prob_rtol: float) -> dict:
    """Asserts parity of one group; returns counts of exact and boundary-classified rows, and for each of the
    latter its row, distance and tolerance (``boundary_rows``)."""
    n_exact = n_tok_boundary = n_sup_boundary = 0
    notes = []
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
                notes.append(f"row {i}: support at the top-p cut")
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
            dist, tol = draw_margin(x, float(ref["uniforms"][i]), got_t, want_t)
            assert dist <= tol, (f"{name} row {i}: token {got_t} vs oracle {want_t} away from a CDF boundary "
                                 f"(distance {dist:.3g} of the total, tolerance {tol:.3g})")
            n_tok_boundary += 1
            notes.append(f"row {i}: token {got_t} vs {want_t}, distance {dist:.3g} <= {tol:.3g}")
        else:
            n_exact += 1
    return {"exact": n_exact, "token_boundary": n_tok_boundary, "support_boundary": n_sup_boundary,
            "boundary_rows": notes}


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
