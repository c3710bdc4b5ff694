"""Tolerance contract of the summary-state parity tests: 1e-5 relative.

The expected state comes from the oracle's formula evaluated in fp64.  "1e-5
relative" is taken in the sense that is meaningful for a weighted sum:
  * an output entry ``sum_i w_i x_i`` (the prior output and the new value
    rows, with non-negative softmax weights w_i) must lie within 1e-5 of the
    magnitude of its summands, ``sum_i w_i |x_i|``.  That magnitude is the
    same merge applied to ``|prior|`` and ``|v|`` (the weights do not change).
    An entry whose summands cancel has no meaningful relative error of its
    own, so its bound is the summands' scale, never a fixed absolute floor;
  * an LSE is the logarithm of a mass, so it must lie within 1e-5 in
    absolute terms: that is 1e-5 relative error of the mass ``exp(lse)``.
Both sides must be -inf together (an empty state).
"""

from __future__ import annotations

import torch

from oracle import summary as osm

REL = 1e-5


def merged(prior_out, prior_lse, prior_mag, query, keys, values, lens, scale, softcap=0.0):
    """One fp64 merge step: returns (out, lse, magnitude) after folding the
    first ``lens[b]`` rows of ``keys`` / ``values`` ``[B, W, Hkv, D]``."""
    sc = osm.position_scores(query, keys, scale, softcap, dtype=torch.float64)
    dim = values.shape[-1]
    # one merge over [values | |values|]: the weights are the same for both halves
    both, lse = osm.merge_accepted_positions(torch.cat([prior_out.double(), prior_mag.double()], -1), prior_lse,
                                             sc, torch.cat([values.double(), values.double().abs()], -1), lens,
                                             dtype=torch.float64)
    return both[..., :dim], lse, both[..., dim:]


def check(out, lse, ref_out, ref_lse, mag, rel=REL, what="summary state"):
    """Assert the contract above; returns the worst output and LSE errors (in
    units of the bound) for the log."""
    out, lse = out.double(), lse.double()
    err = (out - ref_out).abs()
    bound = rel * mag
    ok = err <= bound
    worst_o = float((err / bound.clamp_min(1e-300)).max()) if err.numel() else 0.0
    if not bool(ok.all()):
        i = int((~ok).flatten().nonzero()[0])
        raise AssertionError(f"{what}: output entry {i} differs by {float(err.flatten()[i]):.3e}, bound "
                             f"{float(bound.flatten()[i]):.3e} (1e-5 of summand magnitude "
                             f"{float(mag.flatten()[i]):.3e}); {int((~ok).sum())} entries out of bound")
    both_inf = torch.isneginf(lse) & torch.isneginf(ref_lse)
    dl = torch.where(both_inf, torch.zeros_like(lse), (lse - ref_lse).abs())
    worst_l = float(dl.max() / rel) if dl.numel() else 0.0
    if not bool((dl <= rel).all()):
        i = int((dl > rel).flatten().nonzero()[0])
        raise AssertionError(f"{what}: LSE entry {i} differs by {float(dl.flatten()[i]):.3e} "
                             f"(kernel {float(lse.flatten()[i])}, fp64 {float(ref_lse.flatten()[i])})")
    print(f"{what}: worst output error {worst_o:.3f} of the bound, worst LSE error {worst_l:.3f} of the bound",
          flush=True)
    return worst_o, worst_l
