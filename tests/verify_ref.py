"""Shared helpers for the stochastic-verify parity tests: run the CPU oracle on
the same inputs and classify disagreements against the tie contract.

Contract (bit-exact except near-ties): accepted lengths and sampled tokens
must match the oracle exactly unless the decision that differs is within
1e-6 of its threshold -- an acceptance test ``u*q < p`` with
``|u*q - p| <= 1e-6``, an inverse-CDF draw with ``|u*total - cdf_v| <=
1e-6 * total``, or a top-p / min-p support boundary within 1e-6.  Target
probabilities of the drafted tokens must match within 1e-5 relative.
"""

from __future__ import annotations

import torch

from oracle import verify as ov

TIE = 1e-6


def oracle_inputs(d, *, verify_quirk=False, with_penalties=True, with_mask=True):
    """CPU copies of a stochastic_inputs() dict plus the oracle penalty tensors."""
    c = {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in d.items()}
    p = d["params"]
    c["params"] = type(p)(*(t.cpu() for t in (p.temperatures, p.top_ks, p.top_ps, p.min_ps)))
    vocab = c["logits"].shape[1]
    add = scale = None
    if with_penalties and "history" in c:
        add, scale = ov.penalty_tables([h for h in c["history"]], vocab, c["repetition"], c["presence"],
                                       c["frequency"])
    c["additive"], c["scaling"] = add, scale
    c["bitmask"] = c.get("vocab_mask") if with_mask else None
    c["verify_quirk"] = verify_quirk
    return c


def run_oracle(c, *, draft_params=True):
    p = c["params"]
    kw = {}
    if draft_params:
        kw = dict(draft_top_ks=p.top_ks, draft_top_ps=p.top_ps, draft_min_ps=p.min_ps)
    lens, bonus, probs = ov.verify_sample(
        logits=c["logits"], candidates=c["candidates"].long(), draft_logits=c["draft_logits"],
        draft_token_probs=c["draft_token_probs"], uniforms=c["uniforms"], final_uniforms=c["final_uniforms"],
        temperatures=p.temperatures, top_ks=p.top_ks, top_ps=p.top_ps, min_ps=p.min_ps,
        additive=c["additive"], scaling=c["scaling"], bitmask=c["bitmask"], verify_quirk=c["verify_quirk"],
        **kw)
    return lens, bonus, probs


def _support_boundary_near(c, probs_row_logits, temperature, top_k, top_p, min_p):
    """True when a top-p or min-p cut of this row lies within TIE of its limit."""
    if top_p >= 1.0 and min_p <= 0.0:
        return False
    x = probs_row_logits.double() / float(temperature)
    vocab = x.numel()
    if top_k < vocab:
        v, _ = torch.sort(x, descending=True)
        v = v[:top_k]
    else:
        v, _ = torch.sort(x, descending=True)
    p = torch.softmax(v, 0)
    near = False
    n = p.numel()
    if top_p < 1.0:
        excl = torch.cumsum(p, 0) - p
        near |= bool(((excl - top_p).abs() <= TIE).any())
        keep = excl <= top_p
        n = int(keep.sum())
    if min_p > 0.0:
        q = p[:n] / p[:n].sum()
        near |= bool(((q - q[0] * min_p).abs() <= TIE * q[0]).any())
    return near


def cdf_tie(vals, u, tok_a, tok_b) -> bool:
    """Two inverse-CDF draws from ``vals`` (first index whose running sum
    exceeds ``u * total``) that differ only by rounding: the running sum at the
    earlier of the two tokens lies within TIE * total of ``u * total``."""
    vals = vals.double()
    cdf = torch.cumsum(vals, 0)
    total = float(cdf[-1])
    t = min(int(tok_a), int(tok_b))
    if total <= 0.0 or t < 0 or t >= vals.numel():
        return False
    return abs(float(cdf[t]) - float(u) * total) <= TIE * total


def bonus_row(probs_row, q_row, rejected: bool, single_q: bool):
    """The distribution the bonus is drawn from: p, or max(p - q, 0) after a
    rejection (single-q acceptance falls back to p below 1e-8 of mass)."""
    if not rejected:
        return probs_row.double()
    r = (probs_row.double() - q_row.double()).clamp_min(0.0)
    if single_q and float(r.sum()) <= ov.RESIDUAL_MASS_EPS:
        return probs_row.double()
    return r


def classify(c, lens_k, bonus_k, lens_r, bonus_r, probs_r, p_cand_k=None, draft_params=True):
    """Returns (mismatched_requests, exempt_requests, messages)."""
    bsz, width = c["candidates"].shape
    g = width - 1
    cand = c["candidates"].long()
    u, q = c["uniforms"], c["draft_token_probs"]
    logits = c["logits"].float().clone()
    ov.apply_verify_adjustments(logits, additive=c["additive"], scaling=c["scaling"], bitmask=c["bitmask"],
                                rows_per_request=width, verify_quirk=c["verify_quirk"])
    p = c["params"]
    bad, exempt, msgs = [], [], []
    for b in range(bsz):
        same = int(lens_k[b]) == int(lens_r[b]) and int(bonus_k[b]) == int(bonus_r[b])
        pc_ok = True
        if p_cand_k is not None:
            ref = probs_r[b, torch.arange(g), cand[b, 1:]]
            pc_ok = bool(torch.allclose(p_cand_k[b], ref, rtol=1e-5, atol=1e-9))
        if same and pc_ok:
            continue
        reasons = []
        L = int(min(int(lens_k[b]), int(lens_r[b])))
        for j in range(min(max(int(lens_k[b]), int(lens_r[b])) + 1, g)):
            pr = float(probs_r[b, j, cand[b, j + 1]])
            if abs(float(u[b, j]) * float(q[b, j]) - pr) <= TIE:
                reasons.append(f"accept tie at j={j}")
        for j in range(0, min(L + 1, width)):
            row = logits[b * width + j]
            if _support_boundary_near(c, row, p.temperatures[b], int(p.top_ks[b]), float(p.top_ps[b]),
                                      float(p.min_ps[b])):
                reasons.append(f"support boundary tie at row {j}")
        if same and not pc_ok and not reasons:
            bad.append(b)
            msgs.append(f"b={b}: p_cand differs: kernel {p_cand_k[b].tolist()} ref "
                        f"{probs_r[b, torch.arange(g), cand[b, 1:]].tolist()}")
            continue
        if not same and not reasons and int(lens_k[b]) == int(lens_r[b]):
            # inverse-CDF tie of the final draw, on the row the bonus is drawn from
            lr = int(lens_r[b])
            q_row = None
            if lr < g:
                kw = dict(top_ks=p.top_ks, top_ps=p.top_ps, min_ps=p.min_ps) if draft_params else {}
                q_row = ov.draft_q_rows(c["draft_logits"][b:b + 1], torch.tensor([lr]),
                                        temperatures=p.temperatures[b:b + 1],
                                        **{k: v[b:b + 1] for k, v in kw.items()})[0]
            vals = bonus_row(probs_r[b, lr], q_row, lr < g, single_q=True)
            if cdf_tie(vals, float(c["final_uniforms"][b]), int(bonus_k[b]), int(bonus_r[b])):
                reasons.append("cdf tie")
        if reasons:
            exempt.append(b)
            msgs.append(f"b={b}: exempt ({', '.join(reasons)})")
        elif not same:
            bad.append(b)
            msgs.append(f"b={b}: kernel (L={int(lens_k[b])}, tok={int(bonus_k[b])}) vs oracle "
                        f"(L={int(lens_r[b])}, tok={int(bonus_r[b])})")
    return bad, exempt, msgs
