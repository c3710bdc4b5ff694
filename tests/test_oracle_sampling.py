"""Pin the oracle's sampling functions (CPU only).

Each check is independent of the oracle's formulas: pure-python brute force
on tiny vocabularies (sorting with explicit tie rules, fp64), closed forms of
the penalisers, an exhaustive 32-bit bitmask sweep, and the losslessness of
speculative rejection sampling (the emitted token is distributed exactly as
the target, checked by chi-square).
"""

import itertools
import math
import random

import pytest
import torch

from oracle import verify as ov


def brute_dist(logits, t, k, top_p, min_p):
    """fp64 pure-python target distribution with the documented tie rules."""
    v = len(logits)
    s = [x / t for x in logits]
    order = sorted(range(v), key=lambda i: (-s[i], i))  # value desc, index asc
    keep = order[:min(k, v)]
    m = s[keep[0]]
    e = {i: math.exp(s[i] - m) for i in keep}
    z = sum(e.values())
    p = {i: e[i] / z for i in keep}
    if top_p < 1.0:
        kept, cum = [], 0.0
        for i in keep:  # already in (value desc, index asc) order
            if cum > top_p:
                break
            kept.append(i)
            cum += p[i]
        zz = sum(p[i] for i in kept)
        p = {i: p[i] / zz for i in kept}
    if min_p > 0.0:
        pmax = max(p.values())
        p = {i: q for i, q in p.items() if q >= pmax * min_p}
        zz = sum(p.values())
        p = {i: q / zz for i, q in p.items()}
    out = [0.0] * v
    for i, q in p.items():
        out[i] = q
    return out


@pytest.mark.parametrize("seed", range(40))
def test_target_probs_matches_brute_force(seed):
    rng = random.Random(seed)
    v = rng.randint(2, 12)
    vals = [-2.0, -0.5, 0.0, 0.5, 1.0, 3.0]
    logits = [rng.choice(vals) for _ in range(v)]  # many exact ties
    t = rng.choice([0.5, 0.7, 1.0, 1.5])
    k = rng.choice([1, 2, 3, v, v + 5])
    top_p = rng.choice([0.3, 0.6, 0.9, 1.0])
    min_p = rng.choice([0.0, 0.0, 0.2, 0.5])
    ref = brute_dist(logits, t, k, top_p, min_p)
    got = ov.target_probs(torch.tensor([logits]), temperatures=torch.tensor([t]), top_ks=torch.tensor([k]),
                          top_ps=torch.tensor([top_p]), min_ps=torch.tensor([min_p]), rows_per_request=1)[0]
    # support identical, values within fp32 rounding
    assert [i for i, q in enumerate(ref) if q > 0] == [i for i, q in enumerate(got.tolist()) if q > 0], \
        (logits, t, k, top_p, min_p, ref, got.tolist())
    assert torch.allclose(got.double(), torch.tensor(ref, dtype=torch.float64), rtol=1e-5, atol=1e-7)


def test_topk_tie_rule_lowest_index():
    x = torch.tensor([[1.0, 3.0, 2.0, 3.0, 2.0, 2.0, 0.0]])
    vals, idx = ov.stable_topk(x, 4)
    assert idx.tolist() == [[1, 3, 2, 4]] and vals.tolist() == [[3.0, 3.0, 2.0, 2.0]]


def test_top_p_textbook():
    # p = [0.5, 0.3, 0.2]: top_p 0.6 keeps {0, 1} (exclusive sums 0, 0.5 <= 0.6)
    p = torch.tensor([[0.5, 0.3, 0.2]])
    out = ov.top_p_renorm(p, torch.tensor([0.6]))
    assert torch.allclose(out, torch.tensor([[0.625, 0.375, 0.0]]))


def test_penalty_closed_forms():
    vocab = 6
    hist = [torch.tensor([1, 1, 1, 4]), torch.tensor([], dtype=torch.int64)]
    add, scale = ov.penalty_tables(hist, vocab, [1.5, 2.0], [0.5, 0.5], [0.25, 0.25])
    # token 1 seen 3x: -(3*0.25) - 0.5 ; token 4 seen once: -0.25 - 0.5
    assert add[0].tolist() == [0.0, -1.25, 0.0, 0.0, -0.75, 0.0]
    assert scale[0].tolist() == [1.0, 1.5, 1.0, 1.0, 1.5, 1.0]
    assert add[1].abs().sum() == 0 and scale[1].eq(1).all()
    logits = torch.tensor([[2.0, 2.0, -1.0, 0.0, -3.0, 1.0]])
    x = logits.clone()
    ov.apply_verify_adjustments(x, additive=add[:1], scaling=scale[:1], rows_per_request=1)
    # true order: add then scale: token1: (2-1.25)/1.5 = 0.5 ; token4: (-3-0.75)*1.5 = -5.625
    assert x.tolist() == [[2.0, 0.5, -1.0, 0.0, -5.625, 1.0]]
    y = logits.clone()
    ov.apply_verify_adjustments(y, additive=add[:1], scaling=scale[:1], rows_per_request=1, verify_quirk=True)
    # quirk: pen = add scaled on its own sign: token1 -1.25*1.5, token4 -0.75*1.5
    assert y.tolist() == [[2.0, 2.0 - 1.875, -1.0, 0.0, -3.0 - 1.125, 1.0]]


def test_frequency_accumulates_like_repeated_fp32_adds():
    add, _ = ov.penalty_tables([torch.tensor([3] * 7)], 5, [1.0], [0.0], [0.1])
    acc = torch.tensor(0.0, dtype=torch.float32)
    for _ in range(7):
        acc = acc + torch.tensor(0.1, dtype=torch.float32)
    assert float(add[0, 3]) == float(-acc)


def test_bitmask_exhaustive_patterns():
    patterns = [0, 1, 0x80000000, 0xFFFFFFFF, 0x55555555, 0xAAAAAAAA] + [1 << i for i in range(32)]
    for pat in patterns:
        signed = pat - (1 << 32) if pat >= 1 << 31 else pat
        logits = torch.zeros(1, 40)
        ov.apply_token_bitmask(logits, torch.tensor([[signed, -1]], dtype=torch.int32))
        for v in range(32):
            bit = (pat >> v) & 1
            assert (logits[0, v] == float("-inf")) == (bit == 0), (hex(pat), v)
        assert torch.isfinite(logits[0, 32:40]).all()  # second word all ones
    # a narrower mask leaves the tail untouched
    logits = torch.zeros(1, 70)
    ov.apply_token_bitmask(logits, torch.tensor([[0, 0]], dtype=torch.int32))
    assert torch.isinf(logits[0, :64]).all() and torch.isfinite(logits[0, 64:]).all()


def test_acceptance_monotone_in_uniform():
    g = torch.Generator().manual_seed(0)
    b, gam, v = 32, 5, 9
    probs = torch.softmax(torch.randn(b, gam + 1, v, generator=g), -1)
    cand = torch.randint(0, v, (b, gam), generator=g)
    q = torch.rand(b, gam, generator=g)
    u1 = torch.rand(b, gam, generator=g)
    u2 = torch.minimum(u1 + 0.2, torch.ones_like(u1))
    d1 = ov.decide_acceptance(candidates=cand, sampled_q=q, target_probs=probs, uniforms=u1)
    d2 = ov.decide_acceptance(candidates=cand, sampled_q=q, target_probs=probs, uniforms=u2)
    assert (d2.lengths <= d1.lengths).all()


def test_sample_rows_from_probs_inverse_cdf():
    probs = torch.tensor([[0.1, 0.0, 0.6, 0.3]] * 5)
    u = torch.tensor([0.0, 0.0999, 0.1001, 0.7, 0.99])
    assert ov.sample_rows_from_probs(probs, u).tolist() == [0, 0, 2, 2, 3]
    assert ov.sample_rows_from_probs(torch.zeros(1, 4), torch.tensor([0.5])).tolist() == [3]


@pytest.mark.slow
def test_single_q_rejection_sampling_is_lossless():
    """With q the draft distribution and drafted tokens drawn from it, the first
    emitted token (accepted draft or resampled bonus) follows the target
    distribution p exactly (chi-square over 200k trials, V=6)."""
    g = torch.Generator().manual_seed(1)
    v, n = 6, 200_000
    target_logits = torch.tensor([1.0, 0.2, -0.5, 0.8, 0.0, -1.0])
    draft_logits = torch.tensor([0.1, 0.9, 0.3, -0.2, 0.5, 0.0])
    p = torch.softmax(target_logits, 0)
    q = torch.softmax(draft_logits, 0)
    drafted = torch.multinomial(q, n, replacement=True, generator=g)
    width = 2  # one drafted token + bonus row
    cand = torch.stack([torch.zeros(n, dtype=torch.long), drafted], 1)
    probs3 = p.expand(n, width, v)
    lens, bonus = ov.accept_single_q(
        candidates=cand, target_probs_3d=probs3, draft_q_rows_fn=lambda pos: q.expand(n, v),
        draft_token_probs=q[drafted][:, None], uniforms=torch.rand(n, 1, generator=g),
        final_uniforms=torch.rand(n, generator=g))
    first = torch.where(lens > 0, drafted, bonus)
    counts = torch.bincount(first, minlength=v).double()
    expected = p.double() * n
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 25.0, (chi2, counts, expected)  # 5 dof, p ~ 1e-4


def test_chain_sampling_matches_single_q_when_q_is_dense_softmax():
    g = torch.Generator().manual_seed(4)
    b, width, v = 16, 4, 7
    p3 = torch.softmax(torch.randn(b, width, v, generator=g), -1)
    q3 = torch.softmax(torch.randn(b, width - 1, v, generator=g), -1)
    cand = torch.randint(0, v, (b, width), generator=g)
    u = torch.rand(b, width - 1, generator=g)
    uf = torch.rand(b, generator=g)
    preds, aidx, anum = ov.chain_speculative_sampling(candidates=cand, uniform_samples=u, uniform_final=uf,
                                                      target_probs_3d=p3, draft_probs_3d=q3)
    lens, bonus = ov.accept_single_q(
        candidates=cand, target_probs_3d=p3, draft_q_rows_fn=lambda pos: q3[torch.arange(b), pos],
        draft_token_probs=q3.gather(2, cand[:, 1:, None]).squeeze(-1), uniforms=u, final_uniforms=uf)
    assert torch.equal(anum, lens)
    chain_bonus = preds[aidx[torch.arange(b), anum.long()].long()].long()
    # identical except where the residual mass is degenerate (not here) or a CDF tie
    assert (chain_bonus == bonus).float().mean() > 0.9


def test_chain_sampling_hand_cases():
    """reject_sampling.py:5-156 by hand: acceptance u*q < p on the drafted
    token's row, residual max(p - q, 0) (not normalised) with the first index
    whose running sum exceeds u_final * total, all-accepted draws from the
    last target row, a zero residual gives vocab-1, and the predicts /
    accept_index layout over retrive_index = arange(B*K)."""
    p = torch.tensor([[[0.3, 0.3, 0.4, 0.0], [0.1, 0.2, 0.3, 0.4], [0.1, 0.2, 0.3, 0.4]],
                      [[0.3, 0.3, 0.4, 0.0], [0.1, 0.2, 0.3, 0.4], [0.1, 0.2, 0.3, 0.4]],
                      [[0.5, 0.5, 0.0, 0.0], [0.1, 0.2, 0.3, 0.4], [0.1, 0.2, 0.3, 0.4]],
                      [[0.25, 0.25, 0.25, 0.25], [0.1, 0.2, 0.3, 0.4], [0.1, 0.2, 0.3, 0.4]]])
    q = torch.tensor([[[0.1, 0.5, 0.1, 0.3], [0.1, 0.2, 0.3, 0.4]],
                      [[0.1, 0.5, 0.1, 0.3], [0.1, 0.2, 0.3, 0.4]],
                      [[0.5, 0.5, 0.0, 0.0], [0.1, 0.2, 0.3, 0.4]],
                      [[0.25, 0.25, 0.25, 0.25], [0.1, 0.2, 0.3, 0.4]]])
    cand = torch.tensor([[9, 1, 3], [9, 1, 3], [9, 3, 0], [9, 2, 3]])
    u = torch.tensor([[0.8, 0.0], [0.8, 0.0], [0.5, 0.5], [0.9, 0.9]])
    uf = torch.tensor([0.5, 0.3, 0.7, 0.35])
    preds, aidx, anum = ov.chain_speculative_sampling(candidates=cand, uniform_samples=u, uniform_final=uf,
                                                      target_probs_3d=p, draft_probs_3d=q)
    # b0: 0.8*0.5 >= 0.3 rejects; residual [0.2, 0, 0.3, 0], 0.5*0.5 = 0.25 -> index 2
    # b1: same residual, 0.3*0.5 = 0.15 -> index 0
    # b2: token 3 has p = 0: rejected; residual all zero -> vocab-1
    # b3: q = p on both rows: both accepted (u*q < q); bonus from p[2] at 0.35 -> index 2
    assert anum.tolist() == [0, 0, 0, 2]
    bonus = preds[aidx[torch.arange(4), anum.long()].long()].tolist()
    assert bonus == [2, 0, 3, 2]
    assert aidx[3].tolist() == [9, 10, 11] and preds[9:12].tolist() == [2, 3, 2]


@pytest.mark.slow
def test_chain_sampling_is_lossless():
    """With one drafted token drawn from the dense q row, the first emitted
    token (the accepted draft, or the residual draw) follows p (chi-square,
    20k trials, V=6)."""
    g = torch.Generator().manual_seed(2)
    v, n = 6, 20_000
    p = torch.softmax(torch.tensor([1.0, 0.2, -0.5, 0.8, 0.0, -1.0]), 0)
    q = torch.softmax(torch.tensor([0.1, 0.9, 0.3, -0.2, 0.5, 0.0]), 0)
    drafted = torch.multinomial(q, n, replacement=True, generator=g)
    cand = torch.stack([torch.zeros(n, dtype=torch.long), drafted], 1)
    preds, aidx, anum = ov.chain_speculative_sampling(
        candidates=cand, uniform_samples=torch.rand(n, 1, generator=g), uniform_final=torch.rand(n, generator=g),
        target_probs_3d=p.expand(n, 2, v), draft_probs_3d=q.expand(n, 1, v))
    first = preds[aidx[:, 0].long()].long()
    counts = torch.bincount(first, minlength=v).double()
    expected = p.double() * n
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 25.0, (chi2, counts, expected)  # 5 dof, p ~ 1e-4


def test_finalize_outputs_hand_case():
    cand = torch.tensor([[5, 11, 12, 13], [7, 21, 22, 23]])
    out, committed, nxt = ov.finalize_verify_outputs(cand, torch.tensor([1, 3], dtype=torch.int32),
                                                     torch.tensor([99, 98]), torch.tensor([100, 200]))
    # request 0 accepts one draft (11), bonus at column 1; request 1 accepts all three
    assert out.tolist() == [[11, 99, 13, 0], [21, 22, 23, 98]]
    assert committed.tolist() == [2, 4] and nxt.tolist() == [102, 204]


# ---------------------------------------------------------------- proposal step

def test_exponential_race_samples_p():
    """argmax_v p_v / E_v with E ~ Exp(1) draws v with probability p_v
    (chi-square, 60k rows, V=6), and q is p at the drawn token."""
    g = torch.Generator().manual_seed(5)
    n, v = 60_000, 6
    logits = torch.tensor([1.0, 0.2, -0.5, 0.8, 0.0, -1.0]).expand(n, v)
    t = torch.full((n,), 0.9)
    noise = torch.empty(n, v).exponential_(1, generator=g)
    tokens, q, valid = ov.sample_step_tokens_with_q(logits, t, noise)
    p = torch.softmax(logits[0].double() / 0.9, 0)
    assert bool(valid.all())
    counts = torch.bincount(tokens, minlength=v).double()
    chi2 = float(((counts - p * n) ** 2 / (p * n)).sum())
    assert chi2 < 25.0, (chi2, counts, p * n)
    assert torch.allclose(q.double(), p[tokens], rtol=1e-6)


def test_sample_step_tile_combine_equals_whole_row():
    """The reference's tile form (sample_step_tokens_with_q.py:72-187: tile max
    m_t, sums and keys relative to m_t, combined with exp(m_t - m)) equals the
    whole-row softmax form in fp64."""
    g = torch.Generator().manual_seed(6)
    rows, vocab, tile = 5, 3000, 1024
    x = 3 * torch.randn(rows, vocab, generator=g, dtype=torch.float64)
    x[:, 1500:2700] = float("-inf")       # a tile with no finite entry, a partly masked tile
    t = torch.tensor([0.5, 0.8, 1.0, 1.3, 2.0], dtype=torch.float64)
    noise = torch.empty(rows, vocab, dtype=torch.float64).exponential_(1, generator=g)
    tok_ref, q_ref, _ = ov.sample_step_tokens_with_q(x, t, noise, compute_dtype=torch.float64)
    s = x / t[:, None]
    for r in range(rows):
        tm, ts, tk, ti, tn = [], [], [], [], []
        for c0 in range(0, vocab, tile):
            seg, nz = s[r, c0:c0 + tile], noise[r, c0:c0 + tile]
            m = seg.max()
            e = torch.exp(seg - m) if torch.isfinite(m) else torch.zeros_like(seg)
            keys = torch.where(torch.isfinite(m) & torch.ones_like(seg, dtype=torch.bool), e / nz,
                               torch.full_like(seg, -1.0))
            k = int(torch.argmax(keys))
            tm.append(m), ts.append(e.sum()), tk.append(keys[k]), ti.append(c0 + k), tn.append(e[k])
        gm = max(tm)
        resc = [torch.exp(m - gm) if torch.isfinite(m) else torch.tensor(0.0, dtype=torch.float64) for m in tm]
        den = sum(a * b for a, b in zip(ts, resc))
        rk = [k * r_ if torch.isfinite(m) else -1.0 for k, r_, m in zip(tk, resc, tm)]
        best = max(range(len(rk)), key=lambda i: (float(rk[i]), -ti[i]))
        assert ti[best] == int(tok_ref[r])
        assert abs(float(tn[best] * resc[best] / den) - float(q_ref[r])) <= 1e-6 * float(q_ref[r])


def test_sample_step_invalid_rows_and_ties():
    inf = float("inf")
    x = torch.tensor([[0.0, 1.0, 1.0, -inf],       # tie between 1 and 2 with equal noise -> 1
                      [0.0, float("nan"), 1.0, 2.0],  # NaN logit: invalid
                      [0.0, inf, 1.0, 2.0],        # +inf logit: invalid
                      [-inf, -inf, -inf, -inf],    # no finite entry: invalid
                      [0.0, 1.0, 2.0, 3.0],        # T = 0: invalid
                      [0.0, 1.0, 2.0, 3.0],        # zero noise at a finite entry: invalid
                      [0.0, 1.0, 2.0, -inf]])      # zero noise at a masked entry: valid
    t = torch.tensor([1.0, 1.0, 1.0, 1.0, 0.0, 1.0, 1.0])
    noise = torch.ones(7, 4)
    noise[5, 2] = 0.0
    noise[6, 3] = 0.0
    tokens, q, valid = ov.sample_step_tokens_with_q(x, t, noise)
    assert valid.tolist() == [True, False, False, False, False, False, True]
    assert tokens.tolist() == [1, 0, 0, 0, 0, 0, 2]
    assert bool(torch.isnan(q[1:6]).all())
    assert abs(float(q[0]) - float(torch.softmax(torch.tensor([0.0, 1.0, 1.0]), 0)[1])) < 1e-7


def test_assign_fixed_verify_cache_locs_hand_case():
    rtt = torch.zeros(3, 8, dtype=torch.int32)
    locs = torch.tensor([[10, 11, 12], [20, 21, 22]])
    out = ov.assign_fixed_verify_cache_locs(torch.tensor([2, 0]), rtt, torch.tensor([1, 6]), torch.tensor([2, 3]),
                                            locs)
    # request 0 -> slot 2, positions 1-2; request 1 -> slot 0, positions 6-7 (8 is past the map)
    assert out[2].tolist() == [0, 10, 11, 0, 0, 0, 0, 0]
    assert out[0].tolist() == [0, 0, 0, 0, 0, 0, 20, 21]
    assert int(out[1].abs().sum()) == 0 and int(rtt.abs().sum()) == 0


# ---------------------------------------------------------------------------
# split engine (src/longspark/engine/sampling.py:19-57): hand-worked cases
# ---------------------------------------------------------------------------

def _split_decision(cand, q, u, p):
    return ov.decide_acceptance(candidates=cand, sampled_q=q, target_probs=p, uniforms=u)


def test_decide_acceptance_hand_cases():
    from tests import split_cases as sc
    p, cand, q, u, exp = sc.decide_case()
    d = _split_decision(cand, q, u, p)
    assert d.lengths.tolist() == exp["lengths"]
    assert d.rejected_rows.tolist() == exp["rejected_rows"]
    assert d.rejection_positions.tolist() == exp["rejection_positions"]
    for b, j in enumerate(exp["target_row_index"]):
        assert torch.equal(d.target_rows[b], p[b, j]), b


def test_finish_sampling_hand_cases():
    from tests import split_cases as sc
    p, cand, q, u, _ = sc.decide_case()
    d = _split_decision(cand, q, u, p)
    q_rows, uf, expected = sc.finish_case()
    assert ov.finish_sampling(d, q_rows, uf).tolist() == expected


def test_finish_sampling_mass_threshold_and_clamp():
    from tests import split_cases as sc
    cases, (clamp_row, u_clamp, tok_clamp) = sc.threshold_cases()
    for label, p_row, q_row, uf, tok in cases:
        p = torch.stack([p_row, p_row])[None]             # [1, gamma + 1 = 2, V]
        d = _split_decision(torch.tensor([[0]]), torch.tensor([[1.0]]), torch.tensor([[0.5]]), p)
        assert d.lengths.tolist() == [0] and d.rejected_rows.tolist() == [0], label
        assert ov.finish_sampling(d, q_row[None], torch.tensor([uf])).tolist() == [tok], label
    p = torch.stack([torch.tensor([0.0, 1.0, 0.0, 0.0]), clamp_row])[None]
    d = _split_decision(torch.tensor([[1]]), torch.tensor([[0.5]]), torch.tensor([[0.5]]), p)
    assert d.lengths.tolist() == [1] and d.rejected_rows.numel() == 0
    assert ov.finish_sampling(d, torch.zeros(0, 4), torch.tensor([u_clamp])).tolist() == [tok_clamp]
