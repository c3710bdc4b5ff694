"""Split-engine verification on dense target probabilities and the
fixed-width verify outputs, on the GPU vs the CPU oracle.

Cases: 7 drafted positions over vocabularies of 1,000 and 151,936 with
random and forced-accept proposals; int32 and int64 candidates; rejected and
accepted requests in one batch; a degenerate residual (q = p, mass below
1e-8, which falls back to p); uniforms near 0 and near 1; finalize outputs
with every accept length and mixed integer dtypes.  Lengths, target rows and
outputs are bit-exact; sampled tokens are exact except CDF-boundary draws
within 1e-6.
"""

import pytest
import torch

from oracle import verify as ov
from longspark_amd import verify

pytestmark = pytest.mark.gpu


def make_case(batch, gamma, vocab, seed, force_accept=0.0):
    g = torch.Generator().manual_seed(seed)
    p = torch.softmax(2.0 * torch.randn(batch, gamma + 1, vocab, generator=g), -1)
    cand = torch.multinomial(p[:, :gamma].reshape(-1, vocab), 1, generator=g).view(batch, gamma)
    q = torch.rand(batch, gamma, generator=g) * p[:, :gamma].gather(2, cand[..., None]).squeeze(-1) * 2.5
    if force_accept:
        q = torch.where(torch.rand(batch, gamma, generator=g) < force_accept, torch.zeros_like(q), q)
    u = torch.rand(batch, gamma, generator=g)
    return p, cand, q, u


def cdf_boundary_ok(probs_row, u, tok_a, tok_b):
    if tok_a == tok_b:
        return True
    cdf = probs_row.double().cumsum(0)
    lo = min(tok_a, tok_b)
    return abs(float(cdf[lo]) - float(u)) <= 1e-6


@pytest.mark.parametrize("vocab,batch,cand_dtype", [(1000, 32, torch.int64), (151936, 4, torch.int32)])
def test_decide_and_finish(dev, vocab, batch, cand_dtype):
    print(f"split verify V={vocab} B={batch} cand={cand_dtype}", flush=True)
    gamma = 7
    p, cand, q, u = make_case(batch, gamma, vocab, seed=vocab + batch, force_accept=0.3)
    d = verify.decide_acceptance(candidates=cand.to(cand_dtype).to(dev), sampled_q=q.to(dev),
                                 target_probs=p.to(dev), uniforms=u.to(dev))
    ref = ov.decide_acceptance(candidates=cand, sampled_q=q, target_probs=p, uniforms=u)
    torch.cuda.synchronize()
    assert torch.equal(d.lengths.cpu(), ref.lengths)
    assert torch.equal(d.rejected_rows.cpu(), ref.rejected_rows)
    assert torch.equal(d.rejection_positions.cpu(), ref.rejection_positions)
    assert torch.equal(d.target_rows.cpu(), ref.target_rows)
    g = torch.Generator().manual_seed(7)
    qrows = torch.softmax(2.0 * torch.randn(ref.rejected_rows.numel(), vocab, generator=g), -1)
    uf = torch.rand(batch, generator=g)
    uf[0] = 0.0
    uf[-1] = 0.999999
    tok = verify.finish_sampling(d, qrows.to(dev), uniforms=uf.to(dev)).cpu()
    tok_ref = ov.finish_sampling(ref, qrows, uf)
    probs = ref.target_rows.clone()
    if ref.rejected_rows.numel():
        res = (ref.target_rows[ref.rejected_rows] - qrows).clamp_min(0)
        probs[ref.rejected_rows] = res / res.sum(-1, keepdim=True).clamp_min(1e-30)
    for b in range(batch):
        assert cdf_boundary_ok(probs[b], uf[b], int(tok[b]), int(tok_ref[b])), (b, tok[b], tok_ref[b])


def test_degenerate_residual_falls_back_to_target(dev):
    batch, gamma, vocab = 4, 7, 500
    p, cand, q, u = make_case(batch, gamma, vocab, seed=3)
    q = torch.ones_like(q)  # every request rejects at position 0
    d = verify.decide_acceptance(candidates=cand.to(dev), sampled_q=q.to(dev), target_probs=p.to(dev),
                                 uniforms=u.to(dev))
    ref = ov.decide_acceptance(candidates=cand, sampled_q=q, target_probs=p, uniforms=u)
    assert torch.equal(d.lengths.cpu(), torch.zeros(batch, dtype=torch.int64))
    qrows = ref.target_rows.clone()  # q = p: the residual is zero
    uf = torch.tensor([0.1, 0.5, 0.9, 0.3])
    tok = verify.finish_sampling(d, qrows.to(dev), uniforms=uf.to(dev)).cpu()
    tok_ref = ov.finish_sampling(ref, qrows, uf)
    for b in range(batch):
        assert cdf_boundary_ok(ref.target_rows[b], uf[b], int(tok[b]), int(tok_ref[b]))


@pytest.mark.parametrize("dtypes", [(torch.int64, torch.int32, torch.int64, torch.int32),
                                    (torch.int32, torch.int64, torch.int32, torch.int64)])
def test_finalize_outputs(dev, dtypes):
    cd, ld, bd, pd = dtypes
    batch, width = 40, 16
    g = torch.Generator().manual_seed(1)
    cand = torch.randint(0, 151936, (batch, width), generator=g).to(cd)
    lens = (torch.arange(batch) % width).to(ld)
    bonus = torch.randint(0, 151936, (batch,), generator=g).to(bd)
    prefix = torch.randint(0, 100000, (batch,), generator=g).to(pd)
    out, committed, nxt = verify.finalize_verify_outputs(candidates=cand.to(dev), accept_lens=lens.to(dev),
                                                         bonus=bonus.to(dev), prefix_lens=prefix.to(dev))
    ro, rc, rn = ov.finalize_verify_outputs(cand, lens, bonus, prefix)
    assert torch.equal(out.cpu(), ro) and torch.equal(committed.cpu(), rc) and torch.equal(nxt.cpu(), rn)
    assert nxt.dtype == pd
    greedy = verify.build_greedy_verify_out_tokens(candidates=cand.to(dev), accept_lens=lens.to(dev),
                                                   bonus=bonus.to(dev))
    assert torch.equal(greedy.cpu(), ro)


@pytest.mark.parametrize("idx_dtype", [torch.int64, torch.int32])
def test_assign_fixed_verify_cache_locs(dev, idx_dtype):
    g = torch.Generator().manual_seed(41)
    bs, width, slots, pool = 9, 16, 12, 300
    rtt = torch.randint(0, 1 << 20, (slots, pool), generator=g, dtype=torch.int32)
    req = torch.randperm(slots, generator=g)[:bs]
    start = torch.randint(0, pool - width, (bs,), generator=g)
    start[3] = pool - 5                                 # commit runs past the map: the rest is skipped
    commit = torch.randint(0, width + 1, (bs,), generator=g)
    commit[0], commit[1] = 0, width
    locs = torch.randint(0, 1 << 24, (bs, width), generator=g)
    print(f"assign verify cache locs {idx_dtype}", flush=True)
    want = ov.assign_fixed_verify_cache_locs(req, rtt, start, commit, locs)
    got = rtt.to(dev)
    verify.assign_fixed_verify_cache_locs(req_pool_indices=req.to(idx_dtype).to(dev), req_to_token=got,
                                          start_offset=start.to(idx_dtype).to(dev),
                                          commit_lens=commit.to(torch.int32).to(dev),
                                          verify_cache_locs=locs.to(dev), batch_size=bs, verify_width=width)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)


def test_split_hand_cases(dev):
    """The hand-worked cases of tests/split_cases.py through the GPU path."""
    from tests import split_cases as sc
    p, cand, q, u, exp = sc.decide_case()
    for cdt in (torch.int32, torch.int64):
        d = verify.decide_acceptance(candidates=cand.to(cdt).to(dev), sampled_q=q.to(dev), target_probs=p.to(dev),
                                     uniforms=u.to(dev))
        torch.cuda.synchronize()
        assert d.lengths.cpu().tolist() == exp["lengths"]
        assert d.rejected_rows.cpu().tolist() == exp["rejected_rows"]
        assert d.rejection_positions.cpu().tolist() == exp["rejection_positions"]
        for b, j in enumerate(exp["target_row_index"]):
            assert torch.equal(d.target_rows[b].cpu(), p[b, j]), b
        q_rows, uf, expected = sc.finish_case()
        assert verify.finish_sampling(d, q_rows.to(dev), uniforms=uf.to(dev)).cpu().tolist() == expected
    cases, (clamp_row, u_clamp, tok_clamp) = sc.threshold_cases()
    one = lambda x: torch.tensor(x, device=dev)  # noqa: E731
    for label, p_row, q_row, ufin, tok in cases:
        pp = torch.stack([p_row, p_row])[None].to(dev)
        d = verify.decide_acceptance(candidates=one([[0]]), sampled_q=one([[1.0]]), target_probs=pp,
                                     uniforms=one([[0.5]]))
        assert verify.finish_sampling(d, q_row[None].to(dev), uniforms=one([ufin])).cpu().tolist() == [tok], label
    pp = torch.stack([torch.tensor([0.0, 1.0, 0.0, 0.0]), clamp_row])[None].to(dev)
    d = verify.decide_acceptance(candidates=one([[1]]), sampled_q=one([[0.5]]), target_probs=pp,
                                 uniforms=one([[0.5]]))
    assert d.lengths.cpu().tolist() == [1]
    tok = verify.finish_sampling(d, torch.zeros(0, 4, device=dev), uniforms=one([u_clamp])).cpu().tolist()
    assert tok == [tok_clamp]
