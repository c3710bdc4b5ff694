"""Acceptance drop-ins on the GPU vs the CPU oracle.

* ``chain_speculative_sampling_triton`` (dense target and draft
  probabilities): partial acceptance, an all-accepted request (bonus from the
  last target row), a degenerate residual (p == q: vocab-1), int32 and int64
  index tensors, a permuted ``retrive_index``, rows that are not 16-byte
  aligned, the full 151,936 vocabulary, a 300,007-token vocabulary and a
  chain of 80 tokens.  Accepted lengths, accept
  indices and accepted tokens bit-exact; the bonus bit-exact except an
  inverse-CDF boundary within 1e-6 of the total (fp64 running sums here,
  fp32 blockwise sums in the reference).
* the verify-length cutoff of the fused verify: capped length, trim and the
  drafted token at the cap, exactly as ``cap_correct_len`` then the
  accepted-slot read back.
* ``AcceptSampling.execute`` (target top-k / top-p, or pure temperature,
  dense q) and ``execute_single_q`` against the oracle on the same draws
  (``torch.rand`` after the same seed), with the tie contract of
  tests/verify_ref.py.
* ``accept_draft_tokens``: each dispatch branch against the ops it must run.
* ``apply_dflash_verify_logits_adjustments`` and ``add_request_bias_``: bit-exact
  against the reference's tensor operations evaluated on the CPU.
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import verify as ov
from longspark_amd import accept, dense, penalties, verify, workloads
from tests import verify_ref as vr

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------ chain

def chain_inputs(batch, width, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    x = 3.0 * torch.randn(batch, width, vocab, generator=g)
    # every other target row top-k sparse: zeros in p
    x[:, ::2, :] = torch.where(x[:, ::2, :] >= torch.topk(x[:, ::2, :], 40, dim=-1).values[..., -1:],
                               x[:, ::2, :], torch.full_like(x[:, ::2, :], float("-inf")))
    p = torch.softmax(x / 0.8, dim=-1)
    q = torch.softmax((3.0 * torch.randn(batch, width - 1, vocab, generator=g) + x[:, :-1].clamp_min(-20)) / 0.8,
                      dim=-1)
    cand = torch.randint(0, vocab, (batch, width), generator=g)
    cand[:, 1:] = torch.multinomial(q.reshape(-1, vocab), 1, generator=g).view(batch, width - 1)
    # request 0: q = p at every drafted row and drafted tokens in the support -> all accepted
    q[0] = p[0, :-1]
    cand[0, 1:] = torch.argmax(p[0, :-1], dim=-1)
    # request 1: rejection at j = 0 on a token outside p's support with q = p there -> zero residual
    q[1, 0] = p[1, 0]
    cand[1, 1] = int(torch.nonzero(p[1, 0] == 0)[0])
    u = torch.rand(batch, width - 1, generator=g)
    uf = torch.rand(batch, generator=g)
    return p, q, cand, u, uf


def misaligned(t):
    """Same values with a row stride of V+1 and a start 4 bytes off alignment."""
    big = torch.empty(*t.shape[:-1], t.shape[-1] + 1, dtype=t.dtype)
    big[..., 1:] = t
    return big[..., 1:]


@pytest.mark.parametrize("batch,width,vocab,idx_dtype,aligned,permute", [
    (6, 8, 5000, torch.int64, True, False),
    (5, 8, 5001, torch.int32, False, True),
    (3, 16, workloads.VOCAB, torch.int64, True, True),
    (2, 4, 300_007, torch.int32, True, False),   # more than 256 chunk sums: the looped walk
    (3, 80, 3000, torch.int64, True, True),      # more than 64 accepted tokens: the looped writes
])
def test_chain_sampling(dev, batch, width, vocab, idx_dtype, aligned, permute):
    p, q, cand, u, uf = chain_inputs(batch, width, vocab, seed=vocab + width)
    print(f"chain sampling B={batch} K={width} V={vocab} {idx_dtype} aligned={aligned}", flush=True)
    ridx, nxt, sib, predicts, aidx, anum = accept.chain_verify_buffers(bs=batch, draft_token_num=width, device=dev)
    if permute:
        ridx = torch.randperm(batch * width, generator=torch.Generator().manual_seed(3)).view(batch, width).to(dev)
    pd, qd = (p, q) if aligned else (misaligned(p), misaligned(q))
    accept.chain_speculative_sampling_triton(
        predicts=predicts, accept_index=aidx, accept_token_num=anum, candidates=cand.to(idx_dtype).to(dev),
        retrive_index=ridx.to(idx_dtype), retrive_next_token=nxt, retrive_next_sibling=sib, uniform_samples=u.to(dev),
        uniform_samples_for_final_sampling=uf.to(dev), target_probs=pd.to(dev), draft_probs=qd.to(dev),
        threshold_single=1.0, threshold_acc=1.0, deterministic=True)
    torch.cuda.synchronize()
    pr, ar, nr = ov.chain_speculative_sampling(candidates=cand, uniform_samples=u, uniform_final=uf,
                                               target_probs_3d=p, draft_probs_3d=q)
    predicts, aidx, anum, ridx = predicts.cpu(), aidx.cpu(), anum.cpu(), ridx.cpu().long()
    assert torch.equal(anum, nr), (anum, nr)
    assert int(anum[0]) == width - 1, "request 0 must accept every draft"
    assert int(anum[1]) == 0
    for b in range(batch):
        L = int(anum[b])
        assert torch.equal(aidx[b, :L + 1].long(), ridx[b, :L + 1]), b
        got = predicts[ridx[b, :L + 1]].long()
        ref = pr[b * width: b * width + L + 1].long()
        assert torch.equal(got[:L], ref[:L]), (b, got, ref)
        if int(got[L]) != int(ref[L]):
            vals = vr.bonus_row(p[b, L], q[b, L] if L < width - 1 else None, L < width - 1, single_q=False)
            assert vr.cdf_tie(vals, float(uf[b]), int(got[L]), int(ref[L])), (b, int(got[L]), int(ref[L]))
    assert int(predicts[ridx[1, 0]]) == vocab - 1, "a zero residual must return vocab - 1"


# ------------------------------------------------------------------ cutoff

@pytest.mark.parametrize("cand_dtype", [torch.int32, torch.int64])
def test_verify_sample_cutoff(dev, cand_dtype):
    d = workloads.stochastic_inputs(12, 8, 20000, seed=71, temperature=0.9, top_k=50, top_p=0.95)
    # most drafts accepted: q of the drafted tokens tiny
    d["draft_token_probs"] = torch.full_like(d["draft_token_probs"], 1e-9)
    p = d["params"]
    common = dict(logits=d["logits"].to(dev), candidates=d["candidates"].to(cand_dtype).to(dev), width=8,
                  temperatures=p.temperatures.to(dev), top_ks=p.top_ks.to(dev), top_ps=p.top_ps.to(dev),
                  uniforms=d["uniforms"].to(dev), final_uniforms=d["final_uniforms"].to(dev),
                  draft_logits=d["draft_logits"].to(dev), draft_token_probs=d["draft_token_probs"].to(dev))
    print("verify_sample cutoff", cand_dtype, flush=True)
    lens, bonus = verify.verify_sample(**common)
    cutoff = torch.tensor([1, 2, 3, 4, 5, 6, 7, 8, 8, 1, 3, 0], dtype=torch.int32)
    lc, bc, tc = verify.verify_sample(**common, cutoff_verify_lens=cutoff.to(dev), return_cap_trim=True)
    torch.cuda.synchronize()
    lens, bonus, lc, bc, tc = lens.cpu(), bonus.cpu(), lc.cpu(), bc.cpu(), tc.cpu()
    cap = (cutoff - 1).clamp_min(0)
    want_len = torch.minimum(lens, cap)
    cand = d["candidates"].long()
    at_cap = cand[torch.arange(12), (want_len + 1).clamp(max=7).long()]
    want_bonus = torch.where(want_len < lens, at_cap, bonus)
    assert torch.equal(lc, want_len), (lc, want_len)
    assert torch.equal(tc, lens - want_len), (tc, lens - want_len)
    assert torch.equal(bc, want_bonus), (bc, want_bonus)
    assert int((lens > want_len).sum()) >= 4, "the cutoff must bind for several requests"


# --------------------------------------------------------- AcceptSampling

def info_of(params, dev, *, need_top_k=True, need_top_p=True):
    return SimpleNamespace(temperatures=params.temperatures.reshape(-1, 1).to(dev),
                           top_ks=params.top_ks.to(dev), top_ps=params.top_ps.to(dev),
                           min_ps=params.min_ps.to(dev), need_top_k_sampling=need_top_k,
                           need_top_p_sampling=need_top_p, need_min_p_sampling=False, is_all_greedy=False,
                           is_any_greedy=False, penalizer_orchestrator=None, has_custom_logit_processor=False)


def draws(dev, seed, bs, gamma):
    torch.cuda.manual_seed(seed)
    return torch.rand((bs, gamma), device=dev).cpu(), torch.rand((bs,), device=dev).cpu()


def check_against_chain(lens, bonus, probs, q, cand, u, uf):
    pr, ar, nr = ov.chain_speculative_sampling(candidates=cand, uniform_samples=u, uniform_final=uf,
                                               target_probs_3d=probs.float(), draft_probs_3d=q)
    width = cand.shape[1]
    ref_bonus = pr[ar[torch.arange(cand.shape[0]), nr.long()].long()].long()
    bad = []
    for b in range(cand.shape[0]):
        if int(lens[b]) == int(nr[b]) and int(bonus[b]) == int(ref_bonus[b]):
            continue
        L = min(int(lens[b]), int(nr[b]))
        ties = [j for j in range(min(max(int(lens[b]), int(nr[b])) + 1, width - 1))
                if abs(float(u[b, j]) * float(q[b, j, cand[b, j + 1]]) - float(probs[b, j, cand[b, j + 1]]))
                <= vr.TIE]
        if ties:
            continue
        if int(lens[b]) == int(nr[b]):
            vals = vr.bonus_row(probs[b, L], q[b, L] if L < width - 1 else None, L < width - 1, single_q=False)
            if vr.cdf_tie(vals, float(uf[b]), int(bonus[b]), int(ref_bonus[b])):
                continue
        bad.append((b, int(lens[b]), int(nr[b]), int(bonus[b]), int(ref_bonus[b])))
    assert not bad, f"requests differ beyond the tie contract: {bad}"


@pytest.mark.parametrize("need_top,vocab", [(True, 30000), (False, 30000), (True, workloads.VOCAB)])
def test_accept_sampling_dense_q(dev, need_top, vocab):
    bs, width = 6, 8
    d = workloads.stochastic_inputs(bs, width, vocab, seed=72 + vocab % 7, temperature=0.9, top_k=30, top_p=0.9)
    p = d["params"]
    q = ov.softmax_temp(d["draft_logits"].reshape(-1, vocab), p.temperatures, width - 1).view(bs, width - 1, vocab)
    info = info_of(p, dev, need_top_k=need_top, need_top_p=need_top)
    cand = d["candidates"].long()
    print(f"AcceptSampling.execute top={need_top} V={vocab}", flush=True)
    torch.cuda.manual_seed(901)
    lens, bonus, trim = accept.AcceptSampling.execute(
        candidates=cand.to(dev), target_logits=d["logits"].to(dev), draft_probs=q.to(dev), sampling_info=info,
        draft_input=SimpleNamespace(max_top_k=None, uniform_top_k_value=None), gamma=width - 1,
        verify_num_draft_tokens=width)
    torch.cuda.synchronize()
    u, uf = draws(dev, 901, bs, width - 1)
    x = d["logits"].float()
    if need_top:
        probs = ov.target_probs(x, temperatures=p.temperatures, top_ks=p.top_ks, top_ps=p.top_ps,
                                min_ps=torch.zeros(bs), rows_per_request=width, compute_dtype=torch.float64)
    else:
        probs = vr_softmax64(x, p.temperatures, width)
    check_against_chain(lens.cpu(), bonus.cpu(), probs.view(bs, width, vocab), q, cand, u, uf)
    assert int(trim.abs().sum()) == 0


def vr_softmax64(x, temps, rpr):
    t = torch.repeat_interleave(temps.reshape(-1).float(), rpr)
    return torch.softmax((x / t[:, None]).double(), dim=-1).float()


def test_accept_sampling_cutoff_and_max_top_k(dev):
    bs, width, vocab = 8, 8, 30000
    d = workloads.stochastic_inputs(bs, width, vocab, seed=74, temperature=0.9, top_k=30, top_p=0.9)
    p = d["params"]
    p.top_ks[::2] = 60   # every other request asks for 60; max_top_k 40 clamps them
    q = ov.softmax_temp(d["draft_logits"].reshape(-1, vocab), p.temperatures, width - 1).view(bs, width - 1, vocab)
    info = info_of(p, dev)
    cand = d["candidates"].long()
    cutoff = torch.tensor([8, 1, 2, 3, 8, 5, 6, 2], dtype=torch.int32)
    print("AcceptSampling.execute cutoff + max_top_k", flush=True)
    torch.cuda.manual_seed(902)
    lens, bonus, trim = accept.AcceptSampling.execute(
        candidates=cand.to(dev), target_logits=d["logits"].to(dev), draft_probs=q.to(dev), sampling_info=info,
        draft_input=SimpleNamespace(max_top_k=40, uniform_top_k_value=None), gamma=width - 1,
        verify_num_draft_tokens=width, cutoff_verify_lens=cutoff.to(dev))
    torch.cuda.synchronize()
    torch.cuda.manual_seed(902)
    ln, bn, _ = accept.AcceptSampling.execute(
        candidates=cand.to(dev), target_logits=d["logits"].to(dev), draft_probs=q.to(dev), sampling_info=info,
        draft_input=SimpleNamespace(max_top_k=40, uniform_top_k_value=None), gamma=width - 1,
        verify_num_draft_tokens=width)
    torch.cuda.synchronize()
    u, uf = draws(dev, 902, bs, width - 1)
    probs = ov.target_probs(d["logits"].float(), temperatures=p.temperatures, top_ks=p.top_ks.clamp(max=40),
                            top_ps=p.top_ps, min_ps=torch.zeros(bs), rows_per_request=width,
                            compute_dtype=torch.float64).view(bs, width, vocab)
    check_against_chain(ln.cpu(), bn.cpu(), probs, q, cand, u, uf)
    ln, bn, lens, bonus, trim = ln.cpu(), bn.cpu(), lens.cpu(), bonus.cpu(), trim.cpu()
    capped = torch.minimum(ln, (cutoff - 1).clamp_min(0))
    assert torch.equal(lens, capped) and torch.equal(trim, ln - capped)
    at_cap = cand[torch.arange(bs), (capped + 1).clamp(max=width - 1).long()]
    assert torch.equal(bonus, torch.where(capped < ln, at_cap, bn))


def test_accept_sampling_single_q(dev):
    bs, width, vocab = 8, 8, 30000
    d = workloads.stochastic_inputs(bs, width, vocab, seed=75, temperature=0.8)
    p = d["params"]
    dtemps = p.temperatures * 1.1
    info = info_of(p, dev, need_top_k=False, need_top_p=False)
    print("AcceptSampling.execute_single_q", flush=True)
    torch.cuda.manual_seed(903)
    lens, bonus, zeros = accept.AcceptSampling.execute_single_q(
        candidates=d["candidates"].long().to(dev), target_logits=d["logits"].to(dev),
        corrected_logits=d["draft_logits"].to(dev), draft_token_probs=d["draft_token_probs"].to(dev),
        draft_temperatures=dtemps.to(dev), sampling_info=info, draft_input=None, gamma=width - 1,
        verify_num_draft_tokens=width)
    torch.cuda.synchronize()
    u, uf = draws(dev, 903, bs, width - 1)
    probs = vr_softmax64(d["logits"].float(), p.temperatures, width).view(bs, width, vocab)
    lr, br = ov.accept_single_q(
        candidates=d["candidates"].long(), target_probs_3d=probs,
        draft_q_rows_fn=lambda pos: ov.draft_q_rows(d["draft_logits"], pos, temperatures=dtemps),
        draft_token_probs=d["draft_token_probs"], uniforms=u, final_uniforms=uf)
    lens, bonus = lens.cpu(), bonus.cpu()
    cand = d["candidates"].long()
    for b in range(bs):
        if int(lens[b]) == int(lr[b]) and int(bonus[b]) == int(br[b]):
            continue
        j = min(int(lens[b]), int(lr[b]))
        if j < width - 1 and abs(float(u[b, j] * d["draft_token_probs"][b, j]) -
                                 float(probs[b, j, cand[b, j + 1]])) <= vr.TIE:
            continue
        L = int(lr[b])
        assert int(lens[b]) == L, (b, int(lens[b]), L)
        qrow = ov.draft_q_rows(d["draft_logits"][b:b + 1], torch.tensor([min(L, width - 2)]),
                               temperatures=dtemps[b:b + 1])[0]
        vals = vr.bonus_row(probs[b, L], qrow, L < width - 1, single_q=True)
        assert vr.cdf_tie(vals, float(uf[b]), int(bonus[b]), int(br[b])), (b, int(bonus[b]), int(br[b]))
    assert int(zeros.abs().sum()) == 0
    with pytest.raises(ValueError, match="cutoff"):
        accept.AcceptSampling.execute_single_q(
            candidates=d["candidates"].long().to(dev), target_logits=d["logits"].to(dev),
            corrected_logits=d["draft_logits"].to(dev), draft_token_probs=d["draft_token_probs"].to(dev),
            draft_temperatures=dtemps.to(dev), sampling_info=info, draft_input=None, gamma=width - 1,
            verify_num_draft_tokens=width, cutoff_verify_lens=torch.ones(bs, dtype=torch.int32, device=dev))


# ------------------------------------------------------ accept_draft_tokens

def test_accept_draft_tokens_dispatch(dev):
    bs, width, vocab = 6, 8, 20000
    d = workloads.stochastic_inputs(bs, width, vocab, seed=76, temperature=0.9, top_k=40, top_p=0.9)
    p = d["params"]
    cand = d["candidates"].long().to(dev)
    logits = d["logits"].to(dev)
    block = SimpleNamespace(draft_tokens=cand[:, 1:], corrected_logits=d["draft_logits"].to(dev),
                            greedy_mask=torch.tensor([1, 0, 0, 1, 0, 0], dtype=torch.bool, device=dev),
                            temperatures=p.temperatures.to(dev), draft_token_probs=d["draft_token_probs"].to(dev))
    din = SimpleNamespace(max_top_k=None, uniform_top_k_value=None)
    kw = dict(candidates=cand, target_logits=logits, draft_block=block, draft_input=din, gamma=width - 1,
              verify_num_draft_tokens=width)
    print("accept_draft_tokens dispatch", flush=True)

    # greedy batch
    out = accept.accept_draft_tokens(sampling_info=None, **kw)
    ref = verify.AcceptGreedy.execute(candidates=cand, target_logits=logits, verify_num_draft_tokens=width)
    assert all(torch.equal(a, b) for a, b in zip(out, ref))
    lr, br, _ = ov.accept_greedy(d["candidates"].long(), d["logits"].float(), width)
    assert torch.equal(out[0].cpu().long(), lr.long()) and torch.equal(out[1].cpu(), br.long())

    # nonstrict: every scheduled draft committed, bonus = argmax at the committed length
    cut = SimpleNamespace(verify_lens=torch.tensor([8, 1, 3, 0, 5, 9], dtype=torch.int32, device=dev))
    out = accept.accept_draft_tokens(sampling_info=None, nonstrict_verify=True, cutoff_layout=cut, **kw)
    truth = d["logits"].float().argmax(-1).view(bs, width)
    want = (cut.verify_lens.cpu() - 1).clamp(0, width - 1)
    assert torch.equal(out[0].cpu(), want.to(torch.int32))
    assert torch.equal(out[1].cpu(), truth[torch.arange(bs), want.long()])

    # pure temperature with the drafter's q: single-q path
    info = info_of(p, dev, need_top_k=False, need_top_p=False)
    torch.cuda.manual_seed(904)
    out = accept.accept_draft_tokens(sampling_info=info, **kw)
    torch.cuda.manual_seed(904)
    ref = accept.AcceptSampling.execute_single_q(
        candidates=cand, target_logits=logits, corrected_logits=block.corrected_logits,
        draft_token_probs=block.draft_token_probs, draft_temperatures=block.temperatures, sampling_info=info,
        draft_input=din, gamma=width - 1, verify_num_draft_tokens=width)
    assert all(torch.equal(a, b) for a, b in zip(out, ref))

    # top-k / top-p: dense draft probabilities and the chain rule
    info = info_of(p, dev)
    q = dense.SoftmaxTemp.execute(logits=block.corrected_logits.reshape(-1, vocab), temperatures=block.temperatures,
                                  rows_per_request=width - 1).view(bs, width - 1, vocab)
    torch.cuda.manual_seed(905)
    out = accept.accept_draft_tokens(sampling_info=info, **kw)
    torch.cuda.manual_seed(905)
    ref = accept.AcceptSampling.execute(candidates=cand, target_logits=logits, draft_probs=q, sampling_info=info,
                                        draft_input=din, gamma=width - 1, verify_num_draft_tokens=width)
    assert all(torch.equal(a, b) for a, b in zip(out, ref))

    # mixed batch: greedy requests take the greedy result
    info.is_any_greedy = True
    torch.cuda.manual_seed(906)
    out = accept.accept_draft_tokens(sampling_info=info, **kw)
    torch.cuda.manual_seed(906)
    s = accept.AcceptSampling.execute(candidates=cand, target_logits=logits, draft_probs=q, sampling_info=info,
                                      draft_input=din, gamma=width - 1, verify_num_draft_tokens=width)
    g = verify.AcceptGreedy.execute(candidates=cand, target_logits=logits, verify_num_draft_tokens=width)
    m = block.greedy_mask
    for o, gg, ss in zip(out, g, s):
        assert torch.equal(o, torch.where(m, gg.to(ss.dtype), ss))


# ------------------------------------------------------- logit adjustments

class FakeInfo(SimpleNamespace):
    """The parts of SamplingBatchInfo the verify adjustments read; its
    apply_logits_bias follows SRT/sampling/sampling_batch_info.py:269-286 with
    frequency and presence penalisers (subtract their accumulated [B, V]
    tensors), an xgrammar-style packed mask (bit 0 -> -inf) and a logit bias."""

    def __len__(self):
        return self.temperatures.shape[0]

    def apply_logits_bias(self, logits):
        if self.penalizer_orchestrator is not None and self.penalizer_orchestrator.is_required:
            logits.sub_(self.freq_cum.to(logits.device))
            logits.sub_(self.pres_cum.to(logits.device))
        if self.vocab_mask is not None:
            vocab = logits.shape[1]
            bits = unpack_bits(self.vocab_mask.to(logits.device), vocab)
            logits.masked_fill_(~bits, float("-inf"))
        if self.logit_bias is not None:
            logits.add_(self.logit_bias.to(logits.device))


def unpack_bits(mask, vocab):
    v = torch.arange(vocab, device=mask.device)
    return ((mask[:, v >> 5] >> (v & 31)) & 1).bool()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_apply_dflash_verify_logits_adjustments(dev, dtype):
    bs, width, vocab = 4, 8, 30001
    g = torch.Generator().manual_seed(77)
    logits = (3.0 * torch.randn(bs * width, vocab, generator=g)).to(dtype)
    acc = -0.37 * torch.randint(0, 4, (bs, vocab), generator=g).float()
    lb = torch.zeros(bs, vocab)
    lb[:, ::97] = 1.3
    print(f"dflash adjustments {dtype}", flush=True)
    # overlap path: acc_linear_penalties then logit_bias, each in the logits' dtype
    info = FakeInfo(temperatures=torch.ones(bs, 1), acc_linear_penalties=acc.to(dev), penalizer_orchestrator=None,
                    vocab_mask=None, logit_bias=lb.to(dev), has_custom_logit_processor=False)
    x = logits.to(dev)
    penalties.apply_dflash_verify_logits_adjustments(next_token_logits=x, sampling_info=info, draft_token_num=width)
    ref = logits.clone().view(bs, width, vocab)
    ref.add_(acc.to(dtype)[:, None, :])
    ref.add_(lb.to(dtype)[:, None, :])
    assert torch.equal(x.cpu().view(bs, width, vocab), ref)

    # dense path: live penalisers, a grammar mask and a logit bias on a zero bias tensor
    mask = workloads.random_bitmask(bs, vocab, density=0.6, seed=78)
    freq = 0.2 * torch.randint(0, 3, (bs, vocab), generator=g).float()
    pres = 0.5 * (freq > 0).float()
    info = FakeInfo(temperatures=torch.ones(bs, 1), acc_linear_penalties=None,
                    penalizer_orchestrator=SimpleNamespace(is_required=True), freq_cum=freq, pres_cum=pres,
                    vocab_mask=mask.to(dev), logit_bias=lb.to(dev), has_custom_logit_processor=False)
    x = logits.to(dev)
    penalties.apply_dflash_verify_logits_adjustments(next_token_logits=x, sampling_info=info, draft_token_num=width)
    lp = torch.zeros(bs, vocab)
    info_cpu = FakeInfo(**{**vars(info), "vocab_mask": mask, "logit_bias": lb})
    info_cpu.apply_logits_bias(lp)
    ref = logits.clone().view(bs, width, vocab)
    ref.add_(lp[:, None, :].to(dtype))
    assert torch.equal(x.cpu().view(bs, width, vocab), ref)

    # nothing to apply: untouched
    info = FakeInfo(temperatures=torch.ones(bs, 1), acc_linear_penalties=None, penalizer_orchestrator=None,
                    vocab_mask=None, logit_bias=None, has_custom_logit_processor=False)
    x = logits.to(dev)
    penalties.apply_dflash_verify_logits_adjustments(next_token_logits=x, sampling_info=info, draft_token_num=width)
    assert torch.equal(x.cpu(), logits)
    with pytest.raises(ValueError, match="row count mismatch"):
        penalties.apply_dflash_verify_logits_adjustments(next_token_logits=x[:-1], sampling_info=info,
                                                         draft_token_num=width)


@pytest.mark.parametrize("dtype,vocab,offset", [(torch.float16, 5003, 1), (torch.float32, 4096, 0),
                                                (torch.bfloat16, workloads.VOCAB, 0)])
def test_add_request_bias_combined_mask(dev, dtype, vocab, offset):
    bs, rpr = 3, 5
    g = torch.Generator().manual_seed(79)
    base = (2.0 * torch.randn(bs * rpr, vocab + offset, generator=g)).to(dtype)
    bias = 0.3 * torch.randn(bs, vocab, generator=g)
    bias2 = torch.zeros(bs, vocab)
    bias2[:, 5::11] = -0.75
    words = (vocab + 31) // 32 - 1  # a narrower mask: the last columns stay unmasked
    mask = workloads.random_bitmask(bs, 32 * words, density=0.5, seed=80)
    print(f"add_request_bias {dtype} V={vocab} offset={offset}", flush=True)
    x = base.to(dev)
    penalties.add_request_bias_(x[:, offset:], rows_per_request=rpr, bias=bias.to(dev), vocab_mask=mask.to(dev),
                                bias2=bias2.to(dev))
    z = bias.clone()
    z[:, :32 * words].masked_fill_(~unpack_bits(mask, 32 * words), float("-inf"))
    z += bias2
    ref = base.clone()
    ref[:, offset:].view(bs, rpr, vocab).add_(z.to(dtype)[:, None, :])
    assert torch.equal(x.cpu(), ref)


# ------------------------------------------------------------- empty batches

def test_empty_batches(dev):
    """Zero-request inputs give empty outputs and launch nothing, as the
    reference's tensor code does with empty tensors."""
    from longspark_amd import sample
    v = 1000
    print("empty batches", flush=True)
    logits = torch.empty(0, v, dtype=torch.bfloat16, device=dev)
    cand = torch.empty(0, 8, dtype=torch.int64, device=dev)
    acc, bonus, trim = verify.verify_greedy(logits=logits, candidates=cand, width=8)
    assert acc.shape == (0,) and bonus.shape == (0,) and trim.shape == (0,)
    z = torch.empty(0, device=dev)
    acc, bonus, trim, pc = verify.verify_sample(
        logits=logits, candidates=cand, width=8, temperatures=z, uniforms=torch.empty(0, 7, device=dev),
        final_uniforms=z, draft_logits=torch.empty(0, 7, v, device=dev),
        draft_token_probs=torch.empty(0, 7, device=dev), return_cap_trim=True, return_p_cand=True)
    assert acc.shape == (0,) and bonus.shape == (0,) and trim.shape == (0,) and pc.shape == (0, 7)
    assert dense.softmax_temp(logits=logits, temperatures=z, rows_per_request=8).shape == (0, v)
    assert dense.target_probs(logits=logits, temperatures=z, rows_per_request=8, top_ks=torch.empty(0, device=dev),
                              top_ps=z).shape == (0, v)
    tables = penalties.build_penalty_tables(torch.empty(0, 16, dtype=torch.int32, device=dev), v,
                                            repetition=z)
    assert tables.bits.shape[0] == 0
    penalties.adjust_logits_(logits, rows_per_request=8, tables=tables)
    penalties.add_request_bias_(logits, rows_per_request=8, bias=torch.empty(0, v, device=dev))
    ridx, nxt, sib, preds, aidx, anum = accept.chain_verify_buffers(bs=0, draft_token_num=8, device=dev)
    accept.chain_speculative_sampling_triton(preds, aidx, anum, cand, ridx, nxt, sib, torch.empty(0, 7, device=dev),
                                             z, torch.empty(0, 8, v, device=dev), torch.empty(0, 7, v, device=dev),
                                             1.0, 1.0, True)
    tok, q = sample.sample_step_tokens_with_q(step_logits=torch.empty(0, v, device=dev), temperatures=z)
    assert tok.shape == (0,) and q.shape == (0,)
    torch.cuda.synchronize()
