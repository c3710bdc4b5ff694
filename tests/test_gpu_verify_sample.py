"""Fused stochastic verify on the GPU vs the CPU oracle.

Workloads (full 151,936 vocabulary unless stated):
  * temperature 0.7, top-k 50, top-p 0.95, batch 8, block 16;
  * penalised and masked: repetition 1.1 / presence 0.5 / frequency 0.2 over a
    4096-token Zipf(1.1) history, per-row bitmask with ~30% of bits set,
    temperature 0.8, top-p 0.9, min-p 0.05 (batch 4; the workload's batch 32
    runs in the benchmark);
  * top-k 50 / top-p 0.95 with repetition 1.05 over a 2048-token history
    (batch 16; batch 128 runs in the benchmark);
  * pure temperature (dense support), batch 4;
  * dense draft probabilities (q_mode 1), batch 4;
  * the verify-path penalty quirk;
  * small vocabularies with heavy ties and top-k 1 / 5 / 50 / >= V;
  * each scan-kernel choice (raw-only with and without max_top_k, exact
    only), including rows that a raw-only launch sends to the fallback.
Bit-exact accept lengths and tokens except near-ties (tests/verify_ref.py);
drafted-token target probabilities within 1e-5 relative.
"""

import pytest
import torch

from longspark_amd import penalties, verify, workloads
from tests import verify_ref as vr

pytestmark = pytest.mark.gpu


def run_kernel(dev, d, *, verify_quirk=False, draft_params=True, dense_q=None, scan_hint=0, max_top_k=None):
    p = d["params"]
    tables = None
    if "history" in d:
        tables = penalties.build_penalty_tables(d["history"].to(dev), d["logits"].shape[1],
                                                frequency=d["frequency"].to(dev), presence=d["presence"].to(dev),
                                                repetition=d["repetition"].to(dev), verify_quirk=verify_quirk)
    kw = {}
    if draft_params:
        kw = dict(draft_top_ks=p.top_ks.to(dev), draft_top_ps=p.top_ps.to(dev), draft_min_ps=p.min_ps.to(dev))
    width = d["candidates"].shape[1]
    if dense_q is not None:
        kw = dict(draft_probs=dense_q.to(dev))
    else:
        kw.update(draft_logits=d["draft_logits"].to(dev), draft_token_probs=d["draft_token_probs"].to(dev))
    acc, bonus, pc = verify.verify_sample(
        logits=d["logits"].to(dev), candidates=d["candidates"].to(dev), width=width,
        temperatures=p.temperatures.to(dev), top_ks=p.top_ks.to(dev), top_ps=p.top_ps.to(dev),
        min_ps=p.min_ps.to(dev), uniforms=d["uniforms"].to(dev), final_uniforms=d["final_uniforms"].to(dev),
        penalties=tables, vocab_mask=d["vocab_mask"].to(dev) if "vocab_mask" in d else None,
        return_p_cand=True, check=True, scan_hint=scan_hint, max_top_k=max_top_k, **kw)
    torch.cuda.synchronize()
    return acc.cpu(), bonus.cpu(), pc.cpu()


def check_case(dev, d, *, verify_quirk=False, label="", scan_hint=0, max_top_k=None):
    print(f"verify_sample case {label}: B={d['candidates'].shape[0]} V={d['logits'].shape[1]} "
          f"hint={scan_hint} max_top_k={max_top_k}", flush=True)
    acc, bonus, pc = run_kernel(dev, d, verify_quirk=verify_quirk, scan_hint=scan_hint, max_top_k=max_top_k)
    c = vr.oracle_inputs(d, verify_quirk=verify_quirk)
    lens_r, bonus_r, probs_r = vr.run_oracle(c)
    bad, exempt, msgs = vr.classify(c, acc, bonus, lens_r, bonus_r, probs_r, pc)
    for m in msgs:
        print(m)
    assert not bad, f"{len(bad)} requests differ beyond the tie contract: {msgs}"
    assert len(exempt) <= max(1, acc.numel() // 8), f"too many tie exemptions: {msgs}"
    return acc, bonus


def test_topk_topp_full_vocab(dev):
    d = workloads.stochastic_inputs(8, 16, seed=11, temperature=0.7, top_k=50, top_p=0.95)
    acc, _ = check_case(dev, d, label="T0.7 k50 p0.95")
    assert int(acc.min()) >= 0


def test_penalties_mask_topp_minp(dev):
    d = workloads.stochastic_inputs(4, 16, seed=12, temperature=0.8, top_p=0.9, min_p=0.05, history_len=4096,
                                    repetition=1.1, presence=0.5, frequency=0.2, mask_density=0.3)
    check_case(dev, d, label="penalties+mask T0.8 p0.9 minp0.05")


def test_topk_repetition_history(dev):
    d = workloads.stochastic_inputs(16, 16, seed=13, temperature=0.7, top_k=50, top_p=0.95, history_len=2048,
                                    repetition=1.05)
    check_case(dev, d, label="k50 p0.95 rep1.05")


@pytest.mark.parametrize("scan_hint,max_top_k", [(1, 50), (1, None), (2, None), (0, 50)])
def test_scan_hints_topk(dev, scan_hint, max_top_k):
    # (1, 50): raw-only launch in which the wavefront kernels take every row
    # and the draft slices run inside the target launch; (1, None): the
    # workgroup raw scans follow; (2, None): exact scans only.
    d = workloads.stochastic_inputs(16, 16, seed=21, temperature=0.7, top_k=50, top_p=0.95, history_len=2048,
                                    repetition=1.05)
    check_case(dev, d, label="k50 p0.95 rep1.05", scan_hint=scan_hint, max_top_k=max_top_k)


@pytest.mark.parametrize("scan_hint,max_top_k", [(1, 64), (0, 64)])
def test_scan_hints_rows_off_the_raw_path(dev, scan_hint, max_top_k):
    # A negative presence penalty takes every row off the raw-logit path: in a
    # raw-only launch the target rows go to the exact fallback unscanned, the
    # draft slices in the target launch cannot decide the acceptance and leave
    # the draft rows to the exact pass of the resolve kernel.
    d = workloads.stochastic_inputs(6, 16, seed=22, temperature=0.9, top_k=64, top_p=0.9, history_len=3000,
                                    repetition=1.1, presence=-0.7, frequency=0.05)
    check_case(dev, d, label="k64 negative presence", scan_hint=scan_hint, max_top_k=max_top_k)


@pytest.mark.parametrize("scan_hint,max_top_k", [(1, 5), (2, None)])
def test_scan_hints_small_vocab_ties(dev, scan_hint, max_top_k):
    d = workloads.stochastic_inputs(6, 8, 2000, seed=23, temperature=1.0, top_k=5, top_p=0.8)
    g = torch.Generator().manual_seed(5)
    d["logits"] = torch.randint(-4, 5, d["logits"].shape, generator=g).to(torch.bfloat16)
    check_case(dev, d, label="ties k=5", scan_hint=scan_hint, max_top_k=max_top_k)


def test_topk_negative_presence_exact_loop(dev):
    # A negative presence penalty raises repeated tokens: the raw-logit filter
    # is not valid, so these rows take the exact per-element loop.
    d = workloads.stochastic_inputs(6, 16, seed=18, temperature=0.9, top_k=64, top_p=0.9, history_len=3000,
                                    repetition=1.1, presence=-0.7, frequency=0.05)
    check_case(dev, d, label="k64 negative presence")


def test_topk_large_k_full_vocab(dev):
    d = workloads.stochastic_inputs(4, 8, seed=19, temperature=1.1, top_k=700, top_p=0.97, history_len=500,
                                    repetition=1.3)
    check_case(dev, d, label="k700")


def test_verify_quirk(dev):
    d = workloads.stochastic_inputs(4, 16, seed=14, temperature=0.8, top_k=40, top_p=0.9, history_len=1024,
                                    repetition=1.2, presence=0.4, frequency=0.3, mask_density=0.5)
    check_case(dev, d, verify_quirk=True, label="verify quirk")


def test_pure_temperature_dense(dev):
    d = workloads.stochastic_inputs(4, 8, 20000, seed=15, temperature=1.3)
    check_case(dev, d, label="pure temperature")


@pytest.mark.parametrize("top_k", [1, 5, 50, 1000, 2000])
def test_small_vocab_ties(dev, top_k):
    # integer-valued logits -> many exact ties at every threshold
    d = workloads.stochastic_inputs(6, 8, 2000, seed=16 + top_k, temperature=1.0, top_k=top_k, top_p=0.8)
    g = torch.Generator().manual_seed(top_k)
    d["logits"] = torch.randint(-4, 5, d["logits"].shape, generator=g).to(torch.bfloat16)
    check_case(dev, d, label=f"ties k={top_k}")


def test_dense_draft_probs(dev):
    d = workloads.stochastic_inputs(4, 8, 30000, seed=17, temperature=0.9, top_k=30, top_p=0.9)
    from oracle import verify as ov
    p = d["params"]
    q = ov.target_probs(d["draft_logits"].reshape(-1, 30000), temperatures=p.temperatures, top_ks=p.top_ks,
                        top_ps=p.top_ps, min_ps=p.min_ps, rows_per_request=7).view(4, 7, 30000)
    acc, bonus, _ = run_kernel(dev, d, dense_q=q)
    c = vr.oracle_inputs(d)
    x = c["logits"].float()
    probs = ov.target_probs(x, temperatures=p.temperatures, top_ks=p.top_ks, top_ps=p.top_ps, min_ps=p.min_ps,
                            rows_per_request=8).view(4, 8, 30000)
    preds, aidx, anum = ov.chain_speculative_sampling(
        candidates=c["candidates"].long(), uniform_samples=c["uniforms"], uniform_final=c["final_uniforms"],
        target_probs_3d=probs, draft_probs_3d=q)
    ref_bonus = preds[aidx[torch.arange(4), anum.long()].long()]
    assert torch.equal(acc, anum), (acc, anum)
    assert torch.equal(bonus, ref_bonus.long()), (bonus, ref_bonus)


@pytest.mark.parametrize("case", ["ties", "off-raw"])
def test_inline_exact_pass_matches_fallback_launch(dev, case):
    # Without the per-row p(drafted) output the fused launch skips the
    # fallback kernel and the resolve kernel runs the exact pass on the target
    # rows it needs; the results equal the fallback launch's and the oracle's.
    if case == "ties":  # integer logits: ties at the top-k threshold overflow the candidate buffers
        d = workloads.stochastic_inputs(6, 8, seed=24, temperature=1.0, top_k=50, top_p=0.8)
        g = torch.Generator().manual_seed(24)
        d["logits"] = torch.randint(-4, 5, d["logits"].shape, generator=g).to(torch.bfloat16)
        max_top_k = 50
    else:  # a negative presence penalty sends every row to the exact pass unscanned
        d = workloads.stochastic_inputs(6, 16, seed=25, temperature=0.9, top_k=64, top_p=0.9, history_len=3000,
                                        repetition=1.1, presence=-0.7, frequency=0.05)
        max_top_k = 64
    print(f"inline exact pass: {case}", flush=True)
    acc_f, bonus_f, _ = run_kernel(dev, d, scan_hint=1, max_top_k=max_top_k)  # with p_cand: fallback launch
    p = d["params"]
    tables = None
    if "history" in d:
        tables = penalties.build_penalty_tables(d["history"].to(dev), d["logits"].shape[1],
                                                frequency=d["frequency"].to(dev), presence=d["presence"].to(dev),
                                                repetition=d["repetition"].to(dev))
    acc, bonus = verify.verify_sample(
        logits=d["logits"].to(dev), candidates=d["candidates"].to(dev), width=d["candidates"].shape[1],
        temperatures=p.temperatures.to(dev), top_ks=p.top_ks.to(dev), top_ps=p.top_ps.to(dev),
        min_ps=p.min_ps.to(dev), uniforms=d["uniforms"].to(dev), final_uniforms=d["final_uniforms"].to(dev),
        draft_logits=d["draft_logits"].to(dev), draft_token_probs=d["draft_token_probs"].to(dev),
        draft_top_ks=p.top_ks.to(dev), draft_top_ps=p.top_ps.to(dev), draft_min_ps=p.min_ps.to(dev),
        penalties=tables, check=True, scan_hint=1, max_top_k=max_top_k)
    torch.cuda.synchronize()
    assert torch.equal(acc.cpu(), acc_f) and torch.equal(bonus.cpu(), bonus_f), (acc, acc_f, bonus, bonus_f)
    c = vr.oracle_inputs(d)
    lens_r, bonus_r, probs_r = vr.run_oracle(c)
    bad, exempt, msgs = vr.classify(c, acc.cpu(), bonus.cpu(), lens_r, bonus_r, probs_r)
    assert not bad, msgs
