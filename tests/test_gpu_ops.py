"""The custom operators on the GPU: schema and fake-tensor checks
(``torch.library.opcheck``) on real inputs, and the same results as the
drop-ins they wrap."""

import pytest
import torch

from longspark_amd import kvwindow, ops, penalties, verify, workloads  # noqa: F401  (ops registers)

pytestmark = pytest.mark.gpu

CHECKS = ("test_schema", "test_faketensor")
L = torch.ops.longspark_amd


def test_verify_ops(dev):
    logits, cand = workloads.greedy_inputs(4, 8, 5000, seed=1, device=dev)
    torch.library.opcheck(L.verify_greedy.default, (logits, cand, 8), test_utils=CHECKS)
    a, b, _ = L.verify_greedy(logits, cand, 8)
    a2, b2, _ = verify.verify_greedy(logits=logits, candidates=cand, width=8)
    assert torch.equal(a, a2) and torch.equal(b, b2)

    d = workloads.stochastic_inputs(4, 8, 5000, seed=2, temperature=0.7, top_k=50, top_p=0.95, history_len=300,
                                    repetition=1.05, presence=0.2, device=dev)
    p = d["params"]
    bits, rank, add, distinct, nonpos = L.penalty_tables(d["history"], 5000, None, d["presence"])
    args = (d["logits"], d["candidates"], 8, p.temperatures, d["uniforms"], d["final_uniforms"])
    kw = dict(top_ks=p.top_ks, top_ps=p.top_ps, max_top_k=50, draft_token_probs=d["draft_token_probs"],
              draft_logits=d["draft_logits"], draft_top_ks=p.top_ks, draft_top_ps=p.top_ps, pen_bits=bits,
              pen_rank=rank, pen_add=add, pen_nonpositive=nonpos, pen_repetition=d["repetition"])
    torch.library.opcheck(L.verify_sample.default, args, kw, test_utils=CHECKS)
    acc, bonus, _ = L.verify_sample(*args, **kw)
    tables = penalties.build_penalty_tables(d["history"], 5000, presence=d["presence"], repetition=d["repetition"])
    acc2, bonus2 = verify.verify_sample(
        logits=d["logits"], candidates=d["candidates"], width=8, temperatures=p.temperatures,
        uniforms=d["uniforms"], final_uniforms=d["final_uniforms"], top_ks=p.top_ks, top_ps=p.top_ps, max_top_k=50,
        draft_token_probs=d["draft_token_probs"], draft_logits=d["draft_logits"], draft_top_ks=p.top_ks,
        draft_top_ps=p.top_ps, penalties=tables)
    assert torch.equal(acc, acc2) and torch.equal(bonus, bonus2)


def test_dense_and_mask_ops(dev):
    logits, _ = workloads.greedy_inputs(2, 4, 3000, seed=3, device=dev)
    temps = torch.full((2,), 0.8, device=dev)
    torch.library.opcheck(L.softmax_temp.default, (logits, temps, 4), test_utils=CHECKS)
    mask = workloads.random_bitmask(8, 3000, density=0.3, seed=4, device=dev)
    x = logits.clone()
    torch.library.opcheck(L.apply_token_bitmask.default, (x, mask), test_utils=CHECKS)
    x, y = logits.clone(), logits.clone()
    L.apply_token_bitmask(x, mask)
    penalties.apply_token_bitmask_inplace(y, mask)
    assert torch.equal(x, y)


def test_refresh_ops(dev):
    r = workloads.full_round_refresh_inputs(dev, batch=4, layers=2, q_heads=8, kv_heads=2, rows=16)
    out = torch.empty(4, 2, 2, 2, 256, 128, dtype=torch.bfloat16, device=dev)
    args = (r["k"], r["v"], r["table"], r["seq"], 16, 256, out)
    torch.library.opcheck(L.kv_window_gather.default, args, test_utils=CHECKS)
    ref = kvwindow.gather_window(r["k"], r["v"], r["table"], r["seq"], page_size=16, window=256)
    L.kv_window_gather(*args)
    assert torch.equal(out, ref)
    lens = torch.full((4,), 16, dtype=torch.int32, device=dev)
    st, ls = r["state"].clone(), r["lse"].clone()
    sargs = (r["query"], r["k"], r["v"], r["locs"], lens, st, ls, 128 ** -0.5)
    torch.library.opcheck(L.summary_update.default, sargs, test_utils=CHECKS)
    st, ls = r["state"].clone(), r["lse"].clone()
    L.summary_update(r["query"], r["k"], r["v"], r["locs"], lens, st, ls, 128 ** -0.5)
    from longspark_amd import summary
    st2, ls2 = r["state"].clone(), r["lse"].clone()
    summary.summary_update(query=r["query"], key_cache=r["k"], value_cache=r["v"], accepted_cache_locs=r["locs"],
                           accept_lens=lens, state_output=st2, state_lse=ls2, softmax_scale=128 ** -0.5)
    assert torch.equal(st, st2) and torch.equal(ls, ls2)
