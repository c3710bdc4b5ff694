"""One verify-and-refresh round captured in a HIP graph and replayed.

The round is the fused stochastic verify (batch 8 x block 16 x vocab
151,936, the benchmark's sampling configuration and call), the committed
lengths ``accept + 1`` computed on the device, the summary update of 4
layers with those lengths, and the 256-token window gather of 4 layers.
Before capture, one eager round on the capture stream builds the
workspaces, and ``layer_pointers.prepare`` builds the pools' pointer arrays
(a host-to-device copy, which a graph cannot record).  The graph is then
replayed 3 times with eager work and host synchronisations between the
replays; before each replay the summary state is reset to its initial
values, and after each replay every output must equal the eager round's.
"""

import pytest
import torch

from longspark_amd import kvwindow, penalties, summary, verify, workloads

pytestmark = pytest.mark.gpu


def _round(d, p, tables_in, refresh):
    tables = penalties.build_penalty_tables(tables_in["history"], d["logits"].shape[1],
                                            repetition=tables_in["repetition"])
    acc, bonus = verify.verify_sample(
        logits=d["logits"], candidates=d["candidates"], width=16, temperatures=p.temperatures, top_ks=p.top_ks,
        top_ps=p.top_ps, min_ps=p.min_ps, max_top_k=50, draft_logits=d["draft_logits"],
        draft_token_probs=d["draft_token_probs"], draft_top_ks=p.top_ks, draft_top_ps=p.top_ps,
        uniforms=d["uniforms"], final_uniforms=d["final_uniforms"], penalties=tables, scan_hint=1)
    r = refresh
    lens = (acc + 1).clamp_(0, 16)
    summary.summary_update(query=r["query"], key_cache=r["k"], value_cache=r["v"], accepted_cache_locs=r["locs"],
                           accept_lens=lens, state_output=r["state"], state_lse=r["lse"],
                           softmax_scale=128 ** -0.5)
    kvwindow.gather_window(r["k"], r["v"], r["table"], r["seq"], page_size=r["page"], window=r["window"],
                           out=r["out"])
    return acc, bonus, lens


def test_round_graph_capture_and_replay(dev):
    batch, layers = 8, 4
    d = workloads.verify_bench_inputs(dev, batch=batch)
    p = d["params"]
    hist = dict(history=d["history"], repetition=d["repetition"])
    r = workloads.full_round_refresh_inputs(dev, batch=batch, layers=layers)
    r["out"] = torch.empty(batch, layers, 2, 8, 256, 128, dtype=torch.bfloat16, device=dev)
    state0, lse0 = r["state"].clone(), r["lse"].clone()

    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        kvwindow.layer_pointers.prepare(r["k"], r["v"])
        acc_e, bonus_e, lens_e = _round(d, p, hist, r)       # eager round on the capture stream
    torch.cuda.synchronize()
    ref = dict(acc=acc_e.cpu(), bonus=bonus_e.cpu(), lens=lens_e.cpu(), state=r["state"].cpu(),
               lse=r["lse"].cpu(), out=r["out"].cpu())
    print(f"eager round: accept {ref['acc'].tolist()}", flush=True)

    r["state"].copy_(state0)
    r["lse"].copy_(lse0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        acc_g, bonus_g, lens_g = _round(d, p, hist, r)
    torch.cuda.synchronize()

    for replay in range(3):
        # eager work between replays: clobber the outputs, reset the state
        r["out"].fill_(0)
        r["state"].copy_(state0)
        r["lse"].copy_(lse0)
        junk = torch.randn(1 << 20, device=dev).sum()
        torch.cuda.synchronize()
        print(f"replay {replay}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(acc_g.cpu(), ref["acc"]), replay
        assert torch.equal(bonus_g.cpu(), ref["bonus"]), replay
        assert torch.equal(lens_g.cpu(), ref["lens"]), replay
        assert torch.equal(r["state"].cpu(), ref["state"]), replay
        assert torch.equal(r["lse"].cpu(), ref["lse"]), replay
        assert torch.equal(r["out"].cpu().view(torch.int16), ref["out"].view(torch.int16)), replay
        del junk
    # the eager path still works after the graph and agrees with it
    r["state"].copy_(state0)
    r["lse"].copy_(lse0)
    acc2, bonus2, _ = _round(d, p, hist, r)
    torch.cuda.synchronize()
    assert torch.equal(acc2.cpu(), ref["acc"]) and torch.equal(bonus2.cpu(), ref["bonus"])
    assert torch.equal(r["state"].cpu(), ref["state"])


def test_pointer_array_lookup_during_capture_needs_prepare(dev):
    k = [torch.zeros(16, 2, 64, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    v = [torch.zeros(16, 2, 64, dtype=torch.bfloat16, device=dev) for _ in range(2)]
    table = torch.zeros(1, 1, dtype=torch.int32, device=dev)
    seq = torch.full((1,), 16, dtype=torch.int64, device=dev)
    out = torch.empty(1, 2, 2, 2, 16, 64, dtype=torch.bfloat16, device=dev)
    s = torch.cuda.Stream(dev)
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="prepare"):
        with torch.cuda.graph(g, stream=s):
            kvwindow.gather_window(k, v, table, seq, page_size=16, window=16, out=out)
    torch.cuda.synchronize()
