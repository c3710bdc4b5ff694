"""Summary state refresh on the GPU vs the CPU oracle.

Tolerances: scores within 2e-5 (the reference's own GQA-5 test,
tests/gpu/test_gqa5_attention.py:21-50, which is re-created here with its
tolerances); summary entries within 1e-5 relative of the oracle evaluated in
fp64 (tests/summary_ref.py states what "relative" means for a weighted sum).

Cases: the reference test re-created (seed 980426, batch 1 / 3 / 64, 40 query
heads over 8 KV heads, 16 rows, 8 new rows, 16 steps, strided state views,
permuted state slots) and the same with 32 query heads (GQA-4); compact
locations with offsets; fp16; head_dim 64 and 256; softcap; 256 summary rows
per KV head with 16 new rows; the fused all-layer update against per-layer
score + merge; the full-prefix invariant in fp64 after many rounds.
"""

import math

import pytest
import torch

from oracle import summary as osm
from longspark_amd import summary
from tests import summary_ref as sr

pytestmark = pytest.mark.gpu

REF_TOL = dict(rtol=3e-5, atol=3e-5)  # tests/gpu/test_gqa5_attention.py:49-50


@pytest.mark.parametrize("q_heads", [40, 32])
def test_reference_gqa_test_recreated(dev, q_heads):
    g = torch.Generator().manual_seed(980426)
    for batch in (1, 3, 64):
        print(f"summary steps Hq={q_heads} batch={batch}", flush=True)
        query = torch.randn(1, q_heads, 16, 128, generator=g).to(torch.bfloat16).expand(batch, -1, -1, -1)
        capacity = batch + 3
        out_base = torch.randn(capacity, 2, q_heads, 16, 128, generator=g)
        lse_base = torch.randn(capacity, 2, q_heads, 16, generator=g)
        slots = torch.randperm(capacity, generator=g)[:batch].to(torch.int32)
        exp_out, exp_lse = out_base[:, 1][slots.long()].clone(), lse_base[:, 1][slots.long()].clone()
        x_out, x_lse, x_mag = exp_out.double(), exp_lse.double(), exp_out.double().abs()
        out_d, lse_d = out_base.to(dev), lse_base.to(dev)
        output, lse = out_d[:, 1], lse_d[:, 1]
        qd = query.to(dev)
        for step in range(16):
            keys = torch.randn(batch, 8, 8, 128, generator=g).to(torch.bfloat16)
            values = torch.randn(batch, 8, 8, 128, generator=g).to(torch.bfloat16)
            scores = torch.empty(batch, q_heads, 16, 8, device=dev)
            summary.cache_position_scores(layer_id=0, global_query=qd, new_keys=keys.to(dev), output=scores,
                                          softmax_scale=128 ** -.5)
            ref_scores = osm.position_scores(query, keys, 128 ** -.5)
            torch.testing.assert_close(scores.cpu(), ref_scores, rtol=2e-5, atol=2e-5)
            lens = ((torch.arange(batch) + step) % 8 + 1).to(torch.int32)
            locs = torch.arange(batch * 8).reshape(batch, 8)
            exp_out, exp_lse = osm.merge_accepted_positions(exp_out, exp_lse, ref_scores, values, lens)
            x_out, x_lse, x_mag = sr.merged(x_out, x_lse, x_mag, query, keys, values, lens, 128 ** -.5)
            summary.merge_accepted_positions_(state_output=output, state_lse=lse, position_scores=scores,
                                              value_cache=values.reshape(batch * 8, 1, 8, 128).to(dev),
                                              accepted_cache_locs=locs.to(dev), accept_lens=lens.to(dev),
                                              accept_offsets=None, state_slots=slots.to(dev))
            torch.cuda.synchronize()
            # the reference test's own tolerances against the fp32 restatement ...
            torch.testing.assert_close(output.cpu()[slots.long()], exp_out, **REF_TOL)
            torch.testing.assert_close(lse.cpu()[slots.long()], exp_lse, **REF_TOL)
            # ... and 1e-5 relative against the fp64 evaluation of every merge so far
            sr.check(output.cpu()[slots.long()], lse.cpu()[slots.long()], x_out, x_lse, x_mag,
                     what=f"Hq={q_heads} B={batch} step {step}")
        # rows not addressed by a slot are untouched, as is the other half of the view
        untouched = torch.ones(capacity, dtype=torch.bool)
        untouched[slots.long()] = False
        assert torch.equal(out_d[:, 1].cpu()[untouched], out_base[:, 1][untouched])
        assert torch.equal(out_d[:, 0].cpu(), out_base[:, 0]) and torch.equal(lse_d[:, 0].cpu(), lse_base[:, 0])


def test_compact_locations_and_offsets(dev):
    g = torch.Generator().manual_seed(21)
    batch, hq, hkv = 5, 16, 4
    query = torch.randn(batch, hq, 16, 128, generator=g).to(torch.bfloat16)
    lens = torch.tensor([3, 8, 1, 0, 6], dtype=torch.int32)
    total = int(lens.sum())
    cache = torch.randn(200, 1, hkv, 128, generator=g).to(torch.bfloat16)
    flat = torch.randperm(200, generator=g)[:total]
    offs = torch.cat([torch.zeros(1, dtype=torch.int64), lens.cumsum(0)[:-1].long()])
    fixed = torch.zeros(batch, 8, dtype=torch.int64)
    for b in range(batch):
        fixed[b, :int(lens[b])] = flat[offs[b]:offs[b] + lens[b]]
    keys = cache[fixed.reshape(-1), 0].reshape(batch, 8, hkv, 128)
    scores = osm.position_scores(query, keys, 0.1)
    out0 = torch.randn(batch, hq, 16, 128, generator=g)
    lse0 = torch.randn(batch, hq, 16, generator=g)
    out, lse = out0.to(dev), lse0.to(dev)
    offsets = torch.full((batch,), -1, dtype=torch.int32, device=dev)
    summary.merge_accepted_positions_(state_output=out, state_lse=lse, position_scores=scores.to(dev),
                                      value_cache=cache.to(dev), accepted_cache_locs=flat.to(dev),
                                      accept_lens=lens.to(dev), accept_offsets=offsets)
    torch.cuda.synchronize()
    assert torch.equal(offsets.cpu(), offs.to(torch.int32))
    values = cache[fixed.reshape(-1), 0].reshape(batch, 8, hkv, 128)
    ref_o, ref_l, mag = sr.merged(out0.double(), lse0.double(), out0.double().abs(), query, keys, values, lens, 0.1)
    # accept_len 0 leaves the state row unchanged (documented contract)
    assert torch.equal(out.cpu()[3], out0[3]) and torch.equal(lse.cpu()[3], lse0[3])
    sr.check(out.cpu(), lse.cpu(), ref_o, ref_l, mag, what="compact locations")


@pytest.mark.parametrize("dim,dtype,softcap", [(64, torch.float16, 0.0), (256, torch.bfloat16, 0.0),
                                               (128, torch.bfloat16, 5.0)])
def test_scores_geometry_variants(dev, dim, dtype, softcap):
    g = torch.Generator().manual_seed(dim)
    batch, hq, hkv, rows, width = 3, 12, 4, 5, 13
    q = (3 * torch.randn(batch, hq, rows, dim, generator=g)).to(dtype)
    k = torch.randn(batch, width, hkv, dim, generator=g).to(dtype)
    out = torch.empty(batch, hq, rows, width, device=dev)
    summary.cache_position_scores(layer_id=1, global_query=q.to(dev), new_keys=k.to(dev), output=out,
                                  softmax_scale=dim ** -.5, softcap=softcap)
    torch.cuda.synchronize()
    ref = osm.position_scores(q, k, dim ** -.5, softcap=softcap)
    torch.testing.assert_close(out.cpu(), ref, rtol=2e-5, atol=2e-5)


def fused_case(dev, *, layers, batch, hq, hkv, rows, width, capacity, seed, compact=False):
    g = torch.Generator().manual_seed(seed)
    dim = 128
    query = torch.randn(layers, hq, rows, dim, generator=g).to(torch.bfloat16)
    n = 64 * batch
    kc = torch.randn(layers, n, hkv, dim, generator=g).to(torch.bfloat16)
    vc = torch.randn(layers, n, hkv, dim, generator=g).to(torch.bfloat16)
    lens = torch.randint(1, width + 1, (batch,), generator=g).to(torch.int32)
    locs = torch.stack([torch.randperm(n, generator=g)[:width] for _ in range(batch)])
    state = torch.randn(capacity, layers, hq, rows, dim, generator=g)
    lse = torch.randn(capacity, layers, hq, rows, generator=g)
    slots = torch.randperm(capacity, generator=g)[:batch].to(torch.int32)
    ref_s, ref_l, ref_m = state.double(), lse.double(), state.double().abs()
    for l in range(layers):
        nk = kc[l][locs.reshape(-1)].reshape(batch, width, hkv, dim)
        nv = vc[l][locs.reshape(-1)].reshape(batch, width, hkv, dim)
        sl = slots.long()
        o, s, m = sr.merged(ref_s[sl, l], ref_l[sl, l], ref_m[sl, l], query[l][None].expand(batch, -1, -1, -1),
                            nk, nv, lens, dim ** -.5)
        ref_s[sl, l], ref_l[sl, l], ref_m[sl, l] = o, s, m
    sd, ld = state.to(dev), lse.to(dev)
    kw = {}
    if compact:
        flat = torch.cat([locs[b, :int(lens[b])] for b in range(batch)])
        kw = dict(accepted_cache_locs=flat.to(dev), width=width,
                  accept_offsets=torch.empty(batch, dtype=torch.int32, device=dev))
    else:
        kw = dict(accepted_cache_locs=locs.to(dev))
    summary.summary_update(query=query.to(dev), key_cache=kc.to(dev), value_cache=[t.to(dev) for t in vc],
                           accept_lens=lens.to(dev), state_output=sd, state_lse=ld, softmax_scale=dim ** -.5,
                           state_slots=slots.to(dev), **kw)
    torch.cuda.synchronize()
    sr.check(sd.cpu(), ld.cpu(), ref_s, ref_l, ref_m, what=f"fused update L={layers} B={batch} Hq={hq} S={rows}")


def test_fused_update_reference_geometry(dev):
    fused_case(dev, layers=5, batch=16, hq=32, hkv=8, rows=16, width=8, capacity=20, seed=1)


def test_fused_update_gqa5_compact(dev):
    fused_case(dev, layers=3, batch=7, hq=40, hkv=8, rows=16, width=8, capacity=7, seed=2, compact=True)


def test_fused_update_256_rows_per_kv_head(dev):
    # 4 query heads x 64 rows share each KV head; 16 new rows per request
    fused_case(dev, layers=2, batch=4, hq=32, hkv=8, rows=64, width=16, capacity=6, seed=3)


def test_full_prefix_invariant_fp64(dev):
    """Many rounds of GPU merges equal softmax attention over the whole prefix (fp64)."""
    g = torch.Generator().manual_seed(77)
    batch, hq, hkv, rows, dim, width = 4, 8, 2, 16, 128, 8
    q = torch.randn(batch, hq, rows, dim, generator=g).to(torch.bfloat16)
    total = 400
    keys = torch.randn(batch, total, hkv, dim, generator=g).to(torch.bfloat16)
    vals = torch.randn(batch, total, hkv, dim, generator=g).to(torch.bfloat16)
    out, lse = osm.full_prefix_state(q, keys[:, :1], vals[:, :1], dim ** -.5)
    out, lse = out.float().to(dev), lse.float().to(dev)
    pos = torch.ones(batch, dtype=torch.int64)
    qd = q.to(dev)
    cache_k = keys.reshape(batch * total, 1, hkv, dim).to(dev)
    cache_v = vals.reshape(batch * total, 1, hkv, dim).to(dev)
    scores = torch.empty(batch, hq, rows, width, device=dev)
    for step in range(30):
        lens = torch.tensor([(step * 3 + b) % width + 1 for b in range(batch)], dtype=torch.int32)
        locs = (torch.arange(batch)[:, None] * total + pos[:, None] + torch.arange(width)[None, :])
        nk = cache_k[locs.reshape(-1).to(dev), 0].reshape(batch, width, hkv, dim)
        summary.cache_position_scores(layer_id=0, global_query=qd, new_keys=nk, output=scores,
                                      softmax_scale=dim ** -.5)
        summary.merge_accepted_positions_(state_output=out, state_lse=lse, position_scores=scores,
                                          value_cache=cache_v, accepted_cache_locs=locs.to(dev),
                                          accept_lens=lens.to(dev), accept_offsets=None)
        pos += lens.long()
    torch.cuda.synchronize()
    for b in range(batch):
        n = int(pos[b])
        o_ref, l_ref = osm.full_prefix_state(q[b:b + 1], keys[b:b + 1, :n], vals[b:b + 1, :n], dim ** -.5)
        # magnitude of the summands: the same attention over |v|
        m_ref, _ = osm.full_prefix_state(q[b:b + 1], keys[b:b + 1, :n], vals[b:b + 1, :n].abs(), dim ** -.5)
        sr.check(out[b].cpu(), lse[b].cpu(), o_ref[0], l_ref[0], m_ref[0], what=f"full prefix b={b} n={n}")
