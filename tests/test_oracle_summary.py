"""Pin the summary oracle (CPU only).

Checks that do not restate the oracle's formulas:
  * position scores against explicit python loops with the GQA head mapping
    written out (query head h reads KV head h // (Hq // Hkv));
  * the reference's own invariant: folding a prefix chunk by chunk with the
    incremental merge equals the fp64 softmax-attention state of the whole
    prefix (vendor/specforge/modeling/draft/global16_raw256.py:829-915);
  * an empty prior (lse = -inf) gives plain softmax attention over the
    accepted rows; rows at or past accept_len have no influence;
  * softcap's closed form c * tanh(s / c).
"""

import math

import pytest
import torch

from oracle import summary as osm


def loop_scores(q, k, scale):
    b_, hq, s_, d_ = q.shape
    w_, hkv = k.shape[1], k.shape[2]
    g = hq // hkv
    out = torch.zeros(b_, hq, s_, w_, dtype=torch.float64)
    for b in range(b_):
        for h in range(hq):
            for r in range(s_):
                for w in range(w_):
                    acc = 0.0
                    for d in range(d_):
                        acc += float(q[b, h, r, d]) * float(k[b, w, h // g, d])
                    out[b, h, r, w] = acc * scale
    return out


@pytest.mark.parametrize("hq,hkv", [(4, 1), (4, 2), (5, 1), (6, 3)])
def test_position_scores_match_loops(hq, hkv):
    g = torch.Generator().manual_seed(hq * 10 + hkv)
    q = torch.randn(2, hq, 3, 4, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 5, hkv, 4, generator=g).to(torch.bfloat16)
    got = osm.position_scores(q, k, 0.5)
    ref = loop_scores(q, k, 0.5)
    assert torch.allclose(got.double(), ref, rtol=1e-6, atol=1e-6)


def test_softcap_closed_form():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 2, 8, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 3, 1, 8, generator=g).to(torch.bfloat16)
    plain = loop_scores(q, k, 1.0)
    capped = osm.position_scores(q, k, 1.0, softcap=2.0).double()
    assert torch.allclose(capped, 2.0 * torch.tanh(plain / 2.0), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (10, 2)])
def test_incremental_merge_equals_full_prefix(hq, hkv):
    """Chunked folding reproduces the whole-prefix attention state."""
    g = torch.Generator().manual_seed(hq)
    batch, rows, dim, prefix = 3, 4, 16, 20
    scale = dim ** -0.5
    q = torch.randn(batch, hq, rows, dim, generator=g).to(torch.bfloat16)
    keys = torch.randn(batch, 64, hkv, dim, generator=g).to(torch.bfloat16)
    values = torch.randn(batch, 64, hkv, dim, generator=g).to(torch.bfloat16)
    out, lse = osm.full_prefix_state(q, keys[:, :prefix], values[:, :prefix], scale, dtype=torch.float64)
    out, lse = out.float(), lse.float()
    pos = torch.full((batch,), prefix)
    width = 8
    for step in range(5):
        lens = torch.tensor([(step + b) % width + 1 for b in range(batch)], dtype=torch.int32)
        idx = pos[:, None] + torch.arange(width)[None, :]
        nk = torch.stack([keys[b, idx[b]] for b in range(batch)])
        nv = torch.stack([values[b, idx[b]] for b in range(batch)])
        sc = osm.position_scores(q, nk, scale)
        out, lse = osm.merge_accepted_positions(out, lse, sc, nv, lens)
        pos = pos + lens.long()
    for b in range(batch):
        n = int(pos[b])
        o_ref, l_ref = osm.full_prefix_state(q[b:b + 1], keys[b:b + 1, :n], values[b:b + 1, :n], scale)
        assert torch.allclose(out[b].double(), o_ref[0], rtol=1e-5, atol=1e-5)
        assert torch.allclose(lse[b].double(), l_ref[0], rtol=1e-5, atol=1e-5)


def test_empty_prior_is_softmax_attention():
    g = torch.Generator().manual_seed(9)
    batch, hq, hkv, rows, dim, width = 2, 4, 2, 3, 8, 6
    sc = torch.randn(batch, hq, rows, width, generator=g)
    v = torch.randn(batch, width, hkv, dim, generator=g).to(torch.bfloat16)
    lens = torch.tensor([3, 6], dtype=torch.int32)
    out0 = torch.zeros(batch, hq, rows, dim)
    lse0 = torch.full((batch, hq, rows), -math.inf)
    out, lse = osm.merge_accepted_positions(out0, lse0, sc, v, lens)
    for b in range(batch):
        n = int(lens[b])
        for h in range(hq):
            p = torch.softmax(sc[b, h, :, :n].double(), -1)
            ref = p @ v[b, :n, h // (hq // hkv)].double()
            assert torch.allclose(out[b, h].double(), ref, rtol=1e-5, atol=1e-6)
            assert torch.allclose(lse[b, h].double(), torch.logsumexp(sc[b, h, :, :n].double(), -1), rtol=1e-6)


def test_rows_past_accept_len_do_not_matter():
    g = torch.Generator().manual_seed(5)
    batch, hq, hkv, rows, dim, width = 2, 4, 1, 2, 8, 8
    sc = torch.randn(batch, hq, rows, width, generator=g)
    v = torch.randn(batch, width, hkv, dim, generator=g)
    out0 = torch.randn(batch, hq, rows, dim, generator=g)
    lse0 = torch.randn(batch, hq, rows, generator=g)
    lens = torch.tensor([2, 5], dtype=torch.int32)
    a = osm.merge_accepted_positions(out0, lse0, sc, v, lens)
    sc2, v2 = sc.clone(), v.clone()
    sc2[0, :, :, 2:] = 1e4
    v2[1, 5:] = 1e30
    b = osm.merge_accepted_positions(out0, lse0, sc2, v2, lens)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _pool(g, n, hkv, dim, dtype=torch.bfloat16):
    return torch.randn(n, hkv, dim, generator=g).to(dtype), torch.randn(n, hkv, dim, generator=g).to(dtype)


@pytest.mark.parametrize("hq,hkv", [(8, 2), (5, 1)])
def test_prefill_equals_empty_prior_folding(hq, hkv):
    """The prefill state through a permuted location table equals folding the
    prefix from an empty state (lse -inf) with the incremental merge."""
    g = torch.Generator().manual_seed(40 + hq)
    batch, rows, dim, n = 3, 4, 16, 200
    scale = dim ** -0.5
    q = torch.randn(batch, hq, rows, dim, generator=g).to(torch.bfloat16)
    kc, vc = _pool(g, n, hkv, dim)
    table = torch.randperm(n, generator=g)[: batch * 40].view(batch, 40).to(torch.int32)
    lens = torch.tensor([40, 17, 1], dtype=torch.int32)
    out, lse = osm.prefill_global_attention(q, kc, vc, table, lens, scale)
    for b in range(batch):
        o = torch.zeros(1, hq, rows, dim)
        l = torch.full((1, hq, rows), -math.inf)
        width = 8
        for p0 in range(0, int(lens[b]), width):
            m = min(width, int(lens[b]) - p0)
            locs = torch.full((width,), int(table[b, p0]), dtype=torch.long)
            locs[:m] = table[b, p0:p0 + m].long()
            sc = osm.position_scores(q[b:b + 1], kc[locs][None], scale)
            o, l = osm.merge_accepted_positions(o, l, sc, vc[locs][None], torch.tensor([m], dtype=torch.int32))
        assert torch.allclose(out[b].float(), o[0], rtol=1e-5, atol=1e-5)
        assert torch.allclose(lse[b].float(), l[0], rtol=1e-5, atol=1e-5)


def test_prefill_matches_library_attention():
    """Output against torch's scaled_dot_product_attention (fp64, KV heads
    repeated over consecutive query-head groups)."""
    g = torch.Generator().manual_seed(44)
    batch, hq, hkv, rows, dim, n = 2, 6, 2, 5, 32, 90
    scale = 0.3
    q = torch.randn(hq, rows, dim, generator=g).to(torch.bfloat16)   # shared by the requests
    kc, vc = _pool(g, n, hkv, dim)
    table = torch.stack([torch.randperm(n, generator=g)[:60] for _ in range(batch)]).to(torch.int64)
    lens = torch.tensor([60, 23], dtype=torch.int32)
    out, _ = osm.prefill_global_attention(q, kc, vc, table, lens, scale)
    for b in range(batch):
        locs = table[b, : int(lens[b])]
        k = kc[locs].double().permute(1, 0, 2).repeat_interleave(hq // hkv, dim=0)
        v = vc[locs].double().permute(1, 0, 2).repeat_interleave(hq // hkv, dim=0)
        ref = torch.nn.functional.scaled_dot_product_attention(q.double(), k, v, scale=scale)
        assert torch.allclose(out[b], ref, rtol=1e-10, atol=1e-12)


def test_prefill_closed_forms():
    g = torch.Generator().manual_seed(45)
    hq, hkv, rows, dim, scale, cap = 4, 2, 3, 8, 0.5, 2.0
    q = torch.randn(1, hq, rows, dim, generator=g).to(torch.bfloat16)
    kc, vc = _pool(g, 10, hkv, dim)
    # one prefix token: output = its value row, lse = its (capped) score
    table = torch.tensor([[7, 0, 0]], dtype=torch.int32)
    out, lse = osm.prefill_global_attention(q, kc, vc, table, torch.tensor([1]), scale, softcap=cap)
    for h in range(hq):
        kv = h // (hq // hkv)
        assert torch.allclose(out[0, h], vc[7, kv].double()[None].expand(rows, -1))
        s = (q[0, h].double() @ kc[7, kv].double()) * scale
        assert torch.allclose(lse[0, h], cap * torch.tanh(s / cap))
    # n copies of one key: output = mean of the values, lse = s + ln n
    kc[:, :] = kc[3]
    table = torch.tensor([[0, 1, 2, 3, 4, 5]], dtype=torch.int32)
    out, lse = osm.prefill_global_attention(q, kc, vc, table, torch.tensor([6]), scale)
    for h in range(hq):
        kv = h // (hq // hkv)
        assert torch.allclose(out[0, h], vc[:6, kv].double().mean(0)[None].expand(rows, -1))
        s = (q[0, h].double() @ kc[3, kv].double()) * scale
        assert torch.allclose(lse[0, h], s + math.log(6))
    # empty prefix
    out, lse = osm.prefill_global_attention(q, kc, vc, table, torch.tensor([0]), scale)
    assert bool((out == 0).all()) and bool(torch.isneginf(lse).all())
