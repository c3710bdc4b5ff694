"""Pin the drafter-attention oracle (CPU only).

Checks that do not restate the oracle's steps:
  * it equals one softmax attention (fp64) over the concatenation of the
    visible raw rows, the 16 summary rows and the visible local rows, with
    the reference's scores (raw fp32, global/local rounded to bf16), within
    the bound that rounding the weights and the output to bf16 allows;
    the raw rows, key/value heads and summary slot of that reference are
    gathered with explicit loops;
  * closed form: with no raw or local rows and 16 equal summary keys the
    output is the mean of the bf16-rounded summary values;
  * the raw block size does not matter beyond the weight rounding.
"""

import torch

from oracle import draft_attention as oda


def make(seed, batch=2, hq=4, hkv=2, pool=300, lens=(200, 37)):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, hq, 7, 128, generator=g).to(torch.bfloat16) * 0.3
    gk = torch.randn(batch, hq, 16, 128, generator=g).to(torch.bfloat16) * 0.3
    gv = torch.randn(batch + 2, hq, 16, 128, generator=g)
    slots = torch.tensor([batch + 1, 0][:batch], dtype=torch.int32)
    lk = torch.randn(batch, hkv, 7, 128, generator=g).to(torch.bfloat16) * 0.3
    lv = torch.randn(batch, hkv, 7, 128, generator=g).to(torch.bfloat16)
    mask = torch.rand(batch, 7, 7, generator=g) < 0.6
    kc = (torch.randn(pool, 1, hkv, 128, generator=g) * 0.3).to(torch.bfloat16)
    vc = torch.randn(pool, 1, hkv, 128, generator=g).to(torch.bfloat16)
    pt = torch.stack([torch.randperm(pool, generator=g)[:256] for _ in range(batch)]).to(torch.int32)
    rl = torch.tensor(lens[:batch], dtype=torch.int32)
    return q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl


def concat_reference(q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl, scale):
    batch, hq = q.shape[:2]
    hkv = lk.shape[1]
    out = torch.zeros(batch, hq, 7, 128, dtype=torch.float64)
    wabs = torch.zeros_like(out)
    for b in range(batch):
        for h in range(hq):
            kvh = h // (hq // hkv)
            keys, vals = [], []
            for t in range(int(rl[b])):
                keys.append(kc[int(pt[b, t]), 0, kvh].double())
                vals.append(vc[int(pt[b, t]), 0, kvh].double())
            for r in range(7):
                qs = q[b, h, r].double()
                sc = [float(qs @ k) * scale for k in keys]
                sc += [float(torch.tensor(float(qs @ gk[b, h, j].double())).to(torch.bfloat16)) * scale
                       for j in range(16)]
                vv = vals + [gv[int(slots[b]), h, j].to(torch.bfloat16).double() for j in range(16)]
                for j in range(7):
                    if bool(mask[b, r, j]):
                        sc.append(float(torch.tensor(float(qs @ lk[b, kvh, j].double())).to(torch.bfloat16)) * scale)
                        vv.append(lv[b, kvh, j].double())
                p = torch.softmax(torch.tensor(sc, dtype=torch.float64), 0)
                V = torch.stack(vv)
                out[b, h, r] = p @ V
                wabs[b, h, r] = p @ V.abs()
    return out, wabs


def test_oracle_equals_one_softmax_over_all_sources():
    args = make(1)
    scale = 128 ** -0.5
    got = oda.fused_global_local_raw_attention(*args, scale).double()
    ref, wabs = concat_reference(*args, scale)
    bound = 2.0 ** -8 * wabs + 2.0 ** -8 * ref.abs() + 1e-6
    assert bool(((got - ref).abs() <= bound).all()), float(((got - ref).abs() / bound).max())


def test_empty_raw_and_local_gives_mean_of_equal_summary_keys():
    q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl = make(2)
    gk[:] = gk[:, :, :1]
    mask[:] = False
    rl[:] = 0
    got = oda.fused_global_local_raw_attention(q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl, 0.1)
    for b in range(q.shape[0]):
        want = gv[int(slots[b])].to(torch.bfloat16).float().mean(dim=1)       # [Hq, D]
        assert torch.allclose(got[b].float(), want[:, None, :].expand(-1, 7, -1).to(torch.bfloat16).float(),
                              rtol=2 ** -7, atol=1e-6)


def test_raw_block_size_only_moves_weight_rounding():
    args = make(3, lens=(256, 129))
    a = oda.fused_global_local_raw_attention(*args, 0.09, block_n=64).double()
    b = oda.fused_global_local_raw_attention(*args, 0.09, block_n=256).double()
    ref, wabs = concat_reference(*args, 0.09)
    assert bool(((a - b).abs() <= 2.0 ** -7 * wabs + 2.0 ** -7 * ref.abs() + 1e-6).all())


def window_attention(q, kc, vc, pt, rl, scale):
    """Exact (fp64) attention of the query rows over each request's window,
    token-major [B*7, Hq, D] output and [B*7, Hq] LSE, as the reference's
    FA3 call returns them."""
    batch, hq = q.shape[:2]
    hkv = kc.shape[2]
    out = torch.zeros(batch * 7, hq, 128, dtype=torch.float64)
    lse = torch.zeros(batch * 7, hq, dtype=torch.float64)
    for b in range(batch):
        locs = pt[b, : int(rl[b])].long()
        for h in range(hq):
            k = kc[locs, 0, h // (hq // hkv)].double()
            v = vc[locs, 0, h // (hq // hkv)].double()
            s = (q[b, h].double() @ k.T) * scale
            out[b * 7:(b + 1) * 7, h] = torch.softmax(s, 1) @ v
            lse[b * 7:(b + 1) * 7, h] = torch.logsumexp(s, 1)
    return out, lse


def test_merge_of_window_attention_equals_one_kernel_form():
    """Merging an exact window attention with the summary and local sources
    gives the one-softmax-over-everything output, within the rounding bound
    (each source's weighted sum and both outputs rounded to bf16)."""
    q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl = make(4, lens=(150, 60))
    scale = 128 ** -0.5
    raw_out, raw_lse = window_attention(q, kc, vc, pt, rl, scale)
    got = oda.fused_global_local_raw_merge(q, gk, gv, slots, lk, lv, mask, raw_out.to(torch.bfloat16),
                                           raw_lse.float(), scale).double()
    ref, wabs = concat_reference(q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl, scale)
    bound = 2.0 ** -7 * wabs + 2.0 ** -7 * ref.abs() + 1e-6
    assert bool(((got - ref).abs() <= bound).all()), float(((got - ref).abs() / bound).max())


def test_merge_softcap_closed_form():
    """One summary key repeated, no local rows and a window LSE of -inf:
    the output is the mean of the summary values, whatever the softcap."""
    q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl = make(5)
    gk[:] = gk[:, :, :1]
    mask[:] = False
    raw_out = torch.randn(q.shape[0] * 7, q.shape[1], 128).to(torch.bfloat16)
    raw_lse = torch.full((q.shape[0] * 7, q.shape[1]), float("-inf"))
    for cap in (0.0, 3.0):
        got = oda.fused_global_local_raw_merge(q, gk, gv, slots, lk, lv, mask, raw_out, raw_lse, 0.2, softcap=cap)
        for b in range(q.shape[0]):
            want = gv[int(slots[b])].to(torch.bfloat16).float().mean(dim=1)
            assert torch.allclose(got[b].float(), want[:, None, :].expand(-1, 7, -1), rtol=2 ** -6, atol=1e-6)
