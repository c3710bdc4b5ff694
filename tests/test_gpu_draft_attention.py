"""Drafter attention over the three views on the GPU vs the oracle.

``draft_attention.fused_global_local_raw_attention`` against
``oracle.draft_attention`` (the reference's steps and rounding points in fp32).
Both round the attention weights and the output to bf16, so a weight that
lands on a rounding boundary may round differently: output bound
2^-8 * sum p|v| + 2^-7 * |out| + 1e-6 (the weighted absolute value from the
oracle run on |v|).  Cases: 4, 5 and 1 query heads per KV head (one wave per
query head; the single-head case leaves three staging-only waves), window
lengths 0, 1, 63, 64, 65, 200, 256 and an over-long 300 (clamped to the
256-column table), random local masks including all-hidden rows, summary
state rows picked through state_slots, and the contract errors.
"""

import pytest
import torch

from longspark_amd import draft_attention as da
from oracle import draft_attention as oda

pytestmark = pytest.mark.gpu

LENS = [0, 1, 63, 64, 65, 200, 256, 300]


def make(seed, hq, hkv, lens=LENS, pool=2048):
    g = torch.Generator().manual_seed(seed)
    batch = len(lens)
    q = (0.3 * torch.randn(batch, hq, 7, 128, generator=g)).to(torch.bfloat16)
    gk = (0.3 * torch.randn(batch, hq, 16, 128, generator=g)).to(torch.bfloat16)
    gv = torch.randn(batch + 3, hq, 16, 128, generator=g)
    slots = torch.randperm(batch + 3, generator=g)[:batch].to(torch.int32)
    lk = (0.3 * torch.randn(batch, hkv, 7, 128, generator=g)).to(torch.bfloat16)
    lv = torch.randn(batch, hkv, 7, 128, generator=g).to(torch.bfloat16)
    mask = torch.rand(batch, 7, 7, generator=g) < 0.5
    mask[0, 3] = False                               # a row with no visible local row
    kc = (0.3 * torch.randn(pool, 1, hkv, 128, generator=g)).to(torch.bfloat16)
    vc = torch.randn(pool, 1, hkv, 128, generator=g).to(torch.bfloat16)
    pt = torch.stack([torch.randperm(pool, generator=g)[:256] for _ in range(batch)]).to(torch.int32)
    rl = torch.tensor(lens, dtype=torch.int32)
    return [q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl]


def run(dev, args, scale):
    q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl = [t.to(dev) for t in args]
    out = torch.empty_like(q)
    da.fused_global_local_raw_attention(query=q, global_keys=gk, global_values=gv, state_slots=slots,
                                        local_keys=lk, local_values=lv, local_attention_mask=mask,
                                        key_cache=kc, value_cache=vc, page_table=pt, raw_lengths=rl,
                                        output=out, softmax_scale=scale)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("hq,hkv", [(32, 8), (40, 8), (8, 8)])
def test_draft_attention_matches_oracle(dev, hq, hkv):
    args = make(hq * 10 + hkv, hq, hkv)
    scale = 128 ** -0.5
    print(f"draft attention hq={hq} hkv={hkv}", flush=True)
    got = run(dev, args, scale).double()
    ref = oda.fused_global_local_raw_attention(*args, scale).double()
    absargs = list(args)
    absargs[2] = args[2].abs()
    absargs[5] = args[5].abs()
    absargs[8] = args[8].abs()
    wabs = oda.fused_global_local_raw_attention(*absargs, scale).double()
    bound = 2.0 ** -8 * wabs + 2.0 ** -7 * ref.abs() + 1e-6
    err = (got - ref).abs()
    assert bool((err <= bound).all()), (float(err.max()), float((err / bound).max()))


def test_draft_attention_contract(dev):
    args = [t.to(dev) for t in make(5, 8, 2, lens=[10, 20])]
    q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl = args
    kw = dict(query=q, global_keys=gk, global_values=gv, state_slots=slots, local_keys=lk, local_values=lv,
              local_attention_mask=mask, key_cache=kc, value_cache=vc, page_table=pt, raw_lengths=rl,
              output=torch.empty_like(q), softmax_scale=0.1)
    assert da.can_use_fused_global_local_raw_attention(**{k: v for k, v in kw.items() if k != "softmax_scale"})
    with pytest.raises(ValueError, match="softcap=0"):
        da.fused_global_local_raw_attention(**kw, softcap=1.0)
    with pytest.raises(ValueError, match="violate the contract"):
        da.fused_global_local_raw_attention(**{**kw, "page_table": pt[:, :128]})
    with pytest.raises(ValueError, match="violate the contract"):
        da.fused_global_local_raw_attention(**{**kw, "local_attention_mask": mask.to(torch.int32)})


@pytest.mark.parametrize("hq,hkv,cap", [(32, 8, 0.0), (40, 8, 3.0), (8, 8, 0.0)])
def test_draft_merge_matches_oracle(dev, hq, hkv, cap):
    """Merge form: a window attention output and LSE (random here, one row's
    LSE -inf; the LSE given as a transposed view) merged with the summary and
    local sources.  Bound 2^-6 * weighted |v| + 2^-7 * |out| + 1e-6: each
    source's weighted sum and the output are rounded to bf16 on both sides."""
    q, gk, gv, slots, lk, lv, mask, kc, vc, pt, rl = make(hq + 7 * hkv, hq, hkv)
    batch = q.shape[0]
    g = torch.Generator().manual_seed(hq)
    raw_out = torch.randn(batch * 7, hq, 128, generator=g).to(torch.bfloat16)
    raw_lse = (2.0 * torch.randn(hq, batch * 7, generator=g)).t()          # [B*7, Hq], strides (1, B*7)
    raw_lse[1, 0] = float("-inf")
    scale = 128 ** -0.5
    args = [q, gk, gv, slots, lk, lv, mask]
    print(f"draft merge hq={hq} hkv={hkv} cap={cap}", flush=True)
    out = torch.empty_like(q).to(dev)
    da.fused_global_local_raw_merge(query=q.to(dev), global_keys=gk.to(dev), global_values=gv.to(dev),
                                    state_slots=slots.to(dev), local_keys=lk.to(dev), local_values=lv.to(dev),
                                    local_attention_mask=mask.to(dev), raw_output=raw_out.to(dev),
                                    raw_lse=raw_lse.to(dev), output=out, softmax_scale=scale, softcap=cap)
    torch.cuda.synchronize()
    ref = oda.fused_global_local_raw_merge(*args, raw_out, raw_lse, scale, softcap=cap).double()
    wabs = oda.fused_global_local_raw_merge(q, gk, gv.abs(), slots, lk, lv.abs(), mask, raw_out.abs(), raw_lse,
                                            scale, softcap=cap).double()
    err = (out.cpu().double() - ref).abs()
    bound = 2.0 ** -6 * wabs + 2.0 ** -7 * ref.abs() + 1e-6
    assert bool((err <= bound).all()), (float(err.max()), float((err / bound).max()))


def test_draft_merge_contract(dev):
    q, gk, gv, slots, lk, lv, mask, *_ = [t.to(dev) for t in make(6, 8, 2, lens=[10, 20])]
    raw_out = torch.zeros(q.shape[0] * 7, 8, 128, dtype=torch.bfloat16, device=dev)
    raw_lse = torch.zeros(q.shape[0] * 7, 8, device=dev)
    kw = dict(query=q, global_keys=gk, global_values=gv, state_slots=slots, local_keys=lk, local_values=lv,
              local_attention_mask=mask, raw_output=raw_out, raw_lse=raw_lse, output=torch.empty_like(q))
    assert da.can_use_fused_global_local_raw_merge(**kw)
    with pytest.raises(ValueError, match="violate the production contract"):
        da.fused_global_local_raw_merge(**{**kw, "raw_lse": raw_lse.half()}, softmax_scale=0.1)
