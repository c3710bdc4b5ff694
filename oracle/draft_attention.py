"""CPU oracle for the drafter attention over the three views (test infrastructure only).

Restates SRT/speculative/global16_raw256_draft_all_attention.py:52-281 in
torch fp32, one (request, query head) at a time, with the reference's
sources, order and rounding points:
  * raw     -- :122-179: blocks of ``block_n`` window rows through the page
    table; scores (q.k) * scale in fp32; rows at or past raw_lengths[b]
    invisible; an all-invisible maximum is replaced by 0 before the
    exponentials (:159-163);
  * global  -- :181-218: scores bf16(q.k) * scale; values = the fp32 state
    row ``state_slots[b]`` rounded to bf16;
  * local   -- :220-268: scores bf16(q.k) * scale, visibility from the mask;
  * each step: m' = max(m, block max), o = o * exp(m - m') + bf16(exp(s - m')) . v,
    z = z * exp(m - m') + sum exp(s - m');  out = bf16(o / z)  (:270-281).
``SRT`` abbreviates ``vendor/sglang/python/sglang/srt``.  Query head h
reads KV head h // (Hq // Hkv) for the raw and local rows.
"""

from __future__ import annotations

import torch

NEG_INF = float("-inf")


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).to(torch.float32)


def _step(m, z, acc, scores, values, visible=None):
    block_max = scores.max(dim=1).values
    nxt = torch.maximum(m, block_max)
    base = torch.where(nxt == NEG_INF, torch.zeros_like(nxt), nxt)
    old = torch.exp(m - base)
    p = torch.exp(scores - base[:, None])
    if visible is not None:
        p = torch.where(visible, p, torch.zeros_like(p))
    acc = acc * old[:, None] + _bf16(p) @ values
    z = z * old + p.sum(dim=1)
    return nxt, z, acc


def fused_global_local_raw_attention(query, global_keys, global_values, state_slots, local_keys, local_values,
                                     local_attention_mask, key_cache, value_cache, page_table, raw_lengths,
                                     softmax_scale: float, block_n: int = 64) -> torch.Tensor:
    """``[B, Hq, 7, D]`` bf16 output; shapes as in the reference contract
    (key/value cache ``[S, 1, Hkv, D]``, page table ``[B, 256]``)."""
    batch, hq, rows, dim = query.shape
    hkv = local_keys.shape[1]
    groups = hq // hkv
    width = page_table.shape[1]
    out = torch.empty(batch, hq, rows, dim, dtype=torch.bfloat16)
    for b in range(batch):
        raw_len = max(0, min(int(raw_lengths[b]), width))
        slot = int(state_slots[b])
        for h in range(hq):
            kvh = h // groups
            q = query[b, h].float()
            m = torch.full((rows,), NEG_INF)
            z = torch.zeros(rows)
            acc = torch.zeros(rows, dim)
            for start in range(0, width, block_n):
                cols = torch.arange(start, start + block_n)
                vis = cols < raw_len
                if not bool(vis.any()):
                    continue              # an all-invisible block leaves (m, z, acc) unchanged
                locs = page_table[b, cols.clamp(max=raw_len - 1)].long()
                k = key_cache[locs, 0, kvh].float() * vis[:, None]
                v = value_cache[locs, 0, kvh].float() * vis[:, None]
                s = (q @ k.T) * softmax_scale
                s = torch.where(vis[None, :], s, torch.full_like(s, NEG_INF))
                m, z, acc = _step(m, z, acc, s, v)
            s = _bf16(q @ global_keys[b, h].float().T) * softmax_scale
            m, z, acc = _step(m, z, acc, s, _bf16(global_values[slot, h].float()))
            s = _bf16(q @ local_keys[b, kvh].float().T) * softmax_scale
            vis = local_attention_mask[b].bool()
            s = torch.where(vis, s, torch.full_like(s, NEG_INF))
            m, z, acc = _step(m, z, acc, s, local_values[b, kvh].float(), visible=vis)
            out[b, h] = (acc / z[:, None]).to(torch.bfloat16)
    return out


def fused_global_local_raw_merge(query, global_keys, global_values, state_slots, local_keys, local_values,
                                 local_attention_mask, raw_output, raw_lse, softmax_scale: float,
                                 softcap: float = 0.0) -> torch.Tensor:
    """Merge form, SRT/speculative/global16_raw256_draft_fused.py:138-312:
    summary and local sources normalised on their own (bf16 weights and
    values, the weighted sum rounded to bf16, divided by the fp32 sum),
    scores bf16(q.k) * scale then ``softcap * tanh(s / softcap)``; merged with
    ``raw_output [B*7, Hq, D]`` / ``raw_lse [B*7, Hq]`` by their LSEs; a row
    with no visible local row leaves that term out.  bf16 output."""
    batch, hq, rows, dim = query.shape
    hkv = local_keys.shape[1]
    groups = hq // hkv

    def finish(s):
        s = _bf16(s) * softmax_scale
        return torch.tanh(s / softcap) * softcap if softcap > 0 else s

    out = torch.empty(batch, hq, rows, dim, dtype=torch.bfloat16)
    for b in range(batch):
        slot = int(state_slots[b])
        vis = local_attention_mask[b].bool()
        has = vis.any(dim=1)
        for h in range(hq):
            kvh = h // groups
            q = query[b, h].float()
            s = finish(q @ global_keys[b, h].float().T)
            gmax = s.max(dim=1).values
            w = torch.exp(s - gmax[:, None])
            gz = w.sum(dim=1)
            g_out = _bf16(_bf16(w) @ _bf16(global_values[slot, h].float())) / gz[:, None]
            g_lse = gmax + torch.log(gz)
            s = finish(q @ local_keys[b, kvh].float().T)
            s = torch.where(vis, s, torch.full_like(s, NEG_INF))
            safe = torch.where(has, s.max(dim=1).values, torch.zeros(rows))
            w = torch.where(vis, torch.exp(s - safe[:, None]), torch.zeros_like(s))
            lz = torch.where(has, w.sum(dim=1), torch.ones(rows))
            l_out = _bf16(_bf16(w) @ local_values[b, kvh].float()) / lz[:, None]
            l_lse = torch.where(has, safe + torch.log(lz), torch.full((rows,), NEG_INF))
            r_lse = raw_lse[b * rows:(b + 1) * rows, h].float()
            r_out = raw_output[b * rows:(b + 1) * rows, h].float()
            mm = torch.maximum(r_lse, torch.maximum(g_lse, l_lse))
            rw, gw = torch.exp(r_lse - mm), torch.exp(g_lse - mm)
            lw = torch.where(has, torch.exp(l_lse - mm), torch.zeros(rows))
            merged = (r_out * rw[:, None] + g_out * gw[:, None] + l_out * lw[:, None]) / (rw + gw + lw)[:, None]
            out[b, h] = merged.to(torch.bfloat16)
    return out
