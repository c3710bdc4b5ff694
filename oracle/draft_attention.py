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
