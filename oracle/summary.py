"""CPU oracle for the Global16 summary refresh (test infrastructure only).

Restates the reference's fp32 torch functions generically in the number of
summary slots S, new rows W, query heads Hq and KV heads Hkv:
  * position scores  -- SRT/speculative/global16_raw256_incremental.py:50-87
  * accepted merge   -- SRT/speculative/global16_raw256_incremental.py:90-166
  * full-prefix state (fp64 ground truth) -- the definition that
    vendor/specforge/modeling/draft/global16_raw256.py:829-869
    (``global_state_from_full_prefix``) computes and :871-915
    (``commit_accepted_delta``) must reproduce incrementally;
  * prefill initialisation -- SRT/speculative/global16_raw256.py:668-784
    (one FA3 ``flash_attn_with_kvcache`` per layer, non-causal, over each
    request's location-table row): that full-prefix state per request.
``SRT`` abbreviates ``vendor/sglang/python/sglang/srt``.  GQA maps query head
h to KV head ``h // (Hq // Hkv)`` (consecutive groups share a KV head).
"""

from __future__ import annotations

import torch


def position_scores(global_query: torch.Tensor, new_keys: torch.Tensor, softmax_scale: float,
                    softcap: float = 0.0, dtype=torch.float32) -> torch.Tensor:
    """``[B, Hq, S, D]`` x ``[B, W, Hkv, D]`` -> ``[B, Hq, S, W]`` fp32 scores.

    global16_raw256_incremental.py:76-87: fp32 einsum over D, times the scale,
    then ``softcap * tanh(s / softcap)`` when softcap > 0 (:44-47).
    ``dtype=torch.float64`` evaluates the same formula in fp64 (ground truth
    for tolerance checks).
    """
    batch, hq, rows, dim = global_query.shape
    w, hkv = new_keys.shape[1], new_keys.shape[2]
    groups = hq // hkv
    q = global_query.to(dtype).reshape(batch, hkv, groups, rows, dim)
    k = new_keys.to(dtype).permute(0, 2, 1, 3)
    scores = torch.einsum("bhgrd,bhwd->bhgrw", q, k) * float(softmax_scale)
    if softcap > 0:
        scores = torch.tanh(scores / softcap) * softcap
    return scores.reshape(batch, hq, rows, w)


def merge_accepted_positions(state_output, state_lse, position_scores_, accepted_values, accept_lens,
                             dtype=torch.float32):
    """Online-softmax merge of the first ``accept_lens[b]`` rows into (output, lse).

    global16_raw256_incremental.py:124-166 restated with W = ``accepted_values.shape[1]``:
    masked scores, ``merged = logsumexp(stack(lse, logsumexp(scores)))``,
    ``out = out * exp(lse - merged) + sum_w exp(s_w - merged) * v_w``.
    ``dtype=torch.float64`` evaluates the same formula in fp64.
    """
    batch, hq, rows, dim = state_output.shape
    w = accepted_values.shape[1]
    hkv = accepted_values.shape[2]
    positions = torch.arange(w, dtype=accept_lens.dtype)
    valid = positions[None, :] < accept_lens[:, None]
    masked = position_scores_.to(dtype).masked_fill(~valid[:, None, None, :], float("-inf"))
    merged_lse = torch.logsumexp(torch.stack((state_lse.to(dtype), torch.logsumexp(masked, dim=-1))), dim=0)
    prior_weight = torch.exp(state_lse.to(dtype) - merged_lse)
    delta_weight = torch.exp(masked - merged_lse[..., None])
    delta_weight = torch.where(valid[:, None, None, :], delta_weight, torch.zeros_like(delta_weight))
    groups = hq // hkv
    weights = delta_weight.view(batch, hkv, groups, rows, w)
    values = accepted_values.to(dtype).permute(0, 2, 1, 3)
    delta_out = torch.einsum("bhgrw,bhwd->bhgrd", weights, values).reshape(batch, hq, rows, dim)
    return state_output.to(dtype) * prior_weight[..., None] + delta_out, merged_lse


def full_prefix_state(global_query, keys, values, softmax_scale: float, dtype=torch.float64, softcap: float = 0.0):
    """Normalised attention output and LSE of every query row over a whole prefix.

    ``keys``/``values`` are ``[B, T, Hkv, D]``.  This is the quantity the
    incremental merge maintains: after folding every prefix row, the state must
    equal ``softmax(scale * q k^T) v`` with ``lse = logsumexp(scale * q k^T)``
    (scores through ``softcap * tanh(s / softcap)`` when softcap > 0).
    """
    batch, hq, rows, dim = global_query.shape
    hkv = keys.shape[2]
    groups = hq // hkv
    q = global_query.to(dtype).reshape(batch, hkv, groups, rows, dim)
    k = keys.to(dtype).permute(0, 2, 1, 3)
    v = values.to(dtype).permute(0, 2, 1, 3)
    s = torch.einsum("bhgrd,bhtd->bhgrt", q, k) * softmax_scale
    if softcap > 0:
        s = torch.tanh(s / softcap) * softcap
    lse = torch.logsumexp(s, dim=-1)
    out = torch.einsum("bhgrt,bhtd->bhgrd", torch.softmax(s, dim=-1), v)
    return out.reshape(batch, hq, rows, dim), lse.reshape(batch, hq, rows)


def summary_update(state_output, state_lse, global_query, new_keys, new_values, accept_lens,
                   softmax_scale: float, state_slots=None):
    """Score + merge in one call, updating ``state_*[state_slots[b]]``; returns new copies."""
    out = state_output.clone()
    lse = state_lse.clone()
    batch = new_keys.shape[0]
    slots = torch.arange(batch) if state_slots is None else state_slots.long()
    scores = position_scores(global_query, new_keys, softmax_scale)
    o, l = merge_accepted_positions(out[slots], lse[slots], scores, new_values, accept_lens)
    out[slots] = o
    lse[slots] = l
    return out, lse


def prefill_global_attention(global_query, key_cache, value_cache, page_table, seq_lens, softmax_scale: float,
                             softcap: float = 0.0, dtype=torch.float64):
    """One layer's prefill state: ``[B, Hq, S, D]`` output and ``[B, Hq, S]`` LSE.

    global16_raw256.py:709-760: request b attends over the pool rows
    ``page_table[b, :seq_lens[b]]`` of ``key_cache`` / ``value_cache``
    (``[N, Hkv, D]``, page size 1), non-causal, every position visible.
    ``global_query`` is ``[B, Hq, S, D]`` or ``[Hq, S, D]`` (shared).  An
    empty prefix gives a zero output and LSE -inf.  Exact (fp64) values: the
    reference's FA3 rounds the weights and its output to bf16, which the
    comparison tolerance covers.
    """
    batch = page_table.shape[0]
    if global_query.ndim == 3:
        global_query = global_query[None].expand(batch, -1, -1, -1)
    _, hq, rows, dim = global_query.shape
    out = torch.zeros(batch, hq, rows, dim, dtype=dtype)
    lse = torch.full((batch, hq, rows), float("-inf"), dtype=dtype)
    for b in range(batch):
        n = int(seq_lens[b])
        if n <= 0:
            continue
        locs = page_table[b, :n].long()
        o, l = full_prefix_state(global_query[b:b + 1], key_cache[locs][None], value_cache[locs][None],
                                 softmax_scale, dtype=dtype, softcap=softcap)
        out[b], lse[b] = o[0], l[0]
    return out, lse
