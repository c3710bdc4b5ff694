"""CPU oracle for the Raw256 recent-window refresh (test infrastructure only).

  * page table      -- SRT/speculative/global16_raw256_draft_fused.py:35-65 and
                       the torch path SRT/speculative/global16_raw256.py:1343-1361
  * ring table      -- src/longspark/engine/draft.py:14-21
  * window gather   -- the full recent window, gathered through a paged table
                       (the per-layer ``k[locations]`` export of
                       src/longspark/engine/target.py:213-228, generalised to a
                       page size)
  * ring append     -- src/longspark/engine/draft.py:207-212, 255-259
``SRT`` abbreviates ``vendor/sglang/python/sglang/srt``.
"""

from __future__ import annotations

import torch


def raw_page_table(req_to_token, req_pool_indices, seq_lens, window: int = 256):
    """``page_table[b, i] = req_to_token[slot_b, seq_b - raw_b + i]`` for ``i < raw_b``, else 0."""
    batch = req_pool_indices.shape[0]
    table = torch.zeros(batch, window, dtype=torch.int32)
    raw = seq_lens.clamp(max=window).to(torch.int32)
    for b in range(batch):
        n = int(raw[b])
        start = int(seq_lens[b]) - n
        slot = int(req_pool_indices[b])
        table[b, :n] = req_to_token[slot, start:start + n].to(torch.int32)
    return table, raw


def ring_page_table(slots, lengths, window: int = 256):
    """src/longspark/engine/draft.py:14-21 restated."""
    raw = lengths.clamp_max(window).int()
    offsets = torch.arange(window)
    pages = slots[:, None].long() * window + (lengths[:, None].long() - raw[:, None] + offsets).remainder(window)
    return pages.int(), raw


def window_locations(page_table, seq_lens, page_size: int, window: int = 256):
    """Physical token rows of each request's last ``min(seq, window)`` positions.

    ``page_table[b, j]`` is the physical page of logical page j; the location of
    logical position t is ``page_table[b, t // ps] * ps + t % ps``.  Returns
    ``(locs [B, window] int64, raw [B])``; entries at ``i >= raw`` are -1.
    """
    batch = seq_lens.shape[0]
    locs = torch.full((batch, window), -1, dtype=torch.int64)
    raw = seq_lens.clamp(max=window)
    for b in range(batch):
        n = int(raw[b])
        pos = torch.arange(int(seq_lens[b]) - n, int(seq_lens[b]))
        locs[b, :n] = page_table[b, pos // page_size].long() * page_size + pos % page_size
    return locs, raw


def gather_window(k_pool, v_pool, page_table, seq_lens, page_size: int, window: int = 256):
    """Gather ``[B, L, 2, Hkv, window, D]`` from per-layer pools ``[L, N, Hkv, D]``.

    Row i of the window holds position ``seq - raw + i``; rows at ``i >= raw``
    are zero.
    """
    layers, _, hkv, dim = k_pool.shape
    locs, raw = window_locations(page_table, seq_lens, page_size, window)
    batch = seq_lens.shape[0]
    out = torch.zeros(batch, layers, 2, hkv, window, dim, dtype=k_pool.dtype)
    for b in range(batch):
        n = int(raw[b])
        if n == 0:
            continue
        rows = locs[b, :n]
        out[b, :, 0, :, :n] = k_pool[:, rows].permute(0, 2, 1, 3)
        out[b, :, 1, :, :n] = v_pool[:, rows].permute(0, 2, 1, 3)
    return out


def ring_append(ring_keys, ring_values, rows_k, rows_v, slots, previous_lengths, counts, window: int = 256):
    """Write ``counts[b]`` new rows per request at ``slot * window + pos % window``.

    ``rows_*`` are ``[L, N, Hkv, D]`` packed request after request
    (draft.py:228-243 builds the same ``ring_locs``).  Returns new copies.
    """
    rk, rv = ring_keys.clone(), ring_values.clone()
    locs = []
    for b in range(slots.shape[0]):
        prev, n = int(previous_lengths[b]), int(counts[b])
        locs.extend(int(slots[b]) * window + pos % window for pos in range(prev, prev + n))
    locs = torch.tensor(locs, dtype=torch.int64)
    rk[:, locs] = rows_k
    rv[:, locs] = rows_v
    return rk, rv
