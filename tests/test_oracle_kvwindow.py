"""Pin the recent-window oracle (CPU only).

The ground truth is built independently of the oracle's index formulas:
each request's logical token sequence is generated first, then scattered into
a paged pool through a random page permutation (as an allocator would); the
window gather must return the last min(seq, window) logical rows.  The ring
is checked by simulating token-by-token appends.
"""

import pytest
import torch

from oracle import kvwindow as okw


def paged_pool(seqs, page_size, layers, heads, dim, seed, spare_pages=3):
    """Scatter logical sequences into one shuffled paged pool.

    Returns (k_pool, v_pool [L, N, H, D], page_table [B, max_pages], logical K/V per request)."""
    g = torch.Generator().manual_seed(seed)
    pages_per = [(s + page_size - 1) // page_size for s in seqs]
    total_pages = sum(pages_per) + spare_pages
    perm = torch.randperm(total_pages, generator=g)
    n = total_pages * page_size
    k_pool = torch.randn(layers, n, heads, dim, generator=g)
    v_pool = torch.randn(layers, n, heads, dim, generator=g)
    table = torch.zeros(len(seqs), max(pages_per + [1]), dtype=torch.int32)
    logical = []
    nxt = 0
    for b, s in enumerate(seqs):
        lk = torch.randn(layers, s, heads, dim, generator=g)
        lv = torch.randn(layers, s, heads, dim, generator=g)
        for p in range(pages_per[b]):
            phys = int(perm[nxt]); nxt += 1
            table[b, p] = phys
            lo, hi = p * page_size, min(s, (p + 1) * page_size)
            k_pool[:, phys * page_size:phys * page_size + hi - lo] = lk[:, lo:hi]
            v_pool[:, phys * page_size:phys * page_size + hi - lo] = lv[:, lo:hi]
        logical.append((lk, lv))
    return k_pool, v_pool, table, logical


@pytest.mark.parametrize("page_size", [1, 16])
def test_gather_window_returns_last_logical_rows(page_size):
    window = 32
    seqs = [0, 1, 15, 16, 17, 32, 33, 64, 100]
    k_pool, v_pool, table, logical = paged_pool(seqs, page_size, 2, 3, 4, seed=page_size)
    out = okw.gather_window(k_pool, v_pool, table, torch.tensor(seqs), page_size, window)
    for b, s in enumerate(seqs):
        raw = min(s, window)
        lk, lv = logical[b]
        assert torch.equal(out[b, :, 0, :, :raw], lk[:, s - raw:s].permute(0, 2, 1, 3))
        assert torch.equal(out[b, :, 1, :, :raw], lv[:, s - raw:s].permute(0, 2, 1, 3))
        assert out[b, :, :, :, raw:].abs().sum() == 0


def test_raw_page_table_brute_force():
    g = torch.Generator().manual_seed(0)
    rtt = torch.randint(0, 10_000, (6, 600), generator=g, dtype=torch.int32)
    slots = torch.tensor([4, 0, 5, 2])
    seqs = torch.tensor([0, 255, 256, 599])
    table, raw = okw.raw_page_table(rtt, slots, seqs, 256)
    for b in range(4):
        s, n = int(seqs[b]), min(int(seqs[b]), 256)
        assert int(raw[b]) == n
        for i in range(256):
            want = int(rtt[int(slots[b]), s - n + i]) if i < n else 0
            assert int(table[b, i]) == want


def test_ring_table_matches_append_simulation():
    window, slots = 8, [3, 0, 1]
    ring = {}
    lengths = [0, 0, 0]
    g = torch.Generator().manual_seed(1)
    history = [[], [], []]
    for _ in range(12):
        counts = torch.randint(1, 4, (3,), generator=g).tolist()
        rows_k = torch.arange(sum(counts)).float()[None, :, None, None] + 1000 * len(ring)
        ring_k = torch.zeros(1, 4 * window, 1, 1)
        for loc, val in ring.items():
            ring_k[0, loc] = val
        rk, _ = okw.ring_append(ring_k, ring_k.clone(), rows_k, rows_k, torch.tensor(slots), torch.tensor(lengths),
                                torch.tensor(counts), window)
        off = 0
        for b in range(3):
            for j in range(counts[b]):
                history[b].append(float(rows_k[0, off + j]))
            off += counts[b]
            lengths[b] += counts[b]
        ring = {i: rk[0, i].clone() for i in range(4 * window) if rk[0, i].abs().sum() > 0}
        pages, raw = okw.ring_page_table(torch.tensor(slots), torch.tensor(lengths), window)
        for b in range(3):
            n = int(raw[b])
            assert n == min(lengths[b], window)
            got = [float(rk[0, int(pages[b, i]), 0, 0]) for i in range(n)]
            assert got == history[b][-n:]
