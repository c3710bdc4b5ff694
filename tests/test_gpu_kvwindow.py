"""Recent-window refresh on the GPU vs the CPU oracle (bit-exact copies).

Cases: page sizes 1 and 16 (SGLang's req_to_token as a page-size-one table
through table_rows); sequence lengths 0, 1, 15, 16, 17, 255, 256, 257 and
4096 (padding, page and window boundaries); bf16, fp16 and fp32 pools; a
strided output view; the Raw256 page-table builder on int32 and int64
metadata; the ring table; ring append from packed rows and fused with the
target export (source locations), with wrap-around; the selected-row export.
"""

import pytest
import torch

from oracle import kvwindow as okw
from longspark_amd import kvwindow

pytestmark = pytest.mark.gpu

SEQS = [0, 1, 15, 16, 17, 255, 256, 257, 4096]


def make_pool(seqs, page_size, layers, heads, dim, dtype, seed, spare=5):
    g = torch.Generator().manual_seed(seed)
    pages = [(s + page_size - 1) // page_size for s in seqs]
    total = sum(pages) + spare
    perm = torch.randperm(total, generator=g)
    table = torch.zeros(len(seqs), max(pages + [1]), dtype=torch.int32)
    nxt = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[nxt:nxt + n].to(torch.int32)
        nxt += n
    k = torch.randn(layers, total * page_size, heads, dim, generator=g).to(dtype)
    v = torch.randn(layers, total * page_size, heads, dim, generator=g).to(dtype)
    return k, v, table


@pytest.mark.parametrize("page_size", [1, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_window_gather_matches_oracle(dev, page_size, dtype):
    print(f"window gather ps={page_size} dtype={dtype}", flush=True)
    k, v, table = make_pool(SEQS, page_size, 3, 2, 128, dtype, seed=page_size)
    seqs = torch.tensor(SEQS, dtype=torch.int64)
    raw = torch.empty(len(SEQS), dtype=torch.int32, device=dev)
    out = kvwindow.gather_window([t.to(dev) for t in k], [t.to(dev) for t in v], table.to(dev), seqs.to(dev),
                                 page_size=page_size, raw_lengths=raw)
    torch.cuda.synchronize()
    ref = okw.gather_window(k, v, table, seqs, page_size, 256)
    assert torch.equal(out.cpu(), ref)
    assert torch.equal(raw.cpu(), seqs.clamp(max=256).to(torch.int32))


def test_window_gather_req_to_token_rows_and_strided_out(dev):
    # page size 1: the table is req_to_token, indexed through req_pool_indices
    g = torch.Generator().manual_seed(7)
    seqs = [300, 5, 256]
    rtt = torch.zeros(6, 512, dtype=torch.int32)
    perm = torch.randperm(2000, generator=g).to(torch.int32)
    slots = torch.tensor([4, 1, 2], dtype=torch.int32)
    off = 0
    for b, s in enumerate(seqs):
        rtt[int(slots[b]), :s] = perm[off:off + s]
        off += s
    k = torch.randn(2, 2000, 4, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 2000, 4, 64, generator=g).to(torch.bfloat16)
    base = torch.zeros(3, 2, 2, 4, 256, 64 + 32, dtype=torch.bfloat16, device=dev)
    out = base[..., 16:80]
    kvwindow.gather_window(k.to(dev), v.to(dev), rtt.to(dev), torch.tensor(seqs, device=dev), page_size=1,
                           table_rows=slots.to(dev), out=out)
    torch.cuda.synchronize()
    ref = okw.gather_window(k, v, rtt[slots.long()], torch.tensor(seqs), 1, 256)
    assert torch.equal(out.cpu(), ref)
    assert base[..., :16].abs().sum() == 0 and base[..., 80:].abs().sum() == 0


@pytest.mark.parametrize("idx_dtype", [torch.int32, torch.int64])
def test_raw_page_table(dev, idx_dtype):
    g = torch.Generator().manual_seed(3)
    rtt = torch.randint(0, 1 << 20, (9, 5000), generator=g, dtype=torch.int32)
    slots = torch.tensor([8, 0, 3, 5, 1, 2], dtype=idx_dtype)
    seqs = torch.tensor([0, 1, 255, 256, 257, 4999], dtype=idx_dtype)
    table = torch.full((6, 256), -7, dtype=torch.int32, device=dev)
    raw = torch.empty(6, dtype=torch.int32, device=dev)
    kvwindow.build_raw256_page_table(req_to_token=rtt.to(dev), req_pool_indices=slots.to(dev),
                                     seq_lens=seqs.to(dev), page_table=table, raw_lengths=raw)
    torch.cuda.synchronize()
    ref_t, ref_r = okw.raw_page_table(rtt, slots, seqs, 256)
    assert torch.equal(table.cpu(), ref_t) and torch.equal(raw.cpu(), ref_r)


def test_ring_page_table(dev):
    slots = torch.tensor([0, 7, 3, 2], dtype=torch.int32)
    lens = torch.tensor([0, 255, 256, 1000], dtype=torch.int32)
    pages, raw = kvwindow.ring_page_table(slots.to(dev), lens.to(dev))
    ref_p, ref_r = okw.ring_page_table(slots, lens)
    assert torch.equal(pages.cpu(), ref_p) and torch.equal(raw.cpu(), ref_r)


@pytest.mark.parametrize("fused_export", [False, True])
def test_ring_append(dev, fused_export):
    g = torch.Generator().manual_seed(11 + fused_export)
    layers, heads, dim, window = 3, 8, 128, 256
    slots = torch.tensor([2, 0, 5, 1], dtype=torch.int32)
    prev = torch.tensor([0, 250, 511, 77], dtype=torch.int32)   # 250 + 8 wraps
    counts = torch.tensor([8, 8, 1, 5], dtype=torch.int32)
    n = int(counts.sum())
    ring_k = torch.randn(layers, 6 * window, heads, dim, generator=g).to(torch.bfloat16)
    ring_v = torch.randn(layers, 6 * window, heads, dim, generator=g).to(torch.bfloat16)
    pool_k = torch.randn(layers, 3000, heads, dim, generator=g).to(torch.bfloat16)
    pool_v = torch.randn(layers, 3000, heads, dim, generator=g).to(torch.bfloat16)
    locs = torch.randperm(3000, generator=g)[:n]
    rows_k, rows_v = pool_k[:, locs], pool_v[:, locs]
    ref_k, ref_v = okw.ring_append(ring_k, ring_v, rows_k, rows_v, slots, prev, counts, window)
    rk, rv = ring_k.to(dev), ring_v.to(dev)
    if fused_export:
        kvwindow.ring_append(rk, rv, pool_k.to(dev), pool_v.to(dev), slots.to(dev), prev.to(dev), counts.to(dev),
                             src_locs=locs.to(dev))
    else:
        kvwindow.ring_append(rk, rv, rows_k.to(dev), rows_v.to(dev), slots.to(dev), prev.to(dev), counts.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(rk.cpu(), ref_k) and torch.equal(rv.cpu(), ref_v)


def test_gather_selected_kv(dev):
    g = torch.Generator().manual_seed(5)
    pool_k = [torch.randn(900, 8, 128, generator=g).to(torch.bfloat16) for _ in range(5)]
    pool_v = [torch.randn(900, 8, 128, generator=g).to(torch.bfloat16) for _ in range(5)]
    locs = torch.randperm(900, generator=g)[:37]
    keys, values = kvwindow.gather_selected_kv([t.to(dev) for t in pool_k], [t.to(dev) for t in pool_v],
                                               locs.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(keys.cpu(), torch.stack([t.index_select(0, locs) for t in pool_k]))
    assert torch.equal(values.cpu(), torch.stack([t.index_select(0, locs) for t in pool_v]))
