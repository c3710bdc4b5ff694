"""Global16 prefill initialisation on the GPU vs the oracle.

``prefill_global_attention`` (all layers in one launch) against
``oracle.summary.prefill_global_attention`` per layer, exact in fp64.  The
kernel rounds the attention weights to the key type before the weighted sum
of values, as the reference's FA3 does, so the output bound is
2^-8 * sum_t p_t |v_t| (twice the weight rounding's worst case), plus, when
the output is rounded to the query type, 2^-8 * |out|; LSE within
1e-5 + 2e-6 |lse|.  Cases: Qwen3-14B geometry (40 query / 8 KV heads, 16
slots, head_dim 128) with prefixes of 0, 1, 63, 64, 65, 1000 and 3000 tokens
through a permuted location table, on the split + combine path (automatic
and 64-token chunks) and the single-split path; one KV head per query head
(one of four waves busy); 16 query heads per KV head (two row tiles);
52 slots (a partial wave); head_dim 64 and 256; fp16 with softcap and an
int64 table; and the method drop-in on a stand-in context.
"""

from dataclasses import dataclass

import pytest
import torch

from longspark_amd import summary
from oracle import summary as osm

pytestmark = pytest.mark.gpu


def make_case(dev, *, batch_lens, layers, hq, hkv, rows, dim, dtype, seed, pool_extra=64, table_dtype=torch.int32):
    g = torch.Generator().manual_seed(seed)
    lens = torch.tensor(batch_lens, dtype=torch.int32)
    width = max(max(batch_lens), 1)
    n = int(lens.sum()) + pool_extra
    table = torch.stack([torch.randperm(n, generator=g)[:width] for _ in batch_lens]).to(table_dtype)
    q = torch.randn(layers, hq, rows, dim, generator=g).to(dtype)
    kc = [(1.5 * torch.randn(n, hkv, dim, generator=g)).to(dtype) for _ in range(layers)]
    vc = [torch.randn(n, hkv, dim, generator=g).to(dtype) for _ in range(layers)]
    return q, kc, vc, table, lens


def check(out, lse, q, kc, vc, table, lens, scale, softcap=0.0, rounded=True):
    out, lse = out.cpu().double(), lse.cpu().double()
    for layer in range(q.shape[0]):
        o_ref, l_ref = osm.prefill_global_attention(q[layer].cpu(), kc[layer].cpu(), vc[layer].cpu(), table.cpu(),
                                                    lens, scale, softcap=softcap)
        weighted_abs, _ = osm.prefill_global_attention(q[layer].cpu(), kc[layer].cpu(), vc[layer].cpu().abs(),
                                                       table.cpu(), lens, scale, softcap=softcap)
        bound = 2.0 ** -8 * weighted_abs + 1e-6
        if rounded:
            bound = bound + 2.0 ** -8 * o_ref.abs()
        err = (out[:, layer] - o_ref).abs()
        assert bool((err <= bound).all()), (layer, float(err.max()), float((err / bound).max()))
        fin = torch.isfinite(l_ref)
        assert torch.equal(fin, torch.isfinite(lse[:, layer]))
        assert bool(torch.isneginf(lse[:, layer][~fin]).all())
        lerr = (lse[:, layer][fin] - l_ref[fin]).abs()
        assert bool((lerr <= 1e-5 + 2e-6 * l_ref[fin].abs()).all()), (layer, float(lerr.max()))


QWEN_LENS = [0, 1, 63, 64, 65, 1000, 3000]


@pytest.mark.parametrize("chunk", [0, 64, 4096])
def test_prefill_qwen3_geometry(dev, chunk):
    q, kc, vc, table, lens = make_case(dev, batch_lens=QWEN_LENS, layers=2, hq=40, hkv=8, rows=16, dim=128,
                                       dtype=torch.bfloat16, seed=chunk + 1)
    print(f"prefill qwen3 chunk={chunk}", flush=True)
    out, lse = summary.prefill_global_attention(query=q.to(dev), key_cache=[k.to(dev) for k in kc],
                                                value_cache=[v.to(dev) for v in vc], page_table=table.to(dev),
                                                cache_seqlens=lens.to(dev), softmax_scale=128 ** -0.5, chunk=chunk)
    torch.cuda.synchronize()
    assert out.shape == (len(QWEN_LENS), 2, 40, 16, 128) and lse.shape == (len(QWEN_LENS), 2, 40, 16)
    check(out, lse, q, kc, vc, table, lens, 128 ** -0.5)
    # the reference's output is rounded to bf16 before it is widened
    assert torch.equal(out, out.to(torch.bfloat16).float())


@pytest.mark.parametrize("hq,hkv,rows,dim,dtype,softcap,table_dtype,rounded", [
    (8, 8, 16, 64, torch.float16, 5.0, torch.int64, True),     # one row block per KV head
    (32, 2, 16, 128, torch.bfloat16, 0.0, torch.int32, False),  # 256 rows per KV head: two row tiles
    (10, 2, 52, 128, torch.bfloat16, 0.0, torch.int32, True),   # 260 rows: a partial wave
    (16, 4, 16, 256, torch.bfloat16, 0.0, torch.int32, False),  # head_dim 256
])
def test_prefill_geometries(dev, hq, hkv, rows, dim, dtype, softcap, table_dtype, rounded):
    lens = [700, 5, 129]
    q, kc, vc, table, lt = make_case(dev, batch_lens=lens, layers=2, hq=hq, hkv=hkv, rows=rows, dim=dim, dtype=dtype,
                                     seed=hq * 100 + dim, table_dtype=table_dtype)
    scale = dim ** -0.5
    for chunk in (0, 128):
        print(f"prefill hq={hq} hkv={hkv} rows={rows} dim={dim} {dtype} chunk={chunk}", flush=True)
        out, lse = summary.prefill_global_attention(query=q.to(dev), key_cache=torch.stack(kc).to(dev),
                                                    value_cache=torch.stack(vc).to(dev), page_table=table.to(dev),
                                                    cache_seqlens=lt.to(dev), softmax_scale=scale, softcap=softcap,
                                                    round_output=rounded, chunk=chunk)
        torch.cuda.synchronize()
        check(out, lse, q, kc, vc, table, lt, scale, softcap=softcap, rounded=rounded)


def test_prefill_per_request_queries_and_strided_output(dev):
    """[B, L, Hq, S, D] queries (the context's layout) and caller-given output views."""
    lens = [300, 40]
    q, kc, vc, table, lt = make_case(dev, batch_lens=lens, layers=3, hq=8, hkv=2, rows=16, dim=128,
                                     dtype=torch.bfloat16, seed=77)
    qb = torch.stack([q, q.flip(1)])                   # request 1 has the query heads reversed
    big = torch.full((2, 3, 8, 16, 160), 7.0, device=dev)
    out = big[..., :128]
    lse = torch.empty(2, 3, 8, 16, device=dev)
    print("prefill per-request queries", flush=True)
    summary.prefill_global_attention(query=qb.to(dev), key_cache=[k.to(dev) for k in kc],
                                     value_cache=[v.to(dev) for v in vc], page_table=table.to(dev),
                                     cache_seqlens=lt.to(dev), softmax_scale=0.1, output=out, lse=lse, chunk=64)
    torch.cuda.synchronize()
    assert bool((big[..., 128:] == 7.0).all())
    check(out[:1], lse[:1], q, kc, vc, table[:1], lt[:1], 0.1)
    check(out[1:], lse[1:], q.flip(1), kc, vc, table[1:], lt[1:], 0.1)


def test_prefill_rejects_bad_arguments(dev):
    q, kc, vc, table, lt = make_case(dev, batch_lens=[10], layers=1, hq=4, hkv=2, rows=16, dim=128,
                                     dtype=torch.bfloat16, seed=3)
    kw = dict(query=q.to(dev), key_cache=[k.to(dev) for k in kc], value_cache=[v.to(dev) for v in vc],
              page_table=table.to(dev), cache_seqlens=lt.to(dev), softmax_scale=0.1)
    with pytest.raises(ValueError, match="multiple of 64"):
        summary.prefill_global_attention(**{**kw, "chunk": 100})
    with pytest.raises(ValueError, match="lengths must match"):
        summary.prefill_global_attention(**{**kw, "cache_seqlens": lt.repeat(2).to(dev)})
    with pytest.raises(ValueError, match="pools do not match"):
        summary.prefill_global_attention(**{**kw, "key_cache": [kc[0].half().to(dev)]})


# Stand-ins for the reference context's records (global16_raw256.py:240-260);
# the drop-in builds them from the context class's own module.
@dataclass
class Global16Raw256LayerState:
    query: torch.Tensor
    output: torch.Tensor
    logsumexp: torch.Tensor


@dataclass
class Global16Raw256FAEvidence:
    layer_id: int
    fa3_invocations: int
    key_cache_storage_ptr: int
    value_cache_storage_ptr: int
    target_query_rows: int
    global_query_rows: int
    duplicated_page_table_rows: int
    request_layer_base_inits: int
    prefix_rows: int
    query_key_pairs: int


class Context:
    """Holds the attributes run_prefill_global_attention reads."""

    def __init__(self, global_queries, lens, layer_ids):
        self.global_queries = global_queries              # [B, L, Hq, S, D]
        self.batch_size = global_queries.shape[0]
        self.source_batch_rows = torch.arange(self.batch_size)
        self.confirmed_prefix_lens = lens
        self.selected_layer_ids = tuple(layer_ids)
        self._layer_index = {lid: i for i, lid in enumerate(layer_ids)}
        self.incremental_from_prior = False
        self.committed = False
        self.collect_fixed_cost_audit = True
        self.layer_states, self.layer_objects, self.joint_evidence = {}, {}, {}

    def applies_to(self, layer_id):
        return layer_id in self._layer_index

    def _query_for_layer(self, layer_id):
        return self.global_queries[:, self._layer_index[layer_id]]

    run_prefill_global_attention = summary.run_prefill_global_attention


def test_method_drop_in(dev):
    lens = [90, 33]
    q, kc, vc, table, lt = make_case(dev, batch_lens=lens, layers=1, hq=8, hkv=2, rows=16, dim=128,
                                     dtype=torch.bfloat16, seed=11)
    ctx = Context(q.to(dev)[None].expand(2, -1, -1, -1, -1), lt.to(dev), [5])
    print("prefill method drop-in", flush=True)
    ctx.run_prefill_global_attention(layer_id=5, layer="attn-5", key_cache=kc[0].to(dev)[:, None],
                                     value_cache=vc[0].to(dev)[:, None], page_table=table.to(dev),
                                     cache_seqlens=lt.to(dev), flash_attn_with_kvcache=None,
                                     softmax_scale=0.09, softcap=0.0)
    torch.cuda.synchronize()
    st = ctx.layer_states[5]
    assert st.output.shape == (2, 8, 16, 128) and st.logsumexp.shape == (2, 8, 16)
    check(st.output[:, None], st.logsumexp[:, None], q, kc, vc, table, lt, 0.09)
    ev = ctx.joint_evidence[5]
    assert ev.prefix_rows == sum(lens) and ev.query_key_pairs == 16 * sum(lens) and ev.global_query_rows == 32
    assert ctx.layer_objects[5] == "attn-5"
    with pytest.raises(RuntimeError, match="only once"):
        ctx.run_prefill_global_attention(layer_id=5, layer=None, key_cache=kc[0].to(dev), value_cache=vc[0].to(dev),
                                         page_table=table.to(dev), cache_seqlens=lt.to(dev), softmax_scale=0.09,
                                         softcap=0.0)
    with pytest.raises(ValueError, match="not selected"):
        ctx.run_prefill_global_attention(layer_id=6, layer=None, key_cache=kc[0].to(dev), value_cache=vc[0].to(dev),
                                         page_table=table.to(dev), cache_seqlens=lt.to(dev), softmax_scale=0.09,
                                         softcap=0.0)
