"""Summary (Global16) state refresh on the GPU.

Drop-ins for SRT/speculative/global16_raw256_incremental.py:400-584
(``cache_position_scores``, ``merge_accepted_positions_``) -- which also
covers the GQA-5 adapter src/longspark/patches/gqa5_attention.py:43-106,
since the kernels take any query/KV head ratio -- and a fused all-layer
update for the draft-side loop of src/longspark/engine/draft.py:243-253.
``SRT`` = ``vendor/sglang/python/sglang/srt``.

Generalised geometry: S summary rows per query head, W <= 32 new rows,
head_dim 64/128/256 (the reference fixes S = 16, W = 8, D = 128).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .kvwindow import Layers, _check_layers, layer_pointers

GLOBAL_ROWS = 16
VERIFY_ROWS = 8
HEAD_DIM = 128
MAX_WIDTH = 32

_QDTYPES = (torch.bfloat16, torch.float16)


@dataclass(frozen=True)
class Global16IncrementalEvidence:
    """Same fields as the reference's evidence record (global16_raw256_incremental.py:32-41)."""
    layer_id: int
    batch_size: int
    verify_rows: int
    source_key_ptr: int
    score_workspace_ptr: int
    full_prefix_rows_read: int = 0
    target_kv_copy_bytes: int = 0
    postverify_delta_fa_calls: int = 0


def _rows(base: Optional[torch.Tensor] = None, *, layers: Optional[torch.Tensor] = None, stride_layer: int = 0,
          stride_b: int = 0, stride_w: int = 0, stride_loc: int = 0, stride_h: int = 0,
          located: bool = False) -> _lib.KvRows:
    return _lib.KvRows(base=_lib.ptr(base), layers=_lib.ptr(layers), stride_layer=stride_layer, stride_b=stride_b,
                       stride_w=stride_w, stride_loc=stride_loc, stride_h=stride_h, located=int(located))


def _geometry(a: _lib.SummaryArgs, *, batch, layers, q_heads, kv_heads, rows, width, head_dim, dtype, what):
    if q_heads % kv_heads:
        raise ValueError(f"{what}: query heads must be divisible by KV heads")
    if not 1 <= width <= MAX_WIDTH:
        raise ValueError(f"{what}: width must be in [1, {MAX_WIDTH}]")
    if head_dim not in (64, 128, 256):
        raise ValueError(f"{what}: head_dim must be 64, 128 or 256")
    if dtype not in _QDTYPES:
        raise ValueError(f"{what}: queries, keys and values must be bf16 or fp16")
    a.batch, a.layers, a.q_heads, a.kv_heads = batch, layers, q_heads, kv_heads
    a.rows, a.width, a.head_dim, a.dtype = rows, width, head_dim, _lib.dtype_code(torch.empty(0, dtype=dtype))


def _locations(a: _lib.SummaryArgs, locs: torch.Tensor, accept_lens: torch.Tensor, accept_offsets, batch: int,
               width: int, what: str):
    if accept_lens.shape != (batch,) or accept_lens.dtype != torch.int32:
        raise ValueError("accept_lens must be one int32 value per request")
    if locs.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{what}: accepted cache locations must be int32 or int64")
    a.locs, a.locs_dtype, a.accept_lens = locs.data_ptr(), _lib.dtype_code(locs), accept_lens.data_ptr()
    if locs.ndim == 2:
        if locs.shape != (batch, width):
            raise ValueError(f"fixed verify cache locations must have shape [batch, {width}]")
        a.locs_stride_b, a.locs_stride_w, a.compact_locs = locs.stride(0), locs.stride(1), 0
    elif locs.ndim == 1:
        if accept_offsets is None or accept_offsets.shape[0] < batch or accept_offsets.dtype != torch.int32:
            raise ValueError("compact cache locations require int32 accept offsets")
        if locs.stride(0) != 1:
            raise ValueError(f"{what}: compact locations must be contiguous")
        a.compact_locs, a.accept_offsets = 1, accept_offsets.data_ptr()
    else:
        raise ValueError("accepted cache locations must be compact flat or fixed [batch, W]")


def cache_position_scores(*, layer_id: int, global_query: torch.Tensor, new_keys: torch.Tensor, output: torch.Tensor,
                          softmax_scale: float, softcap: float = 0.0) -> Global16IncrementalEvidence:
    """``output[b, h, r, w] = scale * <global_query[b, h, r], new_keys[b, w, h // g]>``
    (fp32; softcap applied when > 0) into a caller-owned ``[B, Hq, S, W]`` fp32 workspace."""
    what = "cache_position_scores"
    dev = _lib.require_cuda(global_query, new_keys, output, what=what)
    if global_query.ndim != 4 or new_keys.ndim != 4:
        raise ValueError("Global query and new Target keys must be rank-4")
    batch, q_heads, rows, dim = global_query.shape
    width, kv_heads = new_keys.shape[1], new_keys.shape[2]
    if new_keys.shape[0] != batch or new_keys.shape[3] != dim:
        raise ValueError("Global16 incremental score shape is incompatible with GQA")
    if output.shape != (batch, q_heads, rows, width):
        raise ValueError("score output workspace has the wrong shape")
    if output.dtype != torch.float32:
        raise ValueError("score output workspace must use FP32")
    if new_keys.dtype != global_query.dtype:
        raise ValueError("Global query and Target keys must use the same dtype")
    if global_query.stride(3) != 1 or new_keys.stride(3) != 1:
        raise ValueError(f"{what}: head_dim must be contiguous")
    a = _lib.SummaryArgs()
    _geometry(a, batch=batch, layers=1, q_heads=q_heads, kv_heads=kv_heads, rows=rows, width=width, head_dim=dim,
              dtype=global_query.dtype, what=what)
    a.softmax_scale, a.softcap = float(softmax_scale), float(softcap)
    a.query = global_query.data_ptr()
    a.q_stride_b, a.q_stride_h, a.q_stride_s = global_query.stride(0), global_query.stride(1), global_query.stride(2)
    a.keys = _rows(new_keys, stride_b=new_keys.stride(0), stride_w=new_keys.stride(1), stride_h=new_keys.stride(2))
    a.scores = output.data_ptr()
    a.sc_stride_b, a.sc_stride_h, a.sc_stride_s, a.sc_stride_w = output.stride()
    _lib.call("ls_summary_scores", ctypes.byref(a), _lib.stream_of(dev))
    return Global16IncrementalEvidence(layer_id=int(layer_id), batch_size=batch, verify_rows=width,
                                       source_key_ptr=int(new_keys.data_ptr()),
                                       score_workspace_ptr=int(output.data_ptr()))


def merge_accepted_positions_(*, state_output: torch.Tensor, state_lse: torch.Tensor, position_scores: torch.Tensor,
                              value_cache: torch.Tensor, accepted_cache_locs: torch.Tensor, accept_lens: torch.Tensor,
                              accept_offsets: Optional[torch.Tensor], state_slots: Optional[torch.Tensor] = None) -> None:
    """Fold each request's first ``accept_lens[b]`` accepted value rows into the
    persistent normalised output / LSE state (in place, no allocation).

    ``value_cache`` is a page-size-one cache ``[N, 1, Hkv, D]``; locations are
    fixed ``[B, W]`` or compact (flat, with ``accept_offsets`` receiving the
    exclusive prefix sums of ``accept_lens``).  ``state_slots`` selects the
    state row per request (default: row b, which needs capacity == B).
    """
    what = "merge_accepted_positions_"
    dev = _lib.require_cuda(state_output, state_lse, position_scores, value_cache, accepted_cache_locs, accept_lens,
                            accept_offsets, state_slots, what=what)
    if state_output.dtype != torch.float32 or state_lse.dtype != torch.float32 or \
            position_scores.dtype != torch.float32:
        raise ValueError("Global16 state, LSE, and cached scores must use FP32")
    if state_output.ndim != 4:
        raise ValueError("Global16 state output must be [capacity, Hq, S, D]")
    capacity, q_heads, rows, dim = state_output.shape
    batch = int(position_scores.shape[0])
    if state_lse.shape != (capacity, q_heads, rows):
        raise ValueError("Global16 state output/LSE shapes do not match")
    if position_scores.ndim != 4 or position_scores.shape[:3] != (batch, q_heads, rows):
        raise ValueError("Global16 cached score shape is invalid")
    width = position_scores.shape[3]
    if value_cache.ndim != 4 or value_cache.shape[1] != 1:
        raise ValueError("accepted Target V must come from a page-size-one cache")
    kv_heads = int(value_cache.shape[2])
    if value_cache.shape[3] != dim:
        raise ValueError("Target V cache does not match Global16 GQA state")
    if state_output.stride(3) != 1 or value_cache.stride(3) != 1:
        raise ValueError(f"{what}: head_dim must be contiguous")
    if state_slots is None:
        if capacity != batch:
            raise ValueError("batch-local Global16 state must have one row per request")
    elif state_slots.shape != (batch,) or state_slots.dtype != torch.int32:
        raise ValueError("state_slots must be one int32 pool index per request")
    a = _lib.SummaryArgs()
    _geometry(a, batch=batch, layers=1, q_heads=q_heads, kv_heads=kv_heads, rows=rows, width=width, head_dim=dim,
              dtype=value_cache.dtype, what=what)
    a.values = _rows(value_cache, stride_loc=value_cache.stride(0), stride_h=value_cache.stride(2), located=True)
    a.scores = position_scores.data_ptr()
    a.sc_stride_b, a.sc_stride_h, a.sc_stride_s, a.sc_stride_w = position_scores.stride()
    a.state_output = state_output.data_ptr()
    a.so_stride_c, a.so_stride_h, a.so_stride_s = state_output.stride(0), state_output.stride(1), state_output.stride(2)
    a.state_lse = state_lse.data_ptr()
    a.sl_stride_c, a.sl_stride_h, a.sl_stride_s = state_lse.stride()
    a.state_slots = _lib.ptr(state_slots)
    _locations(a, accepted_cache_locs, accept_lens, accept_offsets, batch, width, what)
    _lib.call("ls_summary_merge", ctypes.byref(a), _lib.stream_of(dev))


def summary_update(*, query: torch.Tensor, key_cache: Layers, value_cache: Layers, accepted_cache_locs: torch.Tensor,
                   accept_lens: torch.Tensor, state_output: torch.Tensor, state_lse: torch.Tensor,
                   softmax_scale: float, state_slots: Optional[torch.Tensor] = None, softcap: float = 0.0,
                   width: Optional[int] = None, accept_offsets: Optional[torch.Tensor] = None) -> None:
    """Scores and merge for every layer in one launch (in place).

    ``query`` ``[L, Hq, S, D]`` (shared by all requests) or ``[L, B, Hq, S, D]``;
    ``key_cache`` / ``value_cache`` per-layer ``[N, Hkv, D]`` row pools (a
    list, or one ``[L, N, Hkv, D]`` tensor); ``accepted_cache_locs`` fixed
    ``[B, W]`` or compact (then pass ``width`` and ``accept_offsets``);
    state ``[C, L, Hq, S, D]`` / LSE ``[C, L, Hq, S]`` fp32 (the draft pool
    layout of src/longspark/engine/draft.py:107-108).  Equivalent to
    ``cache_position_scores`` + ``merge_accepted_positions_`` per layer with
    keys and values read at the accepted locations.
    """
    what = "summary_update"
    dev = _lib.require_cuda(query, accepted_cache_locs, accept_lens, state_output, state_lse, state_slots,
                            accept_offsets, what=what)
    ks, vs = _check_layers(key_cache, what, "key_cache"), _check_layers(value_cache, what, "value_cache")
    if query.ndim not in (4, 5):
        raise ValueError(f"{what}: query must be [L, Hq, S, D] or [L, B, Hq, S, D]")
    if state_output.ndim != 5 or state_output.dtype != torch.float32 or state_lse.dtype != torch.float32:
        raise ValueError(f"{what}: state must be fp32 [C, L, Hq, S, D] with LSE [C, L, Hq, S]")
    capacity, layers, q_heads, rows, dim = state_output.shape
    batch = accept_lens.shape[0]
    if state_lse.shape != state_output.shape[:4]:
        raise ValueError("Global16 state output/LSE shapes do not match")
    qshape = (layers, q_heads, rows, dim) if query.ndim == 4 else (layers, batch, q_heads, rows, dim)
    if tuple(query.shape) != qshape or query.stride(-1) != 1:
        raise ValueError(f"{what}: query must be {qshape} with contiguous head_dim")
    if len(ks) != layers or len(vs) != layers:
        raise ValueError(f"{what}: one key and value pool per layer is required")
    kv_heads = ks[0].shape[1]
    if ks[0].shape[2] != dim or vs[0].shape[1:] != ks[0].shape[1:] or ks[0].dtype != query.dtype \
            or vs[0].dtype != query.dtype:
        raise ValueError(f"{what}: key/value pools do not match the query geometry")
    if state_slots is None:
        if capacity != batch:
            raise ValueError("batch-local Global16 state must have one row per request")
    elif state_slots.shape != (batch,) or state_slots.dtype != torch.int32:
        raise ValueError("state_slots must be one int32 pool index per request")
    if width is None:
        if accepted_cache_locs.ndim != 2:
            raise ValueError(f"{what}: compact locations need an explicit width")
        width = accepted_cache_locs.shape[1]
    a = _lib.SummaryArgs()
    _geometry(a, batch=batch, layers=layers, q_heads=q_heads, kv_heads=kv_heads, rows=rows, width=width,
              head_dim=dim, dtype=query.dtype, what=what)
    a.softmax_scale, a.softcap = float(softmax_scale), float(softcap)
    a.query = query.data_ptr()
    if query.ndim == 4:
        a.q_stride_l, a.q_stride_b, a.q_stride_h, a.q_stride_s = query.stride(0), 0, query.stride(1), query.stride(2)
    else:
        a.q_stride_l, a.q_stride_b, a.q_stride_h, a.q_stride_s = query.stride()[:4]
    a.keys = _rows(layers=layer_pointers.get(key_cache, dev), stride_loc=ks[0].stride(0), stride_h=ks[0].stride(1),
                   located=True)
    a.values = _rows(layers=layer_pointers.get(value_cache, dev), stride_loc=vs[0].stride(0),
                     stride_h=vs[0].stride(1), located=True)
    a.state_output = state_output.data_ptr()
    a.so_stride_c, a.so_stride_l, a.so_stride_h, a.so_stride_s = state_output.stride()[:4]
    a.state_lse = state_lse.data_ptr()
    a.sl_stride_c, a.sl_stride_l, a.sl_stride_h, a.sl_stride_s = state_lse.stride()
    a.state_slots = _lib.ptr(state_slots)
    _locations(a, accepted_cache_locs, accept_lens, accept_offsets, batch, width, what)
    _lib.call("ls_summary_update", ctypes.byref(a), _lib.stream_of(dev))


def prefill_global_attention(*, query: torch.Tensor, key_cache: Layers, value_cache: Layers,
                             page_table: torch.Tensor, cache_seqlens: torch.Tensor, softmax_scale: float,
                             softcap: float = 0.0, output: Optional[torch.Tensor] = None,
                             lse: Optional[torch.Tensor] = None, round_output: bool = True, chunk: int = 0):
    """Prefill summary state of every selected layer in one launch.

    The state ``TargetClient._prefill_summaries`` stacks (src/longspark/engine/
    target.py:230-253) from one ``run_prefill_global_attention`` per layer
    (SRT/speculative/global16_raw256.py:668-784): non-causal attention of the
    summary query rows over each request's whole prefix, the prefix read
    through its location-table row (req_to_token, page size 1).

    ``query`` ``[L, Hq, S, D]`` (shared by every request, as target.py:234
    expands it) or ``[B, L, Hq, S, D]``; ``key_cache`` / ``value_cache``
    per-layer ``[N, Hkv, D]`` pools (a list, or one ``[L, N, Hkv, D]``
    tensor); ``page_table`` ``[B, >= max length]`` int32/int64 locations;
    ``cache_seqlens`` ``[B]`` int32.  Returns ``output`` ``[B, L, Hq, S, D]``
    and ``lse`` ``[B, L, Hq, S]`` fp32 (natural log; an empty prefix gives a
    zero output and LSE -inf).  ``round_output`` rounds the output to the
    query dtype, as FA3 returns it in that dtype before the reference widens
    it to fp32.  ``chunk`` (a multiple of 64, 0 = from the sizes) is the
    prefix length one workgroup covers.
    """
    what = "prefill_global_attention"
    dev = _lib.require_cuda(query, page_table, cache_seqlens, output, lse, what=what)
    ks, vs = _check_layers(key_cache, what, "key_cache"), _check_layers(value_cache, what, "value_cache")
    if page_table.ndim != 2 or page_table.dtype not in (torch.int32, torch.int64) or page_table.stride(1) != 1:
        raise ValueError("Global16 prefill page table must be a two-dimensional int32/int64 table "
                         "with contiguous rows")
    batch = page_table.shape[0]
    if cache_seqlens.ndim != 1 or cache_seqlens.shape[0] != batch:
        raise ValueError("Global16 prefill lengths must match the batch")
    lens = cache_seqlens if cache_seqlens.dtype == torch.int32 else cache_seqlens.to(torch.int32)
    lens = lens.contiguous()
    if query.ndim == 4:
        layers, q_heads, rows, dim = query.shape
        qs = (query.stride(0) if query.shape[0] > 1 else 0, 0, query.stride(1), query.stride(2))
    elif query.ndim == 5:
        if query.shape[0] != batch:
            raise ValueError(f"{what}: query batch does not match the page table")
        layers, q_heads, rows, dim = query.shape[1:]
        qs = (query.stride(1) if query.shape[1] > 1 else 0, query.stride(0), query.stride(2), query.stride(3))
    else:
        raise ValueError(f"{what}: query must be [L, Hq, S, D] or [B, L, Hq, S, D]")
    if query.stride(-1) != 1 or query.dtype not in _QDTYPES:
        raise ValueError(f"{what}: query must be bf16/fp16 with a contiguous head dimension")
    if len(ks) != layers or len(vs) != layers:
        raise ValueError(f"{what}: one key and value pool per layer is required")
    kv_heads = ks[0].shape[1]
    if ks[0].shape[2] != dim or vs[0].shape[1:] != ks[0].shape[1:] or ks[0].dtype != query.dtype \
            or vs[0].dtype != query.dtype:
        raise ValueError(f"{what}: key/value pools do not match the query geometry")
    if q_heads % kv_heads:
        raise ValueError(f"{what}: query heads must be divisible by KV heads")
    if output is None:
        output = torch.empty(batch, layers, q_heads, rows, dim, dtype=torch.float32, device=dev)
    if lse is None:
        lse = torch.empty(batch, layers, q_heads, rows, dtype=torch.float32, device=dev)
    if output.shape != (batch, layers, q_heads, rows, dim) or output.dtype != torch.float32 \
            or output.stride(-1) != 1:
        raise ValueError(f"{what}: output must be fp32 [B, L, Hq, S, D] with a contiguous head dimension")
    if lse.shape != (batch, layers, q_heads, rows) or lse.dtype != torch.float32:
        raise ValueError(f"{what}: lse must be fp32 [B, L, Hq, S]")
    a = _lib.PrefillArgs()
    a.batch, a.layers, a.q_heads, a.kv_heads, a.rows, a.head_dim = batch, layers, q_heads, kv_heads, rows, dim
    a.dtype = _lib.dtype_code(query)
    a.softmax_scale, a.softcap = float(softmax_scale), float(softcap or 0.0)
    a.query = query.data_ptr()
    a.q_stride_l, a.q_stride_b, a.q_stride_h, a.q_stride_s = qs
    a.keys = _rows(layers=layer_pointers.get(key_cache, dev), stride_loc=ks[0].stride(0), stride_h=ks[0].stride(1),
                   located=True)
    a.values = _rows(layers=layer_pointers.get(value_cache, dev), stride_loc=vs[0].stride(0),
                     stride_h=vs[0].stride(1), located=True)
    a.page_table, a.pt_dtype = page_table.data_ptr(), _lib.dtype_code(page_table)
    a.pt_stride_b, a.max_len = page_table.stride(0), page_table.shape[1]
    a.seq_lens = lens.data_ptr()
    a.output = output.data_ptr()
    a.o_stride_l, a.o_stride_b, a.o_stride_h, a.o_stride_s = output.stride(1), output.stride(0), \
        output.stride(2), output.stride(3)
    a.lse = lse.data_ptr()
    a.l_stride_l, a.l_stride_b, a.l_stride_h, a.l_stride_s = lse.stride(1), lse.stride(0), lse.stride(2), \
        lse.stride(3)
    a.round_output = _lib.dtype_code(query) if round_output else _lib.LS_F32
    a.chunk = int(chunk)
    need = ctypes.c_int64(0)
    _lib.call("ls_global16_prefill_workspace", ctypes.byref(a), ctypes.byref(need))
    if batch == 0:
        return output, lse
    scratch = torch.empty(max(int(need.value), 16) // 4, dtype=torch.float32, device=dev) if need.value else None
    _lib.call("ls_global16_prefill", ctypes.byref(a), _lib.ptr(scratch), int(need.value), _lib.stream_of(dev))
    return output, lse


def run_prefill_global_attention(self, *, layer_id: int, layer, key_cache: torch.Tensor, value_cache: torch.Tensor,
                                 page_table: torch.Tensor, cache_seqlens: torch.Tensor, flash_attn_with_kvcache=None,
                                 softmax_scale: float, softcap: float, k_descale=None, v_descale=None,
                                 num_splits: int = 0, extra_kwargs: Optional[dict] = None) -> None:
    """Method body for ``Global16Raw256VerifyContext.run_prefill_global_attention``
    (SRT/speculative/global16_raw256.py:668-784): same checks and messages,
    same state record; the attention runs on ``prefill_global_attention``
    instead of the ``flash_attn_with_kvcache`` callable (which is ignored, as
    are ``num_splits`` and ``extra_kwargs``).  ``key_cache`` / ``value_cache``
    are the layer's ``[N, 1, Hkv, D]`` (page size 1) or ``[N, Hkv, D]`` pools.
    """
    import sys

    layer_id = int(layer_id)
    if self.incremental_from_prior or self.committed:
        raise RuntimeError("Global16 prefill scan requires a fresh context")
    if not self.applies_to(layer_id):
        raise ValueError(f"layer {layer_id} is not selected for Global16")
    if layer_id in self.layer_states:
        raise RuntimeError("Global16 prefill state may be initialized only once")
    if page_table.ndim != 2:
        raise ValueError("Global16 prefill page table must be two-dimensional")
    if k_descale is not None or v_descale is not None:
        raise NotImplementedError("Global16 prefill: scaled (fp8) key/value caches are not supported")
    cache_seqlens = cache_seqlens.to(device=self.global_queries.device, dtype=torch.int32)
    if cache_seqlens.ndim != 1 or cache_seqlens.shape[0] != page_table.shape[0]:
        raise ValueError("Global16 prefill lengths must match the batch")
    source_rows = self.source_batch_rows.to(device=page_table.device)
    page_table = page_table.index_select(0, source_rows)
    cache_seqlens = cache_seqlens.index_select(0, source_rows)

    def pool(t: torch.Tensor) -> torch.Tensor:
        if t.ndim == 4:
            if t.shape[1] != 1:
                raise ValueError("Global16 prefill: only page size 1 caches are supported")
            t = t[:, 0]
        return t

    query = self._query_for_layer(layer_id)                      # [B, Hq, S, D]
    output, lse = prefill_global_attention(query=query[:, None], key_cache=[pool(key_cache)],
                                           value_cache=[pool(value_cache)], page_table=page_table,
                                           cache_seqlens=cache_seqlens, softmax_scale=softmax_scale,
                                           softcap=softcap)
    mod = sys.modules[type(self).__module__]
    self.layer_states[layer_id] = mod.Global16Raw256LayerState(query=query, output=output[:, 0],
                                                               logsumexp=lse[:, 0])
    self.layer_objects[layer_id] = layer
    prefix_rows = int(self.confirmed_prefix_lens.sum().item()) if self.collect_fixed_cost_audit else 0
    self.joint_evidence[layer_id] = mod.Global16Raw256FAEvidence(
        layer_id=layer_id, fa3_invocations=1, key_cache_storage_ptr=key_cache.untyped_storage().data_ptr(),
        value_cache_storage_ptr=value_cache.untyped_storage().data_ptr(), target_query_rows=0,
        global_query_rows=self.batch_size * query.shape[2], duplicated_page_table_rows=0,
        request_layer_base_inits=self.batch_size, prefix_rows=prefix_rows,
        query_key_pairs=prefix_rows * query.shape[2])
