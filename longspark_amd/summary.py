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
