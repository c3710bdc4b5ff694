"""Drafter attention over the three refreshed views, on the GPU.

Drop-ins for both forms the reference's drafter uses
(SRT/speculative/global16_raw256.py:1460-1600 picks one):
  * one kernel over all sources -- SRT/speculative/
    global16_raw256_draft_all_attention.py:283-416
    (``can_use_fused_global_local_raw_attention``,
    ``fused_global_local_raw_attention``): for every request and query head
    the Raw256 window (read through the page table), the Global16 summary
    state and the Local7 in-block rows, folded in the reference's order and
    at its rounding points;
  * the merge after a separate window attention (the default) --
    SRT/speculative/global16_raw256_draft_fused.py:314-479
    (``can_use_fused_global_local_raw_merge``,
    ``fused_global_local_raw_merge``).
``SPEC`` = ``SRT/speculative``, ``SRT`` = ``vendor/sglang/python/sglang/srt``.
"""

from __future__ import annotations

import ctypes
import json
import os
import warnings
from typing import Optional

import torch

from . import _lib

GLOBAL_ROWS = 16
LOCAL_ROWS = 7
QUERY_ROWS = 7
RAW_ROWS = 256
HEAD_DIM = 128


def can_use_fused_global_local_raw_attention(*, query: torch.Tensor, global_keys: torch.Tensor,
                                             global_values: torch.Tensor, state_slots: Optional[torch.Tensor],
                                             local_keys: torch.Tensor, local_values: torch.Tensor,
                                             local_attention_mask: torch.Tensor, key_cache: torch.Tensor,
                                             value_cache: torch.Tensor, page_table: torch.Tensor,
                                             raw_lengths: torch.Tensor, output: torch.Tensor) -> bool:
    """The reference's fixed production contract (draft_all_attention.py:283-345),
    with "the gfx950 library is loaded" in place of "triton is importable"."""
    batch = int(query.shape[0]) if query.ndim > 0 else 0
    return bool(
        query.is_cuda and query.dtype == torch.bfloat16 and query.ndim == 4
        and tuple(query.shape[2:]) == (QUERY_ROWS, HEAD_DIM)
        and tuple(global_keys.shape) == (batch, query.shape[1], GLOBAL_ROWS, HEAD_DIM)
        and global_keys.dtype == torch.bfloat16
        and global_values.is_cuda and global_values.dtype == torch.float32 and global_values.ndim == 4
        and tuple(global_values.shape[1:]) == (query.shape[1], GLOBAL_ROWS, HEAD_DIM)
        and state_slots is not None and state_slots.is_cuda and state_slots.dtype == torch.int32
        and tuple(state_slots.shape) == (batch,)
        and local_keys.shape == local_values.shape and local_keys.ndim == 4 and local_keys.shape[0] == batch
        and tuple(local_keys.shape[2:]) == (LOCAL_ROWS, HEAD_DIM)
        and query.shape[1] % local_keys.shape[1] == 0
        and local_keys.dtype == query.dtype and local_values.dtype == query.dtype
        and local_attention_mask.is_cuda and local_attention_mask.dtype == torch.bool
        and tuple(local_attention_mask.shape) == (batch, QUERY_ROWS, LOCAL_ROWS)
        and key_cache.is_cuda and value_cache.is_cuda
        and key_cache.dtype == query.dtype and value_cache.dtype == query.dtype
        and key_cache.shape == value_cache.shape and key_cache.ndim == 4
        and tuple(key_cache.shape[1:]) == (1, local_keys.shape[1], HEAD_DIM)
        and page_table.is_cuda and page_table.dtype == torch.int32
        and tuple(page_table.shape) == (batch, RAW_ROWS)
        and raw_lengths.is_cuda and raw_lengths.dtype == torch.int32 and tuple(raw_lengths.shape) == (batch,)
        and output.is_cuda and output.dtype == query.dtype and output.shape == query.shape
    )


RAW_BLOCK = 64  # window rows per online-softmax step (the reference's default block)
_warned_blocks = set()


def _configured_raw_block(batch: int) -> int:
    """The window block the reference would use for this batch: entry
    ``[block, warps, stages]`` of ``DFK_GLOBAL16_DRAFT_ATTENTION_CONFIGS``
    (a JSON object keyed by batch size or "default"), else 64
    (SPEC/global16_raw256_draft_all_attention.py:20-46, same validation and
    messages).  Warps and stages are launch choices with no effect on the
    result; the block sets where the online softmax rescales and where the
    weights are rounded to bf16."""
    raw = os.getenv("DFK_GLOBAL16_DRAFT_ATTENTION_CONFIGS", "{}")
    table = json.loads(raw)
    if not isinstance(table, dict):
        raise ValueError("Draft attention launch configurations must be a JSON object")
    for key, config in table.items():
        if key != "default" and (not key.isdecimal() or int(key) < 1):
            raise ValueError("Draft attention batch keys must be positive integers or default")
        if (not isinstance(config, list) or len(config) != 3 or config[0] not in (32, 64, 128)
                or config[1] not in (4, 8) or config[2] not in (1, 2, 3)):
            raise ValueError("Unsupported Draft attention launch configuration")
    return int(table.get(str(batch), table.get("default", [RAW_BLOCK]))[0])


def fused_global_local_raw_attention(*, query: torch.Tensor, global_keys: torch.Tensor, global_values: torch.Tensor,
                                     state_slots: torch.Tensor, local_keys: torch.Tensor, local_values: torch.Tensor,
                                     local_attention_mask: torch.Tensor, key_cache: torch.Tensor,
                                     value_cache: torch.Tensor, page_table: torch.Tensor, raw_lengths: torch.Tensor,
                                     output: torch.Tensor, softmax_scale: float, softcap: float = 0.0) -> torch.Tensor:
    """One kernel over all three sources into caller-owned ``output``
    (draft_all_attention.py:348-416, same checks and messages)."""
    if float(softcap) != 0.0:
        raise ValueError("fused all-source Draft attention requires softcap=0")
    block = _configured_raw_block(int(query.shape[0]))
    if block != RAW_BLOCK and block not in _warned_blocks:
        # This kernel always steps the window in blocks of 64 rows, the
        # reference's default; another block moves the result only within the
        # bf16 weight-rounding bound.
        _warned_blocks.add(block)
        warnings.warn(f"DFK_GLOBAL16_DRAFT_ATTENTION_CONFIGS selects a {block}-row window block; the gfx950 "
                      f"drafter attention steps the window in blocks of {RAW_BLOCK} rows (the reference default), "
                      "so results match that configuration", RuntimeWarning, stacklevel=2)
    if not can_use_fused_global_local_raw_attention(
            query=query, global_keys=global_keys, global_values=global_values, state_slots=state_slots,
            local_keys=local_keys, local_values=local_values, local_attention_mask=local_attention_mask,
            key_cache=key_cache, value_cache=value_cache, page_table=page_table, raw_lengths=raw_lengths,
            output=output):
        raise ValueError("fused all-source Draft tensors violate the contract")
    dev = _lib.require_cuda(query, global_keys, global_values, state_slots, local_keys, local_values,
                            local_attention_mask, key_cache, value_cache, page_table, raw_lengths, output,
                            what="fused_global_local_raw_attention")
    for name, t in (("query", query), ("global_keys", global_keys), ("global_values", global_values),
                    ("local_keys", local_keys), ("local_values", local_values), ("key_cache", key_cache),
                    ("value_cache", value_cache), ("output", output)):
        if t.stride(-1) != 1:
            raise ValueError(f"fused_global_local_raw_attention: {name} needs a contiguous head dimension")
    if page_table.stride(1) != 1:
        raise ValueError("fused_global_local_raw_attention: page_table rows must be contiguous")
    a = _lib.DraftAttentionArgs()
    a.batch, a.q_heads, a.kv_heads = query.shape[0], query.shape[1], local_keys.shape[1]
    a.softmax_scale = float(softmax_scale)
    a.query = query.data_ptr()
    a.q_stride_b, a.q_stride_h, a.q_stride_r = query.stride()[:3]
    a.global_keys = global_keys.data_ptr()
    a.gk_stride_b, a.gk_stride_h, a.gk_stride_g = global_keys.stride()[:3]
    a.global_values = global_values.data_ptr()
    a.gv_stride_b, a.gv_stride_h, a.gv_stride_g = global_values.stride()[:3]
    a.state_slots = state_slots.data_ptr()
    a.local_keys = local_keys.data_ptr()
    a.lk_stride_b, a.lk_stride_h, a.lk_stride_l = local_keys.stride()[:3]
    a.local_values = local_values.data_ptr()
    a.lv_stride_b, a.lv_stride_h, a.lv_stride_l = local_values.stride()[:3]
    a.local_mask = local_attention_mask.data_ptr()
    a.lm_stride_b, a.lm_stride_r, a.lm_stride_l = local_attention_mask.stride()
    a.key_cache = key_cache.data_ptr()
    a.kc_stride_s, a.kc_stride_h = key_cache.stride(0), key_cache.stride(2)
    a.value_cache = value_cache.data_ptr()
    a.vc_stride_s, a.vc_stride_h = value_cache.stride(0), value_cache.stride(2)
    a.page_table, a.pt_stride_b = page_table.data_ptr(), page_table.stride(0)
    a.raw_lengths = raw_lengths.data_ptr()
    a.output = output.data_ptr()
    a.o_stride_b, a.o_stride_h, a.o_stride_r = output.stride()[:3]
    _lib.call("ls_draft_attention", ctypes.byref(a), _lib.stream_of(dev))
    return output


def can_use_fused_global_local_raw_merge(*, query: torch.Tensor, global_keys: torch.Tensor,
                                         global_values: torch.Tensor, state_slots: Optional[torch.Tensor],
                                         local_keys: torch.Tensor, local_values: torch.Tensor,
                                         local_attention_mask: torch.Tensor, raw_output: torch.Tensor,
                                         raw_lse: torch.Tensor, output: torch.Tensor) -> bool:
    """The merge form's contract (SPEC/global16_raw256_draft_fused.py:314-369)."""
    batch, heads = (int(query.shape[0]), int(query.shape[1])) if query.ndim == 4 else (0, 0)
    return bool(
        query.is_cuda and query.dtype == torch.bfloat16 and query.ndim == 4
        and tuple(query.shape[2:]) == (QUERY_ROWS, HEAD_DIM)
        and tuple(global_keys.shape) == (batch, heads, GLOBAL_ROWS, HEAD_DIM)
        and global_keys.dtype == torch.bfloat16
        and global_values.is_cuda and global_values.dtype == torch.float32 and global_values.ndim == 4
        and tuple(global_values.shape[1:]) == (heads, GLOBAL_ROWS, HEAD_DIM)
        and state_slots is not None and state_slots.is_cuda and state_slots.dtype == torch.int32
        and tuple(state_slots.shape) == (batch,)
        and local_keys.shape == local_values.shape and local_keys.ndim == 4 and local_keys.shape[0] == batch
        and tuple(local_keys.shape[2:]) == (LOCAL_ROWS, HEAD_DIM)
        and heads % local_keys.shape[1] == 0
        and local_keys.dtype == query.dtype and local_values.dtype == query.dtype
        and local_attention_mask.is_cuda and local_attention_mask.dtype == torch.bool
        and tuple(local_attention_mask.shape) == (batch, QUERY_ROWS, LOCAL_ROWS)
        and raw_output.is_cuda and raw_output.dtype == query.dtype
        and tuple(raw_output.shape) == (batch * QUERY_ROWS, heads, HEAD_DIM)
        and raw_lse.is_cuda and raw_lse.dtype == torch.float32
        and tuple(raw_lse.shape) == (batch * QUERY_ROWS, heads)
        and output.is_cuda and output.dtype == query.dtype and output.shape == query.shape
    )


def fused_global_local_raw_merge(*, query: torch.Tensor, global_keys: torch.Tensor, global_values: torch.Tensor,
                                 state_slots: torch.Tensor, local_keys: torch.Tensor, local_values: torch.Tensor,
                                 local_attention_mask: torch.Tensor, raw_output: torch.Tensor,
                                 raw_lse: torch.Tensor, output: torch.Tensor, softmax_scale: float,
                                 softcap: float = 0.0, validate_contract: bool = True) -> torch.Tensor:
    """Merge the window attention with the summary and local sources into
    caller-owned ``output`` (SPEC/global16_raw256_draft_fused.py:417-479).
    The contract is checked even when ``validate_contract`` is False: the
    kernel relies on it."""
    ok = can_use_fused_global_local_raw_merge(
        query=query, global_keys=global_keys, global_values=global_values, state_slots=state_slots,
        local_keys=local_keys, local_values=local_values, local_attention_mask=local_attention_mask,
        raw_output=raw_output, raw_lse=raw_lse, output=output)
    if not ok:
        raise ValueError("Global16 fused Draft tensors violate the production contract")
    dev = _lib.require_cuda(query, global_keys, global_values, state_slots, local_keys, local_values,
                            local_attention_mask, raw_output, raw_lse, output, what="fused_global_local_raw_merge")
    for name, t in (("query", query), ("global_keys", global_keys), ("global_values", global_values),
                    ("local_keys", local_keys), ("local_values", local_values), ("raw_output", raw_output),
                    ("output", output)):
        if t.stride(-1) != 1:
            raise ValueError(f"fused_global_local_raw_merge: {name} needs a contiguous head dimension")
    a = _lib.DraftAttentionArgs()
    a.batch, a.q_heads, a.kv_heads = query.shape[0], query.shape[1], local_keys.shape[1]
    a.softmax_scale, a.softcap = float(softmax_scale), float(softcap or 0.0)
    a.query = query.data_ptr()
    a.q_stride_b, a.q_stride_h, a.q_stride_r = query.stride()[:3]
    a.global_keys = global_keys.data_ptr()
    a.gk_stride_b, a.gk_stride_h, a.gk_stride_g = global_keys.stride()[:3]
    a.global_values = global_values.data_ptr()
    a.gv_stride_b, a.gv_stride_h, a.gv_stride_g = global_values.stride()[:3]
    a.state_slots = state_slots.data_ptr()
    a.local_keys = local_keys.data_ptr()
    a.lk_stride_b, a.lk_stride_h, a.lk_stride_l = local_keys.stride()[:3]
    a.local_values = local_values.data_ptr()
    a.lv_stride_b, a.lv_stride_h, a.lv_stride_l = local_values.stride()[:3]
    a.local_mask = local_attention_mask.data_ptr()
    a.lm_stride_b, a.lm_stride_r, a.lm_stride_l = local_attention_mask.stride()
    a.raw_output = raw_output.data_ptr()
    a.ro_stride_t, a.ro_stride_h = raw_output.stride(0), raw_output.stride(1)
    a.raw_lse = raw_lse.data_ptr()
    a.rl_stride_t, a.rl_stride_h = raw_lse.stride()
    a.output = output.data_ptr()
    a.o_stride_b, a.o_stride_h, a.o_stride_r = output.stride()[:3]
    _lib.call("ls_draft_merge", ctypes.byref(a), _lib.stream_of(dev))
    return output
