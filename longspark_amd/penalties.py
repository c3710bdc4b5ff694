"""Penalties and vocabulary bitmask on the GPU (drop-ins for the reference's
logit-adjustment call sites).

``SRT`` = ``vendor/sglang/python/sglang/srt``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Union

import torch

from . import _lib


@dataclass
class PenaltyTables:
    """Compact per-request penalty state (see ``ls_penalty_tables`` in
    include/longspark_amd.h): presence bitmap, popcount ranks, additive value
    per present token, repetition scale, and the penalty application mode."""
    bits: torch.Tensor          # [B, ceil(V/32)] int32 (bit pattern)
    rank: torch.Tensor          # [B, ceil(V/32)] int32
    add: torch.Tensor           # [B, H] float32
    distinct: torch.Tensor      # [B] int32
    nonpositive: torch.Tensor   # [B] int32: 1 where every additive value is <= 0
    repetition: Optional[torch.Tensor]  # [B] float32 or None
    verify_quirk: bool = False
    has_additive: bool = True   # False: frequency and presence are off (add is all zero)


def build_penalty_tables(history: torch.Tensor, vocab: int, *, frequency=None, presence=None, repetition=None,
                         history_lens: Optional[torch.Tensor] = None, verify_quirk: bool = False) -> PenaltyTables:
    """Penalty tables from each request's output-token history ``[B, H]`` int32.

    ``frequency`` / ``presence`` / ``repetition`` are per-request ``[B]``
    values (None = the penaliser is off), as the reference penalisers take
    them from each request's sampling params
    (SRT/sampling/penaltylib/{frequency,presence,repetition}_penalty.py).
    ``verify_quirk`` selects the verify-path application of
    SRT/speculative/dflash_utils.py:176-191 (bias built on zeros).
    """
    what = "build_penalty_tables"
    dev = _lib.require_cuda(history, frequency, presence, repetition, history_lens, what=what)
    if history.ndim != 2 or history.dtype != torch.int32 or history.stride(1) != 1:
        raise ValueError(f"{what}: history must be [B, H] int32 with unit column stride")
    batch, cap = history.shape
    words = (vocab + 31) // 32
    bits = torch.empty(batch, words, dtype=torch.int32, device=dev)
    rank = torch.empty(batch, words, dtype=torch.int32, device=dev)
    add = torch.empty(batch, max(cap, 1), dtype=torch.float32, device=dev)
    distinct = torch.empty(batch, dtype=torch.int32, device=dev)
    nonpositive = torch.empty(batch, dtype=torch.int32, device=dev)

    def vec(t, name):
        if t is None:
            return None
        t = torch.as_tensor(t, device=dev, dtype=torch.float32).reshape(-1)
        if t.numel() == 1 and batch > 1:
            t = t.expand(batch).contiguous()
        if t.shape != (batch,):
            raise ValueError(f"{what}: {name} must have one value per request")
        return t.contiguous()

    frequency, presence, repetition = vec(frequency, "frequency"), vec(presence, "presence"), vec(repetition, "repetition")
    if history_lens is not None:
        history_lens = history_lens.to(torch.int32).contiguous()
    if batch > 0:  # an empty batch has empty tables
        _lib.call("ls_penalty_tables", history.data_ptr(), history.stride(0), _lib.ptr(history_lens), batch, cap,
                  vocab, _lib.ptr(frequency), _lib.ptr(presence), bits.data_ptr(), rank.data_ptr(), words, add.data_ptr(),
                  add.shape[1], distinct.data_ptr(), nonpositive.data_ptr(), _lib.stream_of(dev))
    return PenaltyTables(bits=bits, rank=rank, add=add, distinct=distinct, nonpositive=nonpositive,
                         repetition=repetition,
                         verify_quirk=verify_quirk, has_additive=frequency is not None or presence is not None)


def adjust_logits_(logits: torch.Tensor, *, rows_per_request: int, tables: Optional[PenaltyTables] = None,
                   vocab_mask: Optional[torch.Tensor] = None, mask_per_request: bool = False) -> None:
    """In place on ``[B*rows_per_request, V]`` logits: penalties, then the bitmask.

    Drop-in body of SRT/speculative/dflash_utils.py:127-213
    (``apply_dflash_verify_logits_adjustments``) with the penalty state given
    as tables.
    """
    what = "adjust_logits_"
    dev = _lib.require_cuda(logits, vocab_mask, what=what)
    if logits.ndim != 2 or logits.stride(1) != 1:
        raise ValueError(f"{what}: logits must be [rows, V] with unit column stride")
    rows, vocab = logits.shape
    if vocab_mask is not None:
        if vocab_mask.dtype != torch.int32 or vocab_mask.ndim != 2 or vocab_mask.stride(1) != 1:
            raise ValueError(f"{what}: vocab_mask must be [rows or B, W] int32")
        expect = rows // rows_per_request if mask_per_request else rows
        if vocab_mask.shape[0] != expect:
            raise ValueError(f"{what}: vocab_mask has {vocab_mask.shape[0]} rows, expected {expect}")
    if rows == 0:
        return
    t = tables
    _lib.call("ls_adjust_logits", logits.data_ptr(), _lib.dtype_code(logits), logits.stride(0), rows, vocab,
              rows_per_request,
              _lib.ptr(t.bits) if t else None, _lib.ptr(t.rank) if t else None, t.bits.stride(0) if t else 0,
              _lib.ptr(t.add) if (t and t.has_additive) else None, t.add.stride(0) if t else 0,
              _lib.ptr(t.repetition) if t else None, int(bool(t and t.verify_quirk)),
              _lib.ptr(vocab_mask), vocab_mask.stride(0) if vocab_mask is not None else 0,
              rows_per_request if mask_per_request else 1,
              vocab_mask.shape[1] if vocab_mask is not None else 0, _lib.stream_of(dev))


def apply_token_bitmask_inplace(logits: torch.Tensor, bitmask: torch.Tensor,
                                indices: Optional[Union[List[int], torch.Tensor]] = None) -> None:
    """SRT/constrained/triton_ops/bitmask_ops.py:84-141 (``apply_token_bitmask_inplace_triton``)
    and the ROCm binding ``sgl_kernel.apply_token_bitmask_inplace_cuda`` that
    SRT/constrained/xgrammar_backend.py:43-48 calls instead: bit 0 of
    ``bitmask[row, v >> 5] >> (v & 31)`` sets ``logits[row, v] = -inf`` for
    ``v < min(V, 32 * W)``; other columns are untouched.  ``indices`` (a list
    or tensor) selects the rows; the same index selects the logits row and
    the bitmask row.  The checks and their messages are the reference's
    assertions."""
    assert bitmask.dtype == torch.int32, "bitmask must be of type int32"
    if logits.ndim == 1:
        logits = logits.unsqueeze(0)
    if bitmask.ndim == 1:
        bitmask = bitmask.unsqueeze(0)
    required = (logits.shape[1] + 31) // 32
    assert required >= bitmask.shape[1], (
        f"Bitmask width too large: allow at most {required} int32s for logits' width {logits.shape[1]}, "
        f"but got {bitmask.shape[1]}")
    dev = _lib.require_cuda(logits, bitmask, what="apply_token_bitmask_inplace")
    if isinstance(indices, (list, torch.Tensor)):
        idx = torch.as_tensor(indices, dtype=torch.int32, device=dev).reshape(-1).contiguous()
        num_rows = idx.shape[0]
    else:
        assert logits.shape[0] == bitmask.shape[0], (
            f"batch size mismatch: logits {logits.shape[0]} vs bitmask {bitmask.shape[0]}")
        idx, num_rows = None, logits.shape[0]
    if logits.stride(-1) != 1 or bitmask.stride(-1) != 1:
        raise ValueError("apply_token_bitmask_inplace: logits and bitmask rows must be contiguous")
    if num_rows == 0 or logits.shape[0] == 0 or bitmask.shape[1] == 0:
        return
    _lib.call("ls_apply_token_bitmask", logits.data_ptr(), _lib.dtype_code(logits), logits.stride(0),
              logits.shape[0], logits.shape[1], bitmask.data_ptr(), bitmask.stride(0), bitmask.shape[0],
              bitmask.shape[1], _lib.ptr(idx), _lib.LS_I32, num_rows, _lib.stream_of(dev))


def _request_rows(t: Optional[torch.Tensor], batch: int, vocab: int, what: str, name: str):
    """fp32 ``[batch, vocab]`` with unit column stride (other float dtypes
    convert exactly)."""
    if t is None:
        return None
    if t.ndim == 1:
        t = t.unsqueeze(0)
    if t.shape != (batch, vocab):
        raise ValueError(f"{what}: {name} must be [{batch}, {vocab}], got {tuple(t.shape)}")
    if t.dtype != torch.float32:
        t = t.float()
    if t.stride(1) != 1:
        t = t.contiguous()
    return t


def add_request_bias_(logits: torch.Tensor, *, rows_per_request: int, bias: Optional[torch.Tensor] = None,
                      vocab_mask: Optional[torch.Tensor] = None, bias2: Optional[torch.Tensor] = None,
                      separate: bool = False) -> None:
    """In place on ``[B*rows_per_request, V]`` logits (``ls_add_request_bias``).

    ``separate=False`` (SRT/speculative/dflash_utils.py:176-191): one combined
    bias per request -- ``bias`` (0 when None), columns whose packed
    ``vocab_mask`` bit is 0 set to -inf, plus ``bias2`` -- rounded to the
    logits' dtype and added.  ``separate=True`` (:193-213): ``bias`` then
    ``bias2`` added one after the other, each rounded to the logits' dtype.
    """
    what = "add_request_bias_"
    dev = _lib.require_cuda(logits, bias, vocab_mask, bias2, what=what)
    if logits.ndim != 2 or logits.stride(1) != 1:
        raise ValueError(f"{what}: logits must be [rows, V] with unit column stride")
    rows, vocab = logits.shape
    if rows_per_request <= 0 or rows % rows_per_request != 0:
        raise ValueError(f"{what}: {rows} rows are not a multiple of {rows_per_request}")
    batch = rows // rows_per_request
    bias = _request_rows(bias, batch, vocab, what, "bias")
    bias2 = _request_rows(bias2, batch, vocab, what, "bias2")
    if vocab_mask is not None:
        if separate:
            raise ValueError(f"{what}: the mask belongs to the combined form")
        if vocab_mask.dtype != torch.int32 or vocab_mask.ndim != 2 or vocab_mask.shape[0] != batch or \
                vocab_mask.stride(1) != 1 or vocab_mask.shape[1] > (vocab + 31) // 32:
            raise ValueError(f"{what}: vocab_mask must be int32 [{batch}, <= {(vocab + 31) // 32}]")
    if rows == 0:
        return
    _lib.call("ls_add_request_bias", logits.data_ptr(), _lib.dtype_code(logits), logits.stride(0), rows, vocab,
              rows_per_request, _lib.ptr(bias), bias.stride(0) if bias is not None else 0,
              _lib.ptr(vocab_mask), vocab_mask.stride(0) if vocab_mask is not None else 0,
              vocab_mask.shape[1] if vocab_mask is not None else 0,
              _lib.ptr(bias2), bias2.stride(0) if bias2 is not None else 0, int(bool(separate)),
              _lib.stream_of(dev))


def _custom_logit_processor(logits, sampling_info, draft_token_num):
    try:  # the caller's own processors live in the serving stack
        from sglang.srt.layers.sampler import apply_custom_logit_processor
    except ImportError as e:
        raise RuntimeError("custom logit processors need the serving stack's apply_custom_logit_processor") from e
    apply_custom_logit_processor(logits, sampling_info, num_tokens_in_batch=draft_token_num)


def apply_dflash_verify_logits_adjustments(*, next_token_logits: torch.Tensor, sampling_info,
                                           draft_token_num: int) -> None:
    """Drop-in for SRT/speculative/dflash_utils.py:127-213, in place.

    The dense path (live penalisers without ``acc_linear_penalties``, or a
    grammar mask) builds the request bias exactly as the reference does --
    ``sampling_info.apply_logits_bias`` on a zero fp32 ``[B, V]`` tensor, so
    scaling penalties act on zeros -- and the gfx950 kernel adds it to all
    ``draft_token_num`` rows of each request in the logits' dtype.  Otherwise
    ``acc_linear_penalties`` and ``logit_bias`` are added one after the other
    by the same kernel.
    """
    if sampling_info is None:
        return
    if next_token_logits.ndim != 2:
        raise ValueError(f"next_token_logits must be 2D, got shape={tuple(next_token_logits.shape)}.")
    if draft_token_num <= 0:
        raise ValueError(f"draft_token_num must be positive, got {draft_token_num}.")
    bs = len(sampling_info)
    if next_token_logits.shape[0] != bs * draft_token_num:
        raise ValueError("next_token_logits row count mismatch for DFlash verify adjustments. "
                         f"Expected {bs * draft_token_num}, got {next_token_logits.shape[0]}.")
    if getattr(sampling_info, "has_custom_logit_processor", False):
        _custom_logit_processor(next_token_logits, sampling_info, draft_token_num)
    acc = getattr(sampling_info, "acc_linear_penalties", None)
    penalizer = getattr(sampling_info, "penalizer_orchestrator", None)
    vocab_mask = getattr(sampling_info, "vocab_mask", None)
    logit_bias = getattr(sampling_info, "logit_bias", None)
    vocab = next_token_logits.shape[1]
    if (penalizer is not None and penalizer.is_required and acc is None) or vocab_mask is not None:
        linear_penalty = torch.zeros((bs, vocab), dtype=torch.float32, device=next_token_logits.device)
        sampling_info.apply_logits_bias(linear_penalty)
        add_request_bias_(next_token_logits, rows_per_request=draft_token_num, bias=linear_penalty)
        return
    if acc is None and logit_bias is None:
        return
    add_request_bias_(next_token_logits, rows_per_request=draft_token_num, bias=acc, bias2=logit_bias,
                      separate=True)
