"""Verify half of the hot path: drop-in replacements backed by the gfx950 kernels.

Each function keeps the reference call-site signature it replaces (cited per
function; ``SRT`` = ``vendor/sglang/python/sglang/srt``), validates shapes,
dtypes and devices on the host before launching -- raising ``ValueError`` as
the reference wrappers do -- and launches on torch's current stream without
synchronising the host.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _rows_view(logits: torch.Tensor, width: int, what: str) -> torch.Tensor:
    """``[B*K, V]`` (or ``[B, K, V]``) logits with unit stride along V."""
    if logits.ndim == 3:
        if logits.shape[1] != width:
            raise ValueError(f"{what}: logits second dim {logits.shape[1]} != block width {width}")
        logits = logits.reshape(-1, logits.shape[-1])
    if logits.ndim != 2:
        raise ValueError(f"{what}: logits must be [rows, vocab] or [batch, width, vocab]")
    if logits.stride(-1) != 1:
        raise ValueError(f"{what}: logits must be contiguous along the vocabulary")
    return logits


def verify_greedy(*, logits: torch.Tensor, candidates: torch.Tensor, width: int,
                  cand_first_col: int = 1, cutoff_verify_lens: Optional[torch.Tensor] = None,
                  return_truth: bool = False):
    """Fused greedy verify: row argmax, accepted prefix and bonus in one launch.

    ``logits`` ``[B*width, V]`` (bf16/fp16/fp32); ``candidates`` int32/int64
    with drafted token j of request b at ``candidates[b, cand_first_col + j]``.
    Returns ``(accept_lens i32[B], bonus i64[B], cap_trim i32[B])`` and, with
    ``return_truth``, the per-row argmax ``i32[B*width]``.
    """
    what = "verify_greedy"
    logits = _rows_view(logits, width, what)
    dev = _lib.require_cuda(logits, candidates, cutoff_verify_lens, what=what)
    if candidates.ndim != 2:
        raise ValueError(f"{what}: candidates must be rank-2")
    batch = candidates.shape[0]
    if width < 2 or logits.shape[0] != batch * width:
        raise ValueError(f"{what}: expected {batch}*{width} logits rows, got {logits.shape[0]}")
    if candidates.shape[1] < cand_first_col + width - 1:
        raise ValueError(f"{what}: candidates have {candidates.shape[1]} columns; "
                         f"need {cand_first_col + width - 1}")
    if candidates.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{what}: candidates must be int32 or int64")
    vocab = logits.shape[1]
    if cutoff_verify_lens is not None:
        if cutoff_verify_lens.shape != (batch,):
            raise ValueError(f"{what}: cutoff_verify_lens must be [batch]")
        cutoff_verify_lens = cutoff_verify_lens.to(torch.int32).contiguous()
    accept = torch.empty(batch, dtype=torch.int32, device=dev)
    bonus = torch.empty(batch, dtype=torch.int64, device=dev)
    trim = torch.empty(batch, dtype=torch.int32, device=dev)
    truth = torch.empty(batch * width, dtype=torch.int32, device=dev) if return_truth else None
    cnt, scr = _lib.workspaces.get(*_lib.workspace_sizes("ls_verify_greedy_workspace", batch, width, vocab),
                                   dev)
    _lib.call("ls_verify_greedy", logits.data_ptr(), _lib.dtype_code(logits), logits.stride(0),
              candidates.data_ptr(), _lib.dtype_code(candidates), candidates.stride(0),
              candidates.stride(1), cand_first_col, batch, width, vocab,
              _lib.ptr(cutoff_verify_lens), accept.data_ptr(), bonus.data_ptr(), _lib.ptr(truth),
              trim.data_ptr(), cnt.data_ptr(), cnt.numel(), scr.data_ptr(), scr.numel(), _lib.stream_of(dev))
    if return_truth:
        return accept, bonus, trim, truth
    return accept, bonus, trim


def accept_greedy(*, candidates: torch.Tensor, target_logits: torch.Tensor, verify_num_draft_tokens: int,
                  cutoff_verify_lens: Optional[torch.Tensor] = None):
    """SRT/speculative/dspark_components/kernels/accept_greedy.py:62-84 (and the
    Triton variant :114-135): ``(correct_len i32[B], bonus i64[B], cap_trim_lens i32[B])``."""
    return verify_greedy(logits=target_logits, candidates=candidates, width=verify_num_draft_tokens,
                         cand_first_col=1, cutoff_verify_lens=cutoff_verify_lens)


class AcceptGreedy:
    """SRT/speculative/dspark_components/kernels/accept_greedy.py:20-59 with a ``hip`` implementation."""

    @classmethod
    def execute(cls, *args, **kwargs):
        return cls.hip(*args, **kwargs)

    @classmethod
    def hip(cls, *, candidates, target_logits, verify_num_draft_tokens, cutoff_verify_lens=None):
        return accept_greedy(candidates=candidates, target_logits=target_logits,
                             verify_num_draft_tokens=verify_num_draft_tokens,
                             cutoff_verify_lens=cutoff_verify_lens)

    torch = hip
    triton = hip


def greedy_verify_split(drafted: torch.Tensor, logits: torch.Tensor):
    """Split-engine greedy branch, src/longspark/engine/target.py:472-477.

    ``drafted`` ``[B, gamma]`` (drafted tokens only), ``logits`` ``[B, gamma+1, V]``.
    Returns ``(accept i64[B], bonus i64[B])`` like the reference's
    ``cumprod(...).sum(1)`` and ``truth[rows, accept]``.
    """
    if logits.ndim != 3 or drafted.ndim != 2 or logits.shape[1] != drafted.shape[1] + 1:
        raise ValueError("greedy_verify_split: logits must be [B, gamma+1, V] for drafted [B, gamma]")
    accept, bonus, _ = verify_greedy(logits=logits, candidates=drafted, width=logits.shape[1],
                                     cand_first_col=0)
    return accept.to(torch.int64), bonus


def compute_greedy_accept_len_and_bonus_from_logits(*, candidates, target_logits, draft_token_num):
    """The argmax + SRT/speculative/draft_free_kv_utils.py:360-383 pair used by
    SRT/speculative/draft_free_kv_info.py:186-193, fused: ``(accept_lens i32, bonus i64)``."""
    accept, bonus, _ = verify_greedy(logits=target_logits, candidates=candidates, width=draft_token_num,
                                     cand_first_col=1)
    return accept, bonus
