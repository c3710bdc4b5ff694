"""Verify half of the hot path: drop-in replacements backed by the gfx950 kernels.

Each function keeps the reference call-site signature it replaces (cited per
function; ``SRT`` = ``vendor/sglang/python/sglang/srt``), validates shapes,
dtypes and devices on the host before launching -- raising ``ValueError`` as
the reference wrappers do -- and launches on torch's current stream without
synchronising the host.
"""

from __future__ import annotations

from dataclasses import dataclass
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
    if batch == 0:  # an empty batch: empty outputs, as the reference's tensor code gives
        return (accept, bonus, trim, truth) if return_truth else (accept, bonus, trim)
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


# --------------------------------------------------------------------------
# split-engine two-phase rejection sampling (dense target probabilities)
# --------------------------------------------------------------------------

@dataclass
class AcceptanceDecision:
    """Same fields as src/longspark/engine/sampling.py:11-16."""
    lengths: torch.Tensor
    rejected_rows: torch.Tensor
    rejection_positions: torch.Tensor
    target_rows: torch.Tensor


def decide_acceptance(*, candidates, sampled_q, target_probs, uniforms) -> AcceptanceDecision:
    """src/longspark/engine/sampling.py:19-35 on the GPU.

    ``candidates`` ``[B, gamma]`` drafted tokens, ``sampled_q`` / ``uniforms``
    ``[B, gamma]`` fp32, ``target_probs`` ``[B, gamma+1, V]`` fp32.  The
    accepted lengths and the target row at each length come from one kernel;
    ``rejected_rows`` (a data-dependent size) is selected with torch from the
    lengths, as the reference does.
    """
    what = "decide_acceptance"
    batch, gamma = candidates.shape
    if sampled_q.shape != (batch, gamma) or uniforms.shape != (batch, gamma):
        raise ValueError("sampled q and uniforms must match the seven proposal positions")
    if target_probs.shape[:2] != (batch, gamma + 1):
        raise ValueError("target must verify proposal width plus one bonus row")
    dev = _lib.require_cuda(candidates, sampled_q, target_probs, uniforms, what=what)
    if target_probs.dtype != torch.float32 or sampled_q.dtype != torch.float32 or uniforms.dtype != torch.float32:
        raise ValueError(f"{what}: probabilities, q and uniforms must be fp32")
    if target_probs.stride(2) != 1 or sampled_q.stride(1) != 1 or uniforms.stride(1) != 1:
        raise ValueError(f"{what}: the last dimension must be contiguous")
    vocab = target_probs.shape[2]
    lengths = torch.empty(batch, dtype=torch.int64, device=dev)
    rows = torch.empty(batch, vocab, dtype=torch.float32, device=dev)
    _lib.call("ls_decide_acceptance", candidates.data_ptr(), _lib.dtype_code(candidates), candidates.stride(0),
              candidates.stride(1), sampled_q.data_ptr(), sampled_q.stride(0), uniforms.data_ptr(),
              uniforms.stride(0), target_probs.data_ptr(), target_probs.stride(0), target_probs.stride(1), batch,
              gamma, vocab, lengths.data_ptr(), rows.data_ptr(), rows.stride(0), _lib.stream_of(dev))
    rejected = torch.arange(batch, device=dev)[lengths < gamma]
    return AcceptanceDecision(lengths=lengths, rejected_rows=rejected, rejection_positions=lengths[rejected],
                              target_rows=rows)


def finish_sampling(decision: AcceptanceDecision, rejected_q_rows, *, generator=None, uniforms=None):
    """src/longspark/engine/sampling.py:38-57 on the GPU.

    With ``uniforms`` the token is ``#{v : u >= CDF(v)}`` of the request's
    distribution (the normalised residual for rejected requests), clamped to
    V-1.  Without them, one uniform per request is drawn from ``generator``
    on the device and used the same way, which samples the same distribution
    as the reference's ``torch.multinomial``.
    """
    what = "finish_sampling"
    target = decision.target_rows
    expected = (decision.rejected_rows.numel(), target.shape[-1])
    if rejected_q_rows.shape != expected:
        raise ValueError(f"expected rejected q shape {expected}, got {rejected_q_rows.shape}")
    batch, vocab = target.shape
    dev = _lib.require_cuda(target, rejected_q_rows, decision.rejected_rows, uniforms, what=what)
    if uniforms is None:
        uniforms = torch.rand(batch, generator=generator, device=dev)
    if uniforms.shape != (batch,):
        raise ValueError("one final uniform is required per request")
    if target.dtype != torch.float32 or rejected_q_rows.dtype != torch.float32:
        raise ValueError(f"{what}: target rows and q rows must be fp32")
    if target.stride(1) != 1 or (rejected_q_rows.numel() and rejected_q_rows.stride(1) != 1):
        raise ValueError(f"{what}: rows must be contiguous")
    rej = decision.rejected_rows.to(torch.int64).contiguous()
    uniforms = uniforms.to(torch.float32).contiguous()
    out = torch.empty(batch, dtype=torch.int64, device=dev)
    _lib.call("ls_finish_sampling", target.data_ptr(), target.stride(0), rej.data_ptr(), rej.numel(),
              rejected_q_rows.data_ptr(), rejected_q_rows.stride(0) if rejected_q_rows.numel() else 0,
              uniforms.data_ptr(), batch, vocab, out.data_ptr(), _lib.stream_of(dev))
    return out


# --------------------------------------------------------------------------
# fixed-width verify outputs
# --------------------------------------------------------------------------

def _finalize(candidates, accept_lens, bonus, prefix_lens, what, with_counts):
    if candidates.ndim != 2 or candidates.shape[1] < 2:
        raise ValueError("verification candidates must have shape [batch, width>=2]")
    batch, width = candidates.shape
    named = [("accept_lens", accept_lens), ("bonus", bonus)] + ([("prefix_lens", prefix_lens)] if with_counts else [])
    for name, value in named:
        if value.shape != (batch,) or value.device != candidates.device:
            raise ValueError(f"{name} must have one device row per request")
        if value.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"{name} must have an integer dtype")
    dev = _lib.require_cuda(candidates, accept_lens, bonus, prefix_lens, what=what)
    out = torch.empty((batch, width), device=dev, dtype=torch.int64)
    committed = next_lengths = None
    if with_counts:
        committed = torch.empty((batch,), device=dev, dtype=torch.int32)
        next_lengths = torch.empty((batch,), device=prefix_lens.device, dtype=prefix_lens.dtype)
    _lib.call("ls_finalize_verify_outputs", candidates.data_ptr(), _lib.dtype_code(candidates), candidates.stride(0),
              candidates.stride(1), accept_lens.data_ptr(), _lib.dtype_code(accept_lens), accept_lens.stride(0),
              bonus.data_ptr(), _lib.dtype_code(bonus), bonus.stride(0),
              _lib.ptr(prefix_lens), _lib.dtype_code(prefix_lens) if with_counts else _lib.LS_I64,
              prefix_lens.stride(0) if with_counts else 0, batch, width, out.data_ptr(), _lib.ptr(committed),
              _lib.ptr(next_lengths), _lib.stream_of(dev))
    return out, committed, next_lengths


def finalize_verify_outputs(*, candidates, accept_lens, bonus, prefix_lens):
    """SRT/speculative/draft_free_kv_dispatch.py:32-57: ``(out_tokens i64 [B, W],
    committed i32 [B], next_lengths [B])``; fresh tensors, as the scheduler may keep them."""
    return _finalize(candidates, accept_lens, bonus, prefix_lens, "finalize_verify_outputs", True)


def assign_fixed_verify_cache_locs(*, req_pool_indices: torch.Tensor, req_to_token: torch.Tensor,
                                   start_offset: torch.Tensor, commit_lens: torch.Tensor,
                                   verify_cache_locs: torch.Tensor, batch_size: int, verify_width: int) -> None:
    """SRT/speculative/draft_free_kv_info.py:62-82 (``_assign_fixed_verify_cache_locs_func``):
    in place, ``req_to_token[slot_b, start_b + i] = verify_cache_locs[b, i]``
    for ``i < commit_lens[b]``."""
    what = "assign_fixed_verify_cache_locs"
    if verify_cache_locs.shape != (batch_size, verify_width):
        raise ValueError("fixed verify cache locations have the wrong shape")
    dev = _lib.require_cuda(req_pool_indices, req_to_token, start_offset, commit_lens, verify_cache_locs, what=what)
    if req_to_token.dtype != torch.int32 or req_to_token.ndim != 2 or req_to_token.stride(1) != 1:
        raise ValueError(f"{what}: req_to_token must be int32 [slots, pool_len] with unit column stride")
    for name, t in (("req_pool_indices", req_pool_indices), ("start_offset", start_offset),
                    ("commit_lens", commit_lens)):
        if t.shape != (batch_size,):
            raise ValueError(f"{what}: {name} must have one entry per request")
    idx = [t.contiguous() for t in (req_pool_indices, start_offset, commit_lens)]
    locs = verify_cache_locs if verify_cache_locs.stride(1) == 1 else verify_cache_locs.contiguous()
    _lib.call("ls_assign_verify_cache_locs", idx[0].data_ptr(), _lib.dtype_code(idx[0]), idx[1].data_ptr(),
              _lib.dtype_code(idx[1]), idx[2].data_ptr(), _lib.dtype_code(idx[2]), locs.data_ptr(),
              _lib.dtype_code(locs), locs.stride(0), req_to_token.data_ptr(), req_to_token.stride(0),
              req_to_token.shape[1], batch_size, verify_width, _lib.stream_of(dev))


def build_greedy_verify_out_tokens(*, candidates, accept_lens, bonus):
    """SRT/speculative/draft_free_kv_utils.py:386-408: the ``[B, W]`` int64 committed-token buffer."""
    if candidates.ndim != 2 or accept_lens.shape != (candidates.shape[0],):
        raise ValueError("DRAFT_FREE_KV verify tensors have incompatible shapes")
    if bonus.shape != (candidates.shape[0],):
        raise ValueError("DRAFT_FREE_KV bonus must have one token per request")
    return _finalize(candidates, accept_lens, bonus, None, "build_greedy_verify_out_tokens", False)[0]


# --------------------------------------------------------------------------
# stochastic verification
# --------------------------------------------------------------------------

def _per_request(t, batch, dtype, dev, name, what):
    if t is None:
        return None
    t = torch.as_tensor(t, device=dev).reshape(-1)
    if t.numel() == 1 and batch > 1:
        t = t.expand(batch)
    if t.shape != (batch,):
        raise ValueError(f"{what}: {name} must have one value per request")
    return t.to(dtype).contiguous()


def verify_sample(*, logits: torch.Tensor, candidates: torch.Tensor, width: int, temperatures,
                  uniforms: torch.Tensor, final_uniforms: torch.Tensor, top_ks=None, top_ps=None, min_ps=None,
                  max_top_k: Optional[int] = None, draft_token_probs: Optional[torch.Tensor] = None,
                  draft_logits: Optional[torch.Tensor] = None, draft_probs: Optional[torch.Tensor] = None,
                  draft_temperatures=None, draft_top_ks=None, draft_top_ps=None, draft_min_ps=None,
                  penalties=None, vocab_mask: Optional[torch.Tensor] = None, mask_per_request: bool = False,
                  cand_first_col: int = 1, return_p_cand: bool = False, check: bool = False,
                  timing_events=None, scan_hint: int = 0, cutoff_verify_lens: Optional[torch.Tensor] = None,
                  return_cap_trim: bool = False):
    """Fused stochastic verify of a drafted block (one call, three kernels).

    Target: ``logits`` ``[B*width, V]`` (bf16/fp16/fp32) with penalties
    (``penalties``: :class:`longspark_amd.penalties.PenaltyTables`) and a packed
    ``vocab_mask`` applied on the fly, then temperature / top-k / top-p /
    min-p (per-request ``[B]`` values; None disables).
    Draft: either ``draft_token_probs [B, width-1]`` (q of each drafted token)
    with ``draft_logits [B, width-1, V]`` (q row rebuilt at the rejection with
    the ``draft_*`` parameters; pure temperature when they are None), or dense
    ``draft_probs [B, width-1, V]`` fp32 (q read directly).
    Randomness: ``uniforms [B, width-1]`` and ``final_uniforms [B]`` fp32.
    ``cutoff_verify_lens`` ``[B]``: the accepted length is capped at
    ``cutoff - 1`` (a capped request's bonus is its drafted token at the cap).
    Returns ``(accept_lens i32[B], bonus i64[B])``, then ``cap_trim i32[B]``
    with ``return_cap_trim`` and the per-drafted-token target probabilities
    ``[B, width-1]`` with ``return_p_cand``.  With
    ``check`` the call synchronises and raises if a request could not be
    resolved (such requests get -1 in both outputs).  ``timing_events``: an
    optional ctypes array of 4 hipEvent_t recorded around the kernels.
    ``scan_hint``: 0 launches both row-scan kernels; 1 only the raw-logit
    top-k scan (when every request uses top-k with repetition >= 1 and
    non-negative frequency / presence); 2 only the exact scan.  A wrong hint
    costs speed, never correctness.
    """
    what = "verify_sample"
    logits = _rows_view(logits, width, what)
    draft = draft_probs if draft_probs is not None else draft_logits
    dev = _lib.require_cuda(logits, candidates, uniforms, final_uniforms, draft, draft_token_probs, vocab_mask,
                            cutoff_verify_lens, what=what)
    if candidates.ndim != 2 or candidates.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"{what}: candidates must be [B, C] int32/int64")
    batch = candidates.shape[0]
    vocab = logits.shape[1]
    g = width - 1
    if width < 2 or logits.shape[0] != batch * width:
        raise ValueError(f"{what}: expected {batch}*{width} logits rows, got {logits.shape[0]}")
    if candidates.shape[1] < cand_first_col + g:
        raise ValueError(f"{what}: candidates need {cand_first_col + g} columns")
    if draft is None:
        raise ValueError(f"{what}: draft_logits (with draft_token_probs) or draft_probs is required")
    q_mode = 1 if draft_probs is not None else 0
    if draft.ndim != 3 or draft.shape != (batch, g, vocab) or draft.stride(2) != 1:
        raise ValueError(f"{what}: draft rows must be [B, width-1, V] with unit vocabulary stride")
    if q_mode == 1 and draft.dtype != torch.float32:
        raise ValueError(f"{what}: draft_probs must be fp32")
    if q_mode == 0:
        if draft_token_probs is None or draft_token_probs.shape != (batch, g) or \
                draft_token_probs.dtype != torch.float32:
            raise ValueError(f"{what}: draft_token_probs must be [B, width-1] fp32")
        draft_token_probs = draft_token_probs.contiguous()
    if uniforms.shape != (batch, g) or uniforms.dtype != torch.float32 or uniforms.stride(1) != 1:
        raise ValueError(f"{what}: uniforms must be [B, width-1] fp32")
    if final_uniforms.shape != (batch,) or final_uniforms.dtype != torch.float32:
        raise ValueError(f"{what}: final_uniforms must be [B] fp32")
    final_uniforms = final_uniforms.contiguous()
    temps = _per_request(temperatures, batch, torch.float32, dev, "temperatures", what)
    if temps is None:
        raise ValueError(f"{what}: temperatures are required")
    top_ks = _per_request(top_ks, batch, torch.int32, dev, "top_ks", what)
    top_ps = _per_request(top_ps, batch, torch.float32, dev, "top_ps", what)
    min_ps = _per_request(min_ps, batch, torch.float32, dev, "min_ps", what)
    d_t = _per_request(draft_temperatures, batch, torch.float32, dev, "draft_temperatures", what)
    d_k = _per_request(draft_top_ks, batch, torch.int32, dev, "draft_top_ks", what)
    d_p = _per_request(draft_top_ps, batch, torch.float32, dev, "draft_top_ps", what)
    d_m = _per_request(draft_min_ps, batch, torch.float32, dev, "draft_min_ps", what)
    if vocab_mask is not None:
        words = (vocab + 31) // 32
        rows_m = batch if mask_per_request else batch * width
        if vocab_mask.dtype != torch.int32 or vocab_mask.shape != (rows_m, words) or vocab_mask.stride(1) != 1:
            raise ValueError(f"{what}: vocab_mask must be [{rows_m}, {words}] int32")
    mk = 0 if max_top_k is None else int(max_top_k)
    if cutoff_verify_lens is not None:
        if cutoff_verify_lens.shape != (batch,):
            raise ValueError(f"{what}: cutoff_verify_lens must be [batch]")
        cutoff_verify_lens = cutoff_verify_lens.to(torch.int32).contiguous()

    accept = torch.empty(batch, dtype=torch.int32, device=dev)
    trim = torch.empty(batch, dtype=torch.int32, device=dev) if return_cap_trim else None  # written per request
    bonus = torch.empty(batch, dtype=torch.int64, device=dev)
    p_cand = torch.empty(batch, g, dtype=torch.float32, device=dev) if return_p_cand else None
    if batch == 0:  # an empty batch: empty outputs, as the reference's tensor code gives
        out = (accept, bonus)
        if return_cap_trim:
            out += (trim,)
        if return_p_cand:
            out += (p_cand,)
        return out
    status = torch.empty(1, dtype=torch.int32, device=dev)  # cleared by the call's first kernel
    a = _lib.VerifySampleArgs()
    a.logits, a.logits_dtype, a.logits_row_stride = logits.data_ptr(), _lib.dtype_code(logits), logits.stride(0)
    a.candidates, a.candidates_dtype = candidates.data_ptr(), _lib.dtype_code(candidates)
    a.cand_stride_b, a.cand_stride_k, a.cand_first_col = candidates.stride(0), candidates.stride(1), cand_first_col
    a.batch, a.width, a.vocab = batch, width, vocab
    a.temperatures, a.top_ks, a.top_ps, a.min_ps = _lib.ptr(temps), _lib.ptr(top_ks), _lib.ptr(top_ps), _lib.ptr(min_ps)
    a.max_top_k = mk
    t = penalties
    if t is not None:
        a.pen_bits, a.pen_rank, a.pen_words_stride = t.bits.data_ptr(), t.rank.data_ptr(), t.bits.stride(0)
        a.pen_add, a.pen_add_stride = (t.add.data_ptr() if t.has_additive else None), t.add.stride(0)
        a.pen_repetition, a.pen_verify_quirk = _lib.ptr(t.repetition), int(bool(t.verify_quirk))
        a.pen_nonpositive = t.nonpositive.data_ptr()
    if vocab_mask is not None:
        a.vocab_mask, a.mask_row_stride, a.mask_per_request = vocab_mask.data_ptr(), vocab_mask.stride(0), \
            int(mask_per_request)
    a.q_mode = q_mode
    if q_mode == 0:
        a.draft_token_probs, a.dtp_stride_b = draft_token_probs.data_ptr(), draft_token_probs.stride(0)
    a.draft, a.draft_dtype, a.draft_stride_b, a.draft_stride_k = draft.data_ptr(), _lib.dtype_code(draft), \
        draft.stride(0), draft.stride(1)
    a.draft_temperatures, a.draft_top_ks = _lib.ptr(d_t), _lib.ptr(d_k)
    a.draft_top_ps, a.draft_min_ps = _lib.ptr(d_p), _lib.ptr(d_m)
    a.uniforms, a.uniform_stride_b, a.final_uniforms = uniforms.data_ptr(), uniforms.stride(0), \
        final_uniforms.data_ptr()
    a.accept_lens, a.bonus, a.p_cand_out, a.status = accept.data_ptr(), bonus.data_ptr(), _lib.ptr(p_cand), \
        status.data_ptr()
    if scan_hint not in (0, 1, 2):
        raise ValueError(f"{what}: scan_hint must be 0, 1 or 2")
    a.scan_hint = scan_hint
    a.cutoff_verify_lens, a.cap_trim = _lib.ptr(cutoff_verify_lens), _lib.ptr(trim)
    if timing_events is not None:
        a.timing_events = _lib.ctypes.cast(timing_events, _lib.ctypes.c_void_p)
    cnt, scr = _lib.workspaces.get(*_lib.workspace_sizes("ls_verify_sample_workspace", batch, width, vocab, mk), dev)
    _lib.call("ls_verify_sample", ctypes_byref(a), cnt.data_ptr(), cnt.numel(), scr.data_ptr(), scr.numel(),
              _lib.stream_of(dev))
    if check:
        torch.cuda.synchronize(dev)
        if int(status.item()) != 0:
            raise RuntimeError(f"{what}: a request's sampling support exceeded the kernel capacity")
    out = (accept, bonus)
    if return_cap_trim:
        out += (trim,)
    if return_p_cand:
        out += (p_cand,)
    return out


def ctypes_byref(struct):
    import ctypes
    return ctypes.byref(struct)
