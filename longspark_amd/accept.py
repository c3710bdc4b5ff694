"""Acceptance dispatch of the stochastic verify: drop-ins backed by the gfx950 kernels.

* ``AcceptSampling`` -- SPEC/dspark_components/kernels/accept_sampling.py:25-90:
  ``execute`` (dense draft probabilities, chain rule) and ``execute_single_q``
  (only the sampled tokens' q; the q row is rebuilt from the draft logits at
  the rejection) both run the fused verify (``ls_verify_sample``), which
  builds the target distribution from the logits inside the row scan.
* ``chain_speculative_sampling_triton`` -- SPEC/reject_sampling.py:159-204 on
  caller-given dense target and draft probabilities
  (``ls_chain_speculative_sampling``).
* ``accept_draft_tokens`` / ``accept_scheduled_greedy_tokens`` --
  SPEC/dspark_components/dspark_accept.py:20-159: the greedy / single-q /
  dense-q / mixed dispatch.

``SPEC`` = ``vendor/sglang/python/sglang/srt/speculative``.  Uniforms are drawn
with ``torch.rand`` on the device in the reference's order (``gamma`` per
request, then one final per request), so a seeded generator gives the
reference's draws.
"""

from __future__ import annotations

from typing import Any, Optional

import torch

from . import _lib, dense, verify

RESIDUAL_MASS_EPS = 1e-8  # accept_sampling.py:22 (single-q: below it the bonus comes from p)


def _draws(bs: int, gamma: int, width: int, device):
    """``torch.rand((bs, gamma))`` then ``torch.rand((bs,))`` (accept_sampling.py:124-125,
    :297-303); the chain reads the first ``width - 1`` per request."""
    if gamma < width - 1:
        raise ValueError(f"gamma {gamma} is smaller than the verify width - 1 ({width - 1})")
    u = torch.rand((bs, gamma), dtype=torch.float32, device=device)
    uf = torch.rand((bs,), dtype=torch.float32, device=device)
    return u[:, :width - 1], uf


def _temperatures(sampling_info, bs: int) -> torch.Tensor:
    t = sampling_info.temperatures.reshape(-1)
    if t.numel() != bs:
        raise ValueError("sampling_info.temperatures must hold one value per request")
    return t


def _validate_single_q(*, candidates, target_logits, corrected_logits, draft_token_probs, draft_temperatures,
                       sampling_info, gamma, verify_num_draft_tokens):
    """Shape / dtype / device contract of accept_sampling.py:209-256 (same messages)."""
    if candidates.ndim != 2:
        raise ValueError("single-q acceptance candidates must be two-dimensional")
    bs, candidate_rows = candidates.shape
    if candidate_rows != verify_num_draft_tokens or gamma != candidate_rows - 1:
        raise ValueError("single-q acceptance requires gamma = verify width - 1")
    if target_logits.ndim != 2 or target_logits.shape[0] != bs * candidate_rows:
        raise ValueError("single-q acceptance target logits have an invalid shape")
    if corrected_logits.ndim != 3 or corrected_logits.shape[:2] != (bs, gamma):
        raise ValueError("single-q acceptance corrected logits must be [batch, gamma, vocab]")
    if draft_token_probs.ndim != 2 or draft_token_probs.shape != (bs, gamma):
        raise ValueError("single-q acceptance probabilities must be [batch, gamma]")
    if corrected_logits.shape[-1] != target_logits.shape[-1]:
        raise ValueError("single-q acceptance logits use different vocabularies")
    if draft_temperatures.numel() != bs:
        raise ValueError("single-q acceptance temperatures must have one value per request")
    if draft_token_probs.dtype != torch.float32:
        raise ValueError("single-q acceptance probabilities must be FP32")
    tensors = {"target logits": target_logits, "corrected logits": corrected_logits,
               "draft probabilities": draft_token_probs, "draft temperatures": draft_temperatures,
               "target temperatures": sampling_info.temperatures}
    mismatched = [name for name, t in tensors.items() if t.device != candidates.device]
    if mismatched:
        raise ValueError("single-q acceptance inputs must share a device; mismatched: " + ", ".join(mismatched))
    return bs


def accept_sampling_single_q(*, candidates: torch.Tensor, target_logits: torch.Tensor,
                             corrected_logits: torch.Tensor, draft_token_probs: torch.Tensor,
                             draft_temperatures: torch.Tensor, sampling_info, draft_input: Any, gamma: int,
                             verify_num_draft_tokens: int, cutoff_verify_lens: Optional[torch.Tensor] = None):
    """accept_sampling.py:259-343: pure-temperature target (SoftmaxTemp of the
    logits), acceptance ``u * q < p``, bonus from ``max(p - q, 0)`` with q
    rebuilt as ``softmax(corrected[b, L] / T_draft)`` (p itself below the
    1e-8 residual mass).  Returns ``(correct_len i32, bonus i64, zeros i32)``."""
    del draft_input
    if cutoff_verify_lens is not None:
        raise ValueError("single-q acceptance does not support cutoff layouts")
    bs = _validate_single_q(candidates=candidates, target_logits=target_logits, corrected_logits=corrected_logits,
                            draft_token_probs=draft_token_probs, draft_temperatures=draft_temperatures,
                            sampling_info=sampling_info, gamma=gamma,
                            verify_num_draft_tokens=verify_num_draft_tokens)
    u, uf = _draws(bs, gamma, verify_num_draft_tokens, candidates.device)
    lens, bonus = verify.verify_sample(
        logits=target_logits, candidates=candidates, width=verify_num_draft_tokens,
        temperatures=_temperatures(sampling_info, bs), uniforms=u, final_uniforms=uf,
        draft_token_probs=draft_token_probs, draft_logits=corrected_logits,
        draft_temperatures=draft_temperatures.reshape(-1))
    return lens, bonus, torch.zeros_like(lens)


def accept_sampling(*, candidates: torch.Tensor, target_logits: torch.Tensor, draft_probs: torch.Tensor,
                    sampling_info, draft_input: Any, gamma: int, verify_num_draft_tokens: int,
                    cutoff_verify_lens: Optional[torch.Tensor] = None):
    """accept_sampling.py:93-187: target distribution as SoftmaxTemp (no top-k /
    top-p requested) or build_dflash_verify_target_probs (top-k first with the
    draft input's ``max_top_k``, then top-p), chain acceptance against the
    dense draft probabilities, bonus from ``max(p - q, 0)`` (vocab-1 when it is
    all zero), then the cutoff cap.  Fused in one verify call that never
    materialises the target probabilities.  Returns
    ``(correct_len i32, bonus i64, cap_trim_lens i32)``."""
    if candidates.ndim != 2:
        raise ValueError("accept_sampling: candidates must be [batch, width]")
    bs, width = candidates.shape
    if width != verify_num_draft_tokens:
        raise ValueError("accept_sampling: candidates width must equal verify_num_draft_tokens")
    vocab = int(target_logits.shape[-1])
    if draft_probs.ndim != 3 or draft_probs.shape[0] != bs or draft_probs.shape[1] < width - 1 or \
            draft_probs.shape[2] != vocab:
        raise ValueError("accept_sampling: draft_probs must be [batch, >= width-1, vocab]")
    need_top_k = bool(getattr(sampling_info, "need_top_k_sampling", True))
    need_top_p = bool(getattr(sampling_info, "need_top_p_sampling", False))
    ks = ps = mk = None
    if need_top_k or need_top_p:
        ks, ps, mk = dense.dflash_filter_params(sampling_info, vocab, getattr(draft_input, "max_top_k", None))
    u, uf = _draws(bs, gamma, width, candidates.device)
    q = draft_probs[:, :width - 1]
    if q.dtype != torch.float32:
        raise ValueError("accept_sampling: draft_probs must be fp32")
    lens, bonus, trim = verify.verify_sample(
        logits=target_logits, candidates=candidates, width=width, temperatures=_temperatures(sampling_info, bs),
        uniforms=u, final_uniforms=uf, top_ks=ks, top_ps=ps, max_top_k=mk, draft_probs=q,
        cutoff_verify_lens=cutoff_verify_lens, return_cap_trim=True)
    return lens, bonus, trim


class AcceptSampling:
    """accept_sampling.py:25-90 with every implementation selector on the gfx950 path."""

    @classmethod
    def execute_single_q(cls, **kwargs):
        return accept_sampling_single_q(**kwargs)

    @classmethod
    def execute_single_q_torch(cls, **kwargs):
        return accept_sampling_single_q(**kwargs)

    @classmethod
    def execute(cls, *args, **kwargs):
        return cls.hip(*args, **kwargs)

    @classmethod
    def hip(cls, *, candidates, target_logits, draft_probs, sampling_info, draft_input, gamma,
            verify_num_draft_tokens, cutoff_verify_lens=None):
        return accept_sampling(candidates=candidates, target_logits=target_logits, draft_probs=draft_probs,
                               sampling_info=sampling_info, draft_input=draft_input, gamma=gamma,
                               verify_num_draft_tokens=verify_num_draft_tokens, cutoff_verify_lens=cutoff_verify_lens)

    torch = hip
    triton = hip


def chain_speculative_sampling_triton(predicts, accept_index, accept_token_num, candidates, retrive_index,
                                      retrive_next_token, retrive_next_sibling, uniform_samples,
                                      uniform_samples_for_final_sampling, target_probs, draft_probs,
                                      threshold_single, threshold_acc, deterministic):
    """reject_sampling.py:159-204 (chain verification; the tree links, the
    thresholds and ``deterministic`` are unused there too).  Writes
    ``accept_token_num[b]``, ``accept_index[b, :L+1]`` and
    ``predicts[retrive_index[b, :L+1]]`` in place."""
    del retrive_next_token, retrive_next_sibling, threshold_single, threshold_acc, deterministic
    what = "chain_speculative_sampling"
    dev = _lib.require_cuda(predicts, accept_index, accept_token_num, candidates, retrive_index, uniform_samples,
                            uniform_samples_for_final_sampling, target_probs, draft_probs, what=what)
    if candidates.ndim != 2:
        raise ValueError(f"{what}: candidates must be [batch, num_slots]")
    bs, slots = candidates.shape
    if slots < 2:
        raise ValueError(f"{what}: need at least 2 slots")
    vocab = int(target_probs.shape[-1])
    for name, t, rows in (("target_probs", target_probs, slots), ("draft_probs", draft_probs, slots - 1)):
        if t.ndim != 3 or t.shape[0] != bs or t.shape[1] < rows or t.shape[2] != vocab:
            raise ValueError(f"{what}: {name} must be [batch, >= {rows}, vocab]")
        if t.dtype != torch.float32 or t.stride(2) != 1:
            raise ValueError(f"{what}: {name} must be fp32 with unit vocabulary stride")
    if retrive_index.shape[0] != bs or retrive_index.shape[1] < slots:
        raise ValueError(f"{what}: retrive_index must be [batch, num_slots]")
    if accept_index.shape[0] != bs or accept_index.shape[1] < slots or accept_index.dtype != torch.int32:
        raise ValueError(f"{what}: accept_index must be int32 [batch, num_slots]")
    if predicts.dtype != torch.int32 or not predicts.is_contiguous():
        raise ValueError(f"{what}: predicts must be a contiguous int32 tensor")
    if accept_token_num.dtype != torch.int32 or accept_token_num.numel() < bs or \
            not accept_token_num.is_contiguous():
        raise ValueError(f"{what}: accept_token_num must be contiguous int32 [batch]")
    u = uniform_samples
    if u.dtype != torch.float32 or u.shape[0] != bs or u.shape[1] < slots - 1:
        raise ValueError(f"{what}: uniform_samples must be fp32 [batch, >= num_slots-1]")
    if u.stride(1) != 1:
        u = u.contiguous()
    uf = uniform_samples_for_final_sampling.reshape(-1)
    if uf.dtype != torch.float32 or uf.numel() < bs:
        raise ValueError(f"{what}: final uniforms must be fp32 [batch]")
    uf = uf.contiguous()
    for name, t in (("candidates", candidates), ("retrive_index", retrive_index)):
        if t.dtype not in (torch.int32, torch.int64):
            raise ValueError(f"{what}: {name} must be int32 or int64")
    a = _lib.ChainSamplingArgs()
    a.target_probs, a.tp_stride_b, a.tp_stride_k = target_probs.data_ptr(), target_probs.stride(0), \
        target_probs.stride(1)
    a.draft_probs, a.dp_stride_b, a.dp_stride_k = draft_probs.data_ptr(), draft_probs.stride(0), draft_probs.stride(1)
    a.candidates, a.candidates_dtype = candidates.data_ptr(), _lib.dtype_code(candidates)
    a.cand_stride_b, a.cand_stride_k = candidates.stride(0), candidates.stride(1)
    a.retrive_index, a.retrive_index_dtype = retrive_index.data_ptr(), _lib.dtype_code(retrive_index)
    a.ri_stride_b, a.ri_stride_k = retrive_index.stride(0), retrive_index.stride(1)
    a.uniforms, a.uniform_stride_b, a.final_uniforms = u.data_ptr(), u.stride(0), uf.data_ptr()
    a.batch, a.width, a.vocab = bs, slots, vocab
    a.predicts, a.accept_index = predicts.data_ptr(), accept_index.data_ptr()
    a.ai_stride_b, a.ai_stride_k = accept_index.stride(0), accept_index.stride(1)
    a.accept_token_num = accept_token_num.data_ptr()
    cnt, scr = _lib.workspaces.get(*_lib.workspace_sizes("ls_chain_sampling_workspace", bs, vocab), dev)
    _lib.call("ls_chain_speculative_sampling", _lib.ctypes.byref(a), cnt.data_ptr(), cnt.numel(), scr.data_ptr(),
              scr.numel(), _lib.stream_of(dev))


def chain_verify_buffers(*, bs: int, draft_token_num: int, device):
    """The chain layout of SPEC/dflash_utils.py:216-272 (fresh tensors):
    ``(retrieve_index, retrieve_next_token, retrieve_next_sibling, predicts,
    accept_index, accept_token_num)``."""
    retrieve_index = torch.arange(bs * draft_token_num, dtype=torch.int64, device=device).view(bs, draft_token_num)
    row_next = torch.arange(1, draft_token_num + 1, dtype=torch.int64, device=device)
    row_next[-1] = -1
    retrieve_next_token = row_next.unsqueeze(0).expand(bs, -1).clone()
    retrieve_next_sibling = torch.full((bs, draft_token_num), -1, dtype=torch.int64, device=device)
    predicts = torch.empty((bs * draft_token_num,), dtype=torch.int32, device=device)
    accept_index = torch.empty((bs, draft_token_num), dtype=torch.int32, device=device)
    accept_token_num = torch.empty((bs,), dtype=torch.int32, device=device)
    return retrieve_index, retrieve_next_token, retrieve_next_sibling, predicts, accept_index, accept_token_num


def accept_scheduled_greedy_tokens(*, candidates: torch.Tensor, target_logits: torch.Tensor,
                                   verify_num_draft_tokens: int, cutoff_verify_lens: Optional[torch.Tensor] = None):
    """dspark_accept.py:20-49: every scheduled draft is committed
    (``width - 1``, or ``clamp(cutoff - 1, 0, width - 1)``) and the bonus is the
    target argmax at that position."""
    _, _, _, truth = verify.verify_greedy(logits=target_logits, candidates=candidates,
                                          width=verify_num_draft_tokens, return_truth=True)
    bs = candidates.shape[0]
    truth = truth.view(bs, verify_num_draft_tokens)
    if cutoff_verify_lens is None:
        correct_len = torch.full((bs,), verify_num_draft_tokens - 1, dtype=torch.int32, device=truth.device)
    else:
        correct_len = (cutoff_verify_lens.to(torch.int32) - 1).clamp(min=0, max=verify_num_draft_tokens - 1)
    bonus = truth.gather(1, correct_len.to(torch.long)[:, None]).squeeze(1).to(torch.int64)
    return correct_len, bonus, torch.zeros_like(correct_len)


def select_mixed_accept(*, greedy_mask, greedy_len, greedy_bonus, greedy_trim, sampling_len, sampling_bonus,
                        sampling_trim):
    """SPEC/dspark_components/kernels/mixed_accept_select.py:71-89: per request,
    the greedy triple where ``greedy_mask`` is set, else the sampled one."""
    m = greedy_mask.to(torch.bool)
    return (torch.where(m, greedy_len.to(sampling_len.dtype), sampling_len),
            torch.where(m, greedy_bonus, sampling_bonus),
            torch.where(m, greedy_trim.to(sampling_trim.dtype), sampling_trim))


def accept_draft_tokens(*, candidates: torch.Tensor, target_logits: torch.Tensor, draft_block: Any,
                        sampling_info: Any, draft_input: Any, gamma: int, verify_num_draft_tokens: int,
                        cutoff_layout: Any = None, nonstrict_verify: bool = False):
    """dspark_accept.py:52-159: ``(correct_len i32[B], bonus i64[B], cap_trim i32[B])``.

    Greedy batches run the fused greedy verify; sampled batches whose drafter
    kept each token's q and need only temperature run the single-q verify;
    the rest build dense draft probabilities (SoftmaxTemp of the corrected
    logits) and run the chain rule; mixed batches run both and select per
    request.
    """
    greedy_mask = draft_block.greedy_mask
    cutoff = None if cutoff_layout is None else cutoff_layout.verify_lens
    all_greedy = sampling_info is None or sampling_info.is_all_greedy
    if nonstrict_verify:
        if not all_greedy:
            raise ValueError("DSpark nonstrict verify currently supports greedy sampling only.")
        return accept_scheduled_greedy_tokens(candidates=candidates, target_logits=target_logits,
                                              verify_num_draft_tokens=verify_num_draft_tokens,
                                              cutoff_verify_lens=cutoff)
    if all_greedy:
        return verify.AcceptGreedy.execute(candidates=candidates, target_logits=target_logits,
                                       verify_num_draft_tokens=verify_num_draft_tokens, cutoff_verify_lens=cutoff)
    bs, gamma_rows, vocab = draft_block.corrected_logits.shape
    penalizer = getattr(sampling_info, "penalizer_orchestrator", None)
    pure_temperature_scaling = (
        not getattr(sampling_info, "has_custom_logit_processor", False)
        and getattr(sampling_info, "acc_linear_penalties", None) is None
        and not (penalizer is not None and penalizer.is_required)
        and getattr(sampling_info, "vocab_mask", None) is None
        and getattr(sampling_info, "logit_bias", None) is None)

    def dense_q():
        return dense.SoftmaxTemp.execute(logits=draft_block.corrected_logits.reshape(bs * gamma_rows, vocab),
                                         temperatures=draft_block.temperatures,
                                         rows_per_request=gamma_rows).view(bs, gamma_rows, vocab)

    if not sampling_info.is_any_greedy:
        if (draft_block.draft_token_probs is not None and cutoff is None
                and not sampling_info.need_top_k_sampling and not sampling_info.need_top_p_sampling
                and not getattr(sampling_info, "need_min_p_sampling", False) and pure_temperature_scaling):
            return AcceptSampling.execute_single_q(
                candidates=candidates, target_logits=target_logits, corrected_logits=draft_block.corrected_logits,
                draft_token_probs=draft_block.draft_token_probs, draft_temperatures=draft_block.temperatures,
                sampling_info=sampling_info, draft_input=draft_input, gamma=gamma,
                verify_num_draft_tokens=verify_num_draft_tokens)
        return AcceptSampling.execute(candidates=candidates, target_logits=target_logits, draft_probs=dense_q(),
                                      sampling_info=sampling_info, draft_input=draft_input, gamma=gamma,
                                      verify_num_draft_tokens=verify_num_draft_tokens, cutoff_verify_lens=cutoff)
    draft_probs = dense_q()
    g = verify.AcceptGreedy.execute(candidates=candidates, target_logits=target_logits,
                                verify_num_draft_tokens=verify_num_draft_tokens, cutoff_verify_lens=cutoff)
    s = AcceptSampling.execute(candidates=candidates, target_logits=target_logits, draft_probs=draft_probs,
                               sampling_info=sampling_info, draft_input=draft_input, gamma=gamma,
                               verify_num_draft_tokens=verify_num_draft_tokens, cutoff_verify_lens=cutoff)
    return select_mixed_accept(greedy_mask=greedy_mask, greedy_len=g[0], greedy_bonus=g[1], greedy_trim=g[2],
                               sampling_len=s[0], sampling_bonus=s[1], sampling_trim=s[2])
