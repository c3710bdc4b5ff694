"""CPU oracle for the verify half of the hot path (test infrastructure only).

Restates, in torch fp32 on the CPU, the reference's greedy verification,
rejection-sampling acceptance, residual resampling, target-distribution build
(temperature, top-k, top-p, min-p), penalties and vocabulary bitmask.  Paths
below are relative to the reference root; ``SRT`` abbreviates
``vendor/sglang/python/sglang/srt`` and ``SPEC`` abbreviates ``SRT/speculative``.

Tie rules adopted where the reference leaves them to a closed binary or to an
unstable sort (parity against sgl-kernel / flashinfer is unpinned; these
rules are pinned by brute force in tests/test_oracle_greedy.py and
tests/test_oracle_sampling.py):
  * argmax: first maximal index (documented torch.argmax behaviour).
  * top-k: the k largest scaled logits, ties at the k-th value broken towards
    the lowest vocabulary index (the order CUDA torch.topk gathers ties in).
  * top-p / min-p sorting: descending probability, ties by ascending index
    (a stable descending sort).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

# SPEC/dspark_components/kernels/accept_sampling.py:22
RESIDUAL_MASS_EPS = 1e-8


# --------------------------------------------------------------------------
# greedy verification
# --------------------------------------------------------------------------

def greedy_truth(target_logits: torch.Tensor) -> torch.Tensor:
    """Row argmax, first maximal index.

    SPEC/dspark_components/kernels/accept_greedy.py:70 (``torch.argmax``).
    """
    return torch.argmax(target_logits.float(), dim=-1)


def compute_correct_drafts_and_bonus(candidates: torch.Tensor, target_predict: torch.Tensor):
    """Accept length and bonus for the ``[B, K]`` layout (``cand[:, 0]`` = current token).

    SPEC/dflash_utils.py:564-602 and SPEC/draft_free_kv_utils.py:360-383:
    ``matches = cand[:, 1:] == predict[:, :-1]``; ``L = cumprod(matches).sum``;
    ``bonus = predict[b, L]``.
    """
    matches = candidates[:, 1:] == target_predict[:, :-1]
    correct_len = matches.to(torch.int32).cumprod(dim=1).sum(dim=1).to(torch.int32)
    rows = torch.arange(candidates.shape[0])
    bonus = target_predict[rows, correct_len.long()].to(torch.int64)
    return correct_len, bonus


def accept_greedy(candidates: torch.Tensor, target_logits: torch.Tensor, verify_num_draft_tokens: int):
    """SPEC/dspark_components/kernels/accept_greedy.py:62-84 (no cutoff layout)."""
    bs = candidates.shape[0]
    predict = greedy_truth(target_logits).view(bs, verify_num_draft_tokens)
    correct_len, bonus = compute_correct_drafts_and_bonus(candidates, predict)
    return correct_len, bonus, torch.zeros_like(correct_len)


def greedy_verify_split(drafted: torch.Tensor, logits: torch.Tensor):
    """Split-engine greedy verify: src/longspark/engine/target.py:474-477.

    ``drafted`` is ``[B, gamma]`` (drafted tokens only) and ``logits`` is
    ``[B, gamma + 1, V]``.  Returns ``(accept, bonus)`` as int64.
    """
    gamma = drafted.shape[1]
    truth = logits.float().argmax(-1)
    accept = (truth[:, :gamma] == drafted).long().cumprod(1).sum(1)
    bonus = truth[torch.arange(drafted.shape[0]), accept]
    return accept, bonus


# --------------------------------------------------------------------------
# split-engine two-phase rejection sampling
# --------------------------------------------------------------------------

@dataclass
class AcceptanceDecision:
    """src/longspark/engine/sampling.py:11-16."""
    lengths: torch.Tensor
    rejected_rows: torch.Tensor
    rejection_positions: torch.Tensor
    target_rows: torch.Tensor


def decide_acceptance(*, candidates, sampled_q, target_probs, uniforms) -> AcceptanceDecision:
    """src/longspark/engine/sampling.py:19-35 restated."""
    batch, gamma = candidates.shape
    selected_p = target_probs[:, :gamma].gather(2, candidates[..., None]).squeeze(-1)
    accept = uniforms * sampled_q < selected_p
    lengths = accept.to(torch.int64).cumprod(1).sum(1)
    rows = torch.arange(batch)
    rejected_rows = rows[lengths < gamma]
    return AcceptanceDecision(
        lengths=lengths,
        rejected_rows=rejected_rows,
        rejection_positions=lengths[rejected_rows],
        target_rows=target_probs[rows, lengths],
    )


def finish_sampling(decision: AcceptanceDecision, rejected_q_rows, uniforms):
    """src/longspark/engine/sampling.py:38-57 restated (host-supplied uniforms)."""
    target = decision.target_rows
    probs = target.clone()
    if decision.rejected_rows.numel():
        residual = (target[decision.rejected_rows] - rejected_q_rows).clamp_min(0)
        mass = residual.sum(-1, keepdim=True)
        probs[decision.rejected_rows] = torch.where(
            mass > 1e-8, residual / mass.clamp_min(1e-30), target[decision.rejected_rows])
    return (uniforms[:, None] >= probs.cumsum(-1)).sum(-1).clamp_max(probs.shape[-1] - 1)


def finalize_verify_outputs(candidates, accept_lens, bonus, prefix_lens):
    """SPEC/draft_free_kv_dispatch.py:8-57 restated: ``out[b, c]`` is the bonus at
    ``c == L_b``, else ``candidates[b, c+1]`` (0 in the last column);
    ``committed = L + 1``; ``next = prefix + L + 1``."""
    batch, width = candidates.shape
    out = torch.zeros(batch, width, dtype=torch.int64)
    out[:, :-1] = candidates[:, 1:].to(torch.int64)
    out[torch.arange(batch), accept_lens.long()] = bonus.to(torch.int64)
    committed = (accept_lens.to(torch.int64) + 1).to(torch.int32)
    next_lengths = (prefix_lens.to(torch.int64) + accept_lens.to(torch.int64) + 1).to(prefix_lens.dtype)
    return out, committed, next_lengths


# --------------------------------------------------------------------------
# temperature softmax and inverse-CDF sampling
# --------------------------------------------------------------------------

def softmax_temp(logits: torch.Tensor, temperatures: torch.Tensor, rows_per_request: int):
    """SPEC/dspark_components/kernels/softmax_temp.py:69-84 restated."""
    num_rows = logits.shape[0]
    bs = num_rows // rows_per_request
    temp_per_row = torch.repeat_interleave(temperatures.reshape(bs).float(), rows_per_request, dim=0)
    return torch.softmax(logits.float() / temp_per_row[:, None], dim=-1)


def sample_rows_from_probs(probs: torch.Tensor, uniforms: torch.Tensor) -> torch.Tensor:
    """First index whose running sum exceeds ``u * total``; V-1 if none.

    SPEC/dspark_components/kernels/accept_sampling.py:190-206.
    """
    cdf = probs.cumsum(dim=-1)
    row_sums = cdf[:, -1]
    matches = cdf > uniforms[:, None] * row_sums[:, None]
    sampled = matches.to(torch.int32).argmax(dim=-1)
    return torch.where(matches.any(dim=-1) & (row_sums > 0), sampled,
                       torch.full_like(sampled, probs.shape[-1] - 1)).to(torch.int64)


# --------------------------------------------------------------------------
# penalties and vocabulary bitmask
# --------------------------------------------------------------------------

def penalty_tables(history, vocab: int, repetition, presence, frequency):
    """Per-request accumulated penalty tensors, as the penalizers build them.

    ``history[b]`` is request b's output-token history (1-D int tensor).
    Returns ``(additive [B, V], scaling [B, V])`` in fp32:
      * frequency: ``scatter_add_`` of the per-request value once per
        occurrence (SRT/sampling/penaltylib/frequency_penalty.py:35-43), so a
        token seen c times carries the fp32 sum of c copies;
      * presence: ``scatter_`` of the value (presence_penalty.py:35-43);
      * additive = ``(0 - freq_cum) - pres_cum``
        (SRT/sampling/penaltylib/orchestrator.py:87-91);
      * scaling: repetition value where present, 1 elsewhere
        (repetition_penalty.py:31-53).
    """
    bs = len(history)
    freq_cum = torch.zeros(bs, vocab, dtype=torch.float32)
    pres_cum = torch.zeros(bs, vocab, dtype=torch.float32)
    scaling = torch.ones(bs, vocab, dtype=torch.float32)
    for b, ids in enumerate(history):
        ids = torch.as_tensor(ids, dtype=torch.int64).reshape(-1)
        if ids.numel() == 0:
            continue
        f = torch.full((ids.numel(),), float(frequency[b]), dtype=torch.float32)
        # scatter_add_ of identical values: the fp32 partial sums do not depend on order.
        freq_cum[b].scatter_add_(0, ids, f)
        pres_cum[b].scatter_(0, ids, torch.full((ids.numel(),), float(presence[b]), dtype=torch.float32))
        scaling[b].scatter_(0, ids, torch.full((ids.numel(),), float(repetition[b]), dtype=torch.float32))
    additive = torch.zeros(bs, vocab, dtype=torch.float32)
    additive.sub_(freq_cum)
    additive.sub_(pres_cum)
    return additive, scaling


def apply_scaling_penalties(logits: torch.Tensor, scaling: torch.Tensor) -> None:
    """SRT/sampling/penaltylib/repetition_penalty.py:10-15: ``l<0 ? l*r : l/r``."""
    logits[:] = torch.where(logits < 0, logits * scaling, logits / scaling)


def apply_token_bitmask(logits: torch.Tensor, bitmask: torch.Tensor) -> None:
    """In place: bit ``(mask[row, v>>5] >> (v & 31)) & 1 == 0`` sets ``-inf``.

    SRT/constrained/triton_ops/bitmask_ops.py:60-81 (LSB first within a word).
    Only the first ``min(V, 32 * words)`` columns are touched (:110).
    """
    rows, vocab = logits.shape
    width = min(vocab, bitmask.shape[1] * 32)
    v = torch.arange(width)
    words = bitmask.to(torch.int64)[:, v >> 5] & 0xFFFFFFFF
    bits = (words >> (v & 31)) & 1
    logits[:, :width] = torch.where(bits == 0, torch.tensor(float("-inf")), logits[:, :width])


def apply_verify_adjustments(logits, *, additive=None, scaling=None, bitmask=None,
                             rows_per_request: int, verify_quirk: bool = False) -> None:
    """Apply penalties and the bitmask to ``[B*K, V]`` fp32 logits in place.

    True semantics (``verify_quirk=False``): the overlap-mode order of
    ``apply_logits_bias`` (SRT/sampling/sampling_batch_info.py:269-286) on the
    real logits, as the EAGLE verify path does
    (SPEC/eagle_utils.py:436-456): add the additive penalties, then the
    multiplicative repetition scaling, then the bitmask.

    Verify-path quirk (``verify_quirk=True``): SPEC/dflash_utils.py:176-191
    builds the bias on a zero tensor -- ``pen = 0 + additive``, then the
    scaling acts on ``pen`` (so repetition multiplies the negative additive
    penalty of present tokens and is otherwise a no-op), then the bitmask sets
    ``-inf`` in ``pen`` -- and finally adds ``pen`` to every row of the block.
    """
    bs = logits.shape[0] // rows_per_request
    view = logits.view(bs, rows_per_request, -1)
    if verify_quirk:
        pen = torch.zeros(bs, logits.shape[1], dtype=torch.float32)
        if additive is not None:
            pen.add_(additive)
        if scaling is not None:
            apply_scaling_penalties(pen, scaling)
        per_request_mask = bitmask is not None and bitmask.shape[0] == bs and rows_per_request > 1
        if per_request_mask:
            apply_token_bitmask(pen, bitmask)
        view.add_(pen[:, None, :])
        if bitmask is not None and not per_request_mask:
            # The reference's verify path carries one mask row per request; a
            # per-row mask sets -inf row by row, which adding -inf would do.
            apply_token_bitmask(logits, bitmask)
        return
    if additive is not None:
        view.add_(additive[:, None, :])
    if scaling is not None:
        apply_scaling_penalties(logits, torch.repeat_interleave(scaling, rows_per_request, dim=0))
    if bitmask is not None:
        # A per-request mask ([B, W]) is expanded over the block; a per-row
        # mask ([B*K, W]) is applied row by row.
        if bitmask.shape[0] == bs and rows_per_request > 1:
            bitmask = torch.repeat_interleave(bitmask, rows_per_request, dim=0)
        apply_token_bitmask(logits, bitmask)


# --------------------------------------------------------------------------
# target distribution (temperature, top-k, top-p, min-p)
# --------------------------------------------------------------------------

def stable_topk(x: torch.Tensor, k: int):
    """Top-k along the last dim with ties at the k-th value kept lowest-index first.

    Returns (values, indices) ordered by value descending, index ascending.
    Uses ``torch.topk`` only to find the k-th value; membership and order are
    exact.
    """
    rows, vocab = x.shape
    kth = torch.topk(x, k, dim=-1).values[:, -1:]
    greater = x > kth
    equal = x == kth
    need = k - greater.sum(-1, keepdim=True)
    keep = greater | (equal & (equal.cumsum(-1) <= need))
    idx = torch.nonzero(keep)[:, 1].view(rows, k)
    vals = x.gather(1, idx)
    # Order by value descending, then index ascending (stable sort on values).
    order = torch.sort(vals, dim=-1, descending=True, stable=True).indices
    return vals.gather(1, order), idx.gather(1, order)


def top_p_renorm(probs_sorted: torch.Tensor, top_p: torch.Tensor) -> torch.Tensor:
    """Top-p on rows already sorted descending (ties by index); renormalised.

    SRT/layers/sampler.py:666-675 (``top_p_normalize_probs_torch``): drop an
    entry when ``cumsum - p > top_p``; divide by the kept sum.
    """
    cum = torch.cumsum(probs_sorted, dim=-1)
    out = probs_sorted.clone()
    out[(cum - probs_sorted) > top_p.view(-1, 1)] = 0.0
    return out / out.sum(dim=-1, keepdim=True)


def min_p_renorm(probs: torch.Tensor, min_p: torch.Tensor) -> torch.Tensor:
    """Drop ``p < p_max * min_p`` and renormalise (SRT/layers/sampler.py:238-242, 504-510)."""
    thr = probs.max(dim=-1, keepdim=True).values * min_p.view(-1, 1)
    out = torch.where(probs < thr, torch.zeros_like(probs), probs)
    return out / out.sum(dim=-1, keepdim=True)


def target_probs(logits: torch.Tensor, *, temperatures, top_ks, top_ps, min_ps,
                 rows_per_request: int, compute_dtype=torch.float32) -> torch.Tensor:
    """Dense ``[B*K, V]`` fp32 target distribution of adjusted logits.

    SPEC/dflash_utils.py:743-810 (``build_dflash_verify_target_probs``):
    ``scaled = logits / T``; if any request's top-k is below V, the sparse
    exact top-k-first path: top-k (tie rule above) with per-row masking of
    ranks >= k_row, softmax over the kept logits, top-p renorm, scatter to
    dense zeros; otherwise dense softmax and top-p renorm.  Min-p (absent from
    the reference verify path) follows the sampler order: after top-k/top-p,
    ``SRT/layers/sampler.py:238-242``.
    Per-request parameters are ``[B]`` tensors; ``top_k >= V`` disables top-k,
    ``top_p >= 1`` disables top-p and ``min_p <= 0`` disables min-p.
    ``compute_dtype``: precision of everything after ``scaled`` (which is
    always the fp32 quotient the reference computes); float64 gives the exact
    value of the formula, free of fp32 summation order.  Returned as float32.
    """
    rows, vocab = logits.shape
    k = rows_per_request
    temp = torch.repeat_interleave(temperatures.float().reshape(-1), k)
    scaled = (logits.float() / temp[:, None]).to(compute_dtype)
    top_k_rows = torch.repeat_interleave(top_ks.to(torch.int64).reshape(-1), k).clamp(1, vocab)
    top_p_rows = torch.repeat_interleave(top_ps.float().reshape(-1), k)
    min_p_rows = torch.repeat_interleave(min_ps.float().reshape(-1), k)
    need_top_p = bool((top_p_rows < 1.0).any())
    max_k = int(top_k_rows.max())
    if max_k < vocab:
        vals, idx = stable_topk(scaled, max_k)
        ranks = torch.arange(max_k)[None, :]
        vals = vals.masked_fill(ranks >= top_k_rows[:, None], float("-inf"))
        probs_k = torch.softmax(vals, dim=-1)
        if need_top_p:
            probs_k = top_p_renorm(probs_k, top_p_rows.to(compute_dtype))
        dense = torch.zeros(rows, vocab, dtype=compute_dtype)
        dense.scatter_(1, idx, probs_k)
    else:
        dense = torch.softmax(scaled, dim=-1)
        if need_top_p:
            sorted_p, order = torch.sort(dense, dim=-1, descending=True, stable=True)
            dense = torch.zeros_like(dense).scatter_(1, order, top_p_renorm(sorted_p, top_p_rows.to(compute_dtype)))
    if bool((min_p_rows > 0).any()):
        dense = min_p_renorm(dense, min_p_rows.to(compute_dtype))
    return dense.float()


# --------------------------------------------------------------------------
# single-q acceptance with residual resampling (the fused-verify semantics)
# --------------------------------------------------------------------------

def accept_single_q(*, candidates, target_probs_3d, draft_q_rows_fn, draft_token_probs,
                    uniforms, final_uniforms):
    """SPEC/dspark_components/kernels/accept_sampling.py:259-343 restated.

    ``target_probs_3d`` is ``[B, K, V]``; ``candidates`` ``[B, K]`` with
    ``cand[:, 0]`` the current token; ``draft_q_rows_fn(positions)`` returns
    the ``[B, V]`` draft distribution at each request's rejection position
    (the reference rebuilds it as ``softmax(corrected[b, pos] / T_draft)``).
    Returns ``(correct_len i32[B], bonus i64[B])``.
    """
    bs, width = candidates.shape
    gamma = width - 1
    drafted = candidates[:, 1:].long()
    p_cand = target_probs_3d[:, :gamma].gather(2, drafted[:, :, None]).squeeze(-1)
    accepted = uniforms * draft_token_probs < p_cand
    correct_len = torch.cumprod(accepted.to(torch.int32), dim=1).sum(dim=1).to(torch.int32)
    rejected = correct_len < gamma
    rows = torch.arange(bs)
    q_positions = correct_len.clamp(max=gamma - 1).long()
    q = draft_q_rows_fn(q_positions)
    selected = target_probs_3d[rows, correct_len.long(), :]
    residual = (selected - q).clamp_min(0.0)
    mass = residual.sum(dim=-1)
    use_residual = rejected & (mass > RESIDUAL_MASS_EPS)
    probs = torch.where(use_residual[:, None], residual, selected)
    return correct_len, sample_rows_from_probs(probs, final_uniforms)


def draft_q_rows(corrected_logits, positions, *, temperatures, top_ks=None, top_ps=None, min_ps=None):
    """Draft distribution at ``corrected_logits[b, positions[b]]``.

    With only temperatures this is the reference reconstruction
    ``softmax(q_logits / T_draft)`` (accept_sampling.py:322-331).  With
    top-k/top-p/min-p it applies the same transform as the target side, which
    is what a drafter that samples under those parameters drew from.
    """
    bs, _, vocab = corrected_logits.shape
    rows = corrected_logits[torch.arange(bs), positions.long(), :].float()
    if top_ks is None:
        return torch.softmax(rows / temperatures.float().reshape(-1)[:, None], dim=-1)
    return target_probs(rows, temperatures=temperatures, top_ks=top_ks, top_ps=top_ps,
                        min_ps=min_ps, rows_per_request=1)


# --------------------------------------------------------------------------
# dense-q chain rejection sampling
# --------------------------------------------------------------------------

def chain_speculative_sampling(*, candidates, uniform_samples, uniform_final, target_probs_3d,
                               draft_probs_3d):
    """SPEC/reject_sampling.py:5-156 restated for the chain layout.

    ``retrive_index = arange(B*K).view(B, K)`` (SPEC/dflash_utils.py:229-231).
    Returns ``(predicts i32[B*K], accept_index i32[B, K], accept_token_num i32[B])``;
    slots the kernel never writes are returned as -1 (the reference leaves
    them uninitialised).
    """
    bs, num_slots = candidates.shape
    vocab = target_probs_3d.shape[-1]
    predicts = torch.full((bs * num_slots,), -1, dtype=torch.int32)
    accept_index = torch.full((bs, num_slots), -1, dtype=torch.int32)
    accept_num = torch.zeros(bs, dtype=torch.int32)
    for b in range(bs):
        cur_row = 0
        last = b * num_slots
        accept_index[b, 0] = last
        n = 0
        step = 1
        all_accepted = True
        while step < num_slots:
            tok = int(candidates[b, step])
            p = target_probs_3d[b, cur_row, tok]
            q = draft_probs_3d[b, cur_row, tok]
            coin = uniform_samples[b, step - 1]
            if coin * q < p:
                n += 1
                cur_row = step
                predicts[last] = tok
                last = b * num_slots + step
                accept_index[b, n] = last
                step += 1
            else:
                all_accepted = False
                break
        accept_num[b] = n
        p_row = target_probs_3d[b, cur_row].float()
        if all_accepted:
            val = p_row
        else:
            diff = p_row - draft_probs_3d[b, cur_row].float()
            val = torch.where(diff > 0, diff, torch.zeros_like(diff))
        norm = val.sum()
        cdf = torch.cumsum(val, 0)
        hit = torch.nonzero(cdf > uniform_final[b] * norm)
        predicts[last] = int(hit[0]) if hit.numel() else vocab - 1
    return predicts, accept_index, accept_num


# --------------------------------------------------------------------------
# fused stochastic verify (composition of a2..a8 with the single-q rule)
# --------------------------------------------------------------------------

def verify_sample(*, logits, candidates, draft_logits, draft_token_probs, uniforms, final_uniforms,
                  temperatures, top_ks, top_ps, min_ps, additive=None, scaling=None, bitmask=None,
                  verify_quirk=False, draft_temperatures=None, draft_top_ks=None, draft_top_ps=None,
                  draft_min_ps=None):
    """The whole stochastic verify for one round, composed from the functions above.

    ``logits`` ``[B*K, V]`` (bf16 or fp32; converted to fp32 as
    SRT/layers/logits_processor.py:993-1003 does), ``candidates`` ``[B, K]``,
    ``draft_logits`` ``[B, K-1, V]``.  Order: adjustments
    (apply_verify_adjustments) -> target distribution (target_probs) ->
    single-q acceptance with residual resampling (accept_single_q).  Returns
    ``(correct_len i32[B], bonus i64[B], target_probs [B, K, V])``.
    """
    bs, width = candidates.shape
    x = logits.float().clone()
    apply_verify_adjustments(x, additive=additive, scaling=scaling, bitmask=bitmask,
                             rows_per_request=width, verify_quirk=verify_quirk)
    probs = target_probs(x, temperatures=temperatures, top_ks=top_ks, top_ps=top_ps, min_ps=min_ps,
                         rows_per_request=width).view(bs, width, -1)
    dt = temperatures if draft_temperatures is None else draft_temperatures

    def q_fn(pos):
        return draft_q_rows(draft_logits, pos, temperatures=dt, top_ks=draft_top_ks,
                            top_ps=draft_top_ps, min_ps=draft_min_ps)

    correct_len, bonus = accept_single_q(candidates=candidates, target_probs_3d=probs,
                                         draft_q_rows_fn=q_fn, draft_token_probs=draft_token_probs,
                                         uniforms=uniforms, final_uniforms=final_uniforms)
    return correct_len, bonus, probs


def out_tokens(candidates, accept_lens, bonus):
    """Fixed-width committed tokens: SPEC/draft_free_kv_utils.py:386-408 and
    SPEC/draft_free_kv_dispatch.py:8-57: ``out[b, :K-1] = cand[b, 1:]``,
    ``out[b, K-1] = 0``, then ``out[b, L] = bonus``."""
    bs, width = candidates.shape
    out = torch.zeros(bs, width, dtype=torch.int64)
    out[:, :-1] = candidates[:, 1:].long()
    out.scatter_(1, accept_lens.long()[:, None], bonus.long()[:, None])
    return out


# --------------------------------------------------------------------------
# drafter proposal step: exponential race with the sampled q
# --------------------------------------------------------------------------

def sample_step_tokens_with_q(step_logits, temperatures, exp_noise, *, compute_dtype=torch.float32):
    """SPEC/dspark_components/kernels/sample_step_tokens_with_q.py:72-187 over whole rows.

    The reference reduces 1024-element tiles and rescales each tile by
    exp(m_t - m); over a whole row that is ``p = softmax(s)`` with
    ``s = l / T`` for finite ``l`` (-inf otherwise), key ``p / E`` (-1 where
    the noise is not in (0, inf)), token = first index of the largest key,
    q = p at the token.  Invalid rows (:97-106, :170-176) give token 0 and
    q = NaN.  Returns ``(tokens i64[N], q f32[N], valid bool[N])``.
    """
    x = step_logits.float()
    t = temperatures.float().reshape(-1, 1)
    noise = exp_noise.to(compute_dtype)
    finite = torch.isfinite(x)
    scaled = torch.where(finite, x / t, torch.full_like(x, float("-inf")))
    logits_valid = ~torch.isnan(x) & (x != float("inf"))
    scaled_valid = ~torch.isnan(scaled) & (scaled != float("inf"))
    noise_valid = (noise > 0) & torch.isfinite(noise)
    lane_valid = logits_valid & scaled_valid & torch.where(torch.isfinite(scaled), noise_valid,
                                                           torch.ones_like(noise_valid))
    temp_valid = (t.reshape(-1) > 0) & torch.isfinite(t.reshape(-1))
    s = scaled.to(compute_dtype)
    m = s.max(dim=-1).values
    m_fin = torch.isfinite(m)
    safe = torch.where(m_fin, m, torch.zeros_like(m))
    e = torch.where(finite & m_fin[:, None], torch.exp(s - safe[:, None]), torch.zeros_like(s))
    z = e.sum(dim=-1)
    keys = torch.where(m_fin[:, None] & noise_valid, e / noise, torch.full_like(e, -1.0))
    best = keys.max(dim=-1).values
    idx = torch.argmax((keys == best[:, None]).to(torch.int8), dim=-1)  # first index of the maximum
    q = e.gather(1, idx[:, None]).squeeze(1) / z
    valid = temp_valid & lane_valid.all(dim=-1) & m_fin & torch.isfinite(z) & (z > 0)
    tokens = torch.where(valid, idx, torch.zeros_like(idx)).to(torch.int64)
    q = torch.where(valid, q, torch.full_like(q, float("nan"))).float()
    return tokens, q, valid



def assign_fixed_verify_cache_locs(req_pool_indices, req_to_token, start_offset, commit_lens, verify_cache_locs):
    """SPEC/draft_free_kv_info.py:32-59 restated: a copy of ``req_to_token``
    with ``[slot_b, start_b + i] = verify_cache_locs[b, i]`` for
    ``i < commit_lens[b]``.  A commit length above the verify width is clamped
    to it and positions outside the map are skipped (the reference leaves
    both to the caller's contract)."""
    out = req_to_token.clone()
    width = verify_cache_locs.shape[1]
    for b in range(req_pool_indices.numel()):
        n = min(max(int(commit_lens[b]), 0), width)
        for i in range(n):
            pos = int(start_offset[b]) + i
            if 0 <= pos < out.shape[1]:
                out[int(req_pool_indices[b]), pos] = int(verify_cache_locs[b, i])
    return out
