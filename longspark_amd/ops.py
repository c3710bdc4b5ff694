"""The hot-path entry points as PyTorch custom operators (``torch.ops.longspark_amd.*``).

Each operator runs the same C ABI launch as the Python drop-in it wraps and
has a fake (meta) implementation that gives its outputs' shapes and dtypes
without a GPU, so the operators can appear in ``torch.compile`` graphs,
``torch.export`` programs and fake-tensor shape propagation.  Operators that
update caller-owned tensors declare them mutated; none allocates workspace
of its own beyond what the wrapped drop-in keeps per stream.

Operators (reference call sites as in the drop-ins):
  verify_greedy           -- AcceptGreedy.execute (accept_greedy.py:62-135)
  verify_sample           -- fused stochastic verify (accept_sampling.py:259-567,
                             reject_sampling.py:5-204, sampling.py:19-57 with
                             dflash_utils.py:127-213,743-810 fused in)
  penalty_tables          -- penalty state from output histories (penaltylib/*)
  apply_token_bitmask     -- apply_token_bitmask_inplace_triton (bitmask_ops.py:84-141)
  softmax_temp            -- SoftmaxTemp.execute (softmax_temp.py:17-175)
  kv_window_gather        -- Raw256 window gather through a paged table
  cache_position_scores   -- global16_raw256_incremental.py:400-456
  merge_accepted_positions -- global16_raw256_incremental.py:459-584
  summary_update          -- both of the above for every layer in one launch
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch
from torch import Tensor

from . import dense, kvwindow, penalties, summary, verify

NS = "longspark_amd"


# ----------------------------------------------------------------- verify ---

@torch.library.custom_op(f"{NS}::verify_greedy", mutates_args=())
def verify_greedy(logits: Tensor, candidates: Tensor, width: int, cand_first_col: int = 1,
                  cutoff_verify_lens: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    return verify.verify_greedy(logits=logits, candidates=candidates, width=width, cand_first_col=cand_first_col,
                                cutoff_verify_lens=cutoff_verify_lens)


@verify_greedy.register_fake
def _(logits, candidates, width, cand_first_col=1, cutoff_verify_lens=None):
    b = candidates.shape[0]
    return (logits.new_empty(b, dtype=torch.int32), logits.new_empty(b, dtype=torch.int64),
            logits.new_empty(b, dtype=torch.int32))


@torch.library.custom_op(f"{NS}::penalty_tables", mutates_args=())
def penalty_tables(history: Tensor, vocab: int, frequency: Optional[Tensor] = None,
                   presence: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    t = penalties.build_penalty_tables(history, vocab, frequency=frequency, presence=presence)
    return t.bits, t.rank, t.add, t.distinct, t.nonpositive


@penalty_tables.register_fake
def _(history, vocab, frequency=None, presence=None):
    b, cap = history.shape
    words = (vocab + 31) // 32
    i32 = torch.int32
    return (history.new_empty(b, words, dtype=i32), history.new_empty(b, words, dtype=i32),
            history.new_empty(b, max(cap, 1), dtype=torch.float32), history.new_empty(b, dtype=i32),
            history.new_empty(b, dtype=i32))


@torch.library.custom_op(f"{NS}::verify_sample", mutates_args=())
def verify_sample(logits: Tensor, candidates: Tensor, width: int, temperatures: Tensor, uniforms: Tensor,
                  final_uniforms: Tensor, top_ks: Optional[Tensor] = None, top_ps: Optional[Tensor] = None,
                  min_ps: Optional[Tensor] = None, max_top_k: int = 0, draft_token_probs: Optional[Tensor] = None,
                  draft_logits: Optional[Tensor] = None, draft_probs: Optional[Tensor] = None,
                  draft_temperatures: Optional[Tensor] = None, draft_top_ks: Optional[Tensor] = None,
                  draft_top_ps: Optional[Tensor] = None, draft_min_ps: Optional[Tensor] = None,
                  pen_bits: Optional[Tensor] = None, pen_rank: Optional[Tensor] = None,
                  pen_add: Optional[Tensor] = None, pen_nonpositive: Optional[Tensor] = None,
                  pen_repetition: Optional[Tensor] = None, pen_has_additive: bool = True,
                  pen_verify_quirk: bool = False, vocab_mask: Optional[Tensor] = None,
                  mask_per_request: bool = False, cand_first_col: int = 1, scan_hint: int = 0,
                  cutoff_verify_lens: Optional[Tensor] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """Fused stochastic verify; the penalty state is the tensors of
    ``penalty_tables`` (``pen_*``; all None = no penalties).  Returns
    ``(accept_lens i32[B], bonus i64[B], cap_trim i32[B])``."""
    tables = None
    if pen_bits is not None:
        b = candidates.shape[0]
        tables = penalties.PenaltyTables(
            bits=pen_bits, rank=pen_rank, add=pen_add if pen_add is not None else pen_bits.new_zeros(b, 1,
                                                                                               dtype=torch.float32),
            distinct=pen_bits.new_zeros(b), nonpositive=pen_nonpositive, repetition=pen_repetition,
            verify_quirk=pen_verify_quirk, has_additive=pen_add is not None and pen_has_additive)
    acc, bonus, trim = verify.verify_sample(
        logits=logits, candidates=candidates, width=width, temperatures=temperatures, uniforms=uniforms,
        final_uniforms=final_uniforms, top_ks=top_ks, top_ps=top_ps, min_ps=min_ps,
        max_top_k=max_top_k if max_top_k > 0 else None, draft_token_probs=draft_token_probs,
        draft_logits=draft_logits, draft_probs=draft_probs, draft_temperatures=draft_temperatures,
        draft_top_ks=draft_top_ks, draft_top_ps=draft_top_ps, draft_min_ps=draft_min_ps, penalties=tables,
        vocab_mask=vocab_mask, mask_per_request=mask_per_request, cand_first_col=cand_first_col,
        scan_hint=scan_hint, cutoff_verify_lens=cutoff_verify_lens, return_cap_trim=True)
    return acc, bonus, trim


@verify_sample.register_fake
def _(logits, candidates, width, temperatures, uniforms, final_uniforms, *args, **kwargs):
    b = candidates.shape[0]
    return (logits.new_empty(b, dtype=torch.int32), logits.new_empty(b, dtype=torch.int64),
            logits.new_empty(b, dtype=torch.int32))


@torch.library.custom_op(f"{NS}::apply_token_bitmask", mutates_args=("logits",))
def apply_token_bitmask(logits: Tensor, bitmask: Tensor, indices: Optional[Tensor] = None) -> None:
    penalties.apply_token_bitmask_inplace(logits, bitmask, indices)


@apply_token_bitmask.register_fake
def _(logits, bitmask, indices=None):
    return None


@torch.library.custom_op(f"{NS}::softmax_temp", mutates_args=())
def softmax_temp(logits: Tensor, temperatures: Tensor, rows_per_request: int) -> Tensor:
    return dense.softmax_temp(logits=logits, temperatures=temperatures, rows_per_request=rows_per_request)


@softmax_temp.register_fake
def _(logits, temperatures, rows_per_request):
    return logits.new_empty(logits.shape[0], logits.shape[-1], dtype=torch.float32)


# ---------------------------------------------------------------- refresh ---

@torch.library.custom_op(f"{NS}::kv_window_gather", mutates_args=("out",))
def kv_window_gather(k_layers: List[Tensor], v_layers: List[Tensor], page_table: Tensor, seq_lens: Tensor,
                     page_size: int, window: int, out: Tensor, table_rows: Optional[Tensor] = None) -> None:
    kvwindow.gather_window(k_layers, v_layers, page_table, seq_lens, page_size=page_size, window=window,
                           table_rows=table_rows, out=out)


@kv_window_gather.register_fake
def _(k_layers, v_layers, page_table, seq_lens, page_size, window, out, table_rows=None):
    return None


@torch.library.custom_op(f"{NS}::cache_position_scores", mutates_args=("output",))
def cache_position_scores(global_query: Tensor, new_keys: Tensor, output: Tensor, softmax_scale: float,
                          softcap: float = 0.0) -> None:
    summary.cache_position_scores(layer_id=0, global_query=global_query, new_keys=new_keys, output=output,
                                  softmax_scale=softmax_scale, softcap=softcap)


@cache_position_scores.register_fake
def _(global_query, new_keys, output, softmax_scale, softcap=0.0):
    return None


@torch.library.custom_op(f"{NS}::merge_accepted_positions", mutates_args=("state_output", "state_lse",
                                                                           "accept_offsets"))
def merge_accepted_positions(state_output: Tensor, state_lse: Tensor, position_scores: Tensor, value_cache: Tensor,
                             accepted_cache_locs: Tensor, accept_lens: Tensor, accept_offsets: Optional[Tensor] = None,
                             state_slots: Optional[Tensor] = None) -> None:
    summary.merge_accepted_positions_(state_output=state_output, state_lse=state_lse,
                                      position_scores=position_scores, value_cache=value_cache,
                                      accepted_cache_locs=accepted_cache_locs, accept_lens=accept_lens,
                                      accept_offsets=accept_offsets, state_slots=state_slots)


@merge_accepted_positions.register_fake
def _(state_output, state_lse, position_scores, value_cache, accepted_cache_locs, accept_lens, accept_offsets=None,
      state_slots=None):
    return None


@torch.library.custom_op(f"{NS}::summary_update", mutates_args=("state_output", "state_lse"))
def summary_update(query: Tensor, key_cache: List[Tensor], value_cache: List[Tensor], accepted_cache_locs: Tensor,
                   accept_lens: Tensor, state_output: Tensor, state_lse: Tensor, softmax_scale: float,
                   state_slots: Optional[Tensor] = None, softcap: float = 0.0) -> None:
    summary.summary_update(query=query, key_cache=key_cache, value_cache=value_cache,
                           accepted_cache_locs=accepted_cache_locs, accept_lens=accept_lens,
                           state_output=state_output, state_lse=state_lse, softmax_scale=softmax_scale,
                           state_slots=state_slots, softcap=softcap)


@summary_update.register_fake
def _(query, key_cache, value_cache, accepted_cache_locs, accept_lens, state_output, state_lse, softmax_scale,
      state_slots=None, softcap=0.0):
    return None


OPS = ("verify_greedy", "penalty_tables", "verify_sample", "apply_token_bitmask", "softmax_temp", "kv_window_gather",
       "cache_position_scores", "merge_accepted_positions", "summary_update")
