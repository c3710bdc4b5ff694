"""Install these ops in place of the reference implementations.

The reference swaps implementations by module-attribute replacement at
process start and re-applies it in spawned children
(src/longspark/patches/__init__.py:15-33, src/longspark/patches/gqa5_attention.py:109-112).
``install()`` does the same for the hot-path call sites: every target module
that is importable in this process gets its attributes replaced; modules that
are absent are skipped and reported.  Call it at process start and in the
entry point of every spawned worker, before the first verify step.

``SRT`` = ``sglang.srt``.
"""

from __future__ import annotations

import importlib
from typing import Dict, Iterable, List, Optional, Tuple


def replacements() -> Dict[str, Dict[str, object]]:
    """module name -> {attribute: replacement}, for every hot-path call site."""
    from . import accept, dense, draft_attention, kvwindow, penalties, sample, summary, verify

    return {
        # greedy verify (SPEC/dspark_components/kernels/accept_greedy.py:22-60)
        "sglang.srt.speculative.dspark_components.kernels.accept_greedy": {"AcceptGreedy": verify.AcceptGreedy},
        # stochastic acceptance (SPEC/dspark_components/kernels/accept_sampling.py:25-343) and its
        # bindings of the chain sampler, SoftmaxTemp and the target distribution (:11-19)
        "sglang.srt.speculative.dspark_components.kernels.accept_sampling": {
            "AcceptSampling": accept.AcceptSampling, "accept_sampling": accept.accept_sampling,
            "accept_sampling_single_q": accept.accept_sampling_single_q,
            "chain_speculative_sampling_triton": accept.chain_speculative_sampling_triton,
            "SoftmaxTemp": dense.SoftmaxTemp,
            "build_dflash_verify_target_probs": dense.build_dflash_verify_target_probs},
        # dense-q chain sampling (SPEC/reject_sampling.py:159-204)
        "sglang.srt.speculative.reject_sampling": {
            "chain_speculative_sampling_triton": accept.chain_speculative_sampling_triton},
        # acceptance dispatch (SPEC/dspark_components/dspark_accept.py:20-159) and its bindings (:7-17)
        "sglang.srt.speculative.dspark_components.dspark_accept": {
            "accept_draft_tokens": accept.accept_draft_tokens,
            "accept_scheduled_greedy_tokens": accept.accept_scheduled_greedy_tokens,
            "AcceptGreedy": verify.AcceptGreedy, "AcceptSampling": accept.AcceptSampling,
            "SoftmaxTemp": dense.SoftmaxTemp},
        # dense target distributions (SPEC/dspark_components/kernels/softmax_temp.py:17-175,
        # SPEC/dflash_utils.py:743-810)
        "sglang.srt.speculative.dspark_components.kernels.softmax_temp": {"SoftmaxTemp": dense.SoftmaxTemp},
        "sglang.srt.speculative.dflash_utils": {
            "build_dflash_verify_target_probs": dense.build_dflash_verify_target_probs,
            # in-place verify logit adjustments (SPEC/dflash_utils.py:127-213)
            "apply_dflash_verify_logits_adjustments": penalties.apply_dflash_verify_logits_adjustments},
        # drafter proposal step (SPEC/dspark_components/kernels/sample_step_tokens_with_q.py:40-382;
        # its callers import it at call time)
        "sglang.srt.speculative.dspark_components.kernels.sample_step_tokens_with_q": {
            "sample_step_tokens_with_q": sample.sample_step_tokens_with_q,
            "create_sample_step_workspace": sample.create_sample_step_workspace},
        # split-engine two-phase rejection sampling (src/longspark/engine/sampling.py:19-57)
        "longspark.engine.sampling": {"decide_acceptance": verify.decide_acceptance,
                                      "finish_sampling": verify.finish_sampling},
        # fixed-width verify outputs (SPEC/draft_free_kv_utils.py:386-408,
        # SPEC/draft_free_kv_dispatch.py:32-57)
        "sglang.srt.speculative.draft_free_kv_utils": {
            "build_greedy_verify_out_tokens": verify.build_greedy_verify_out_tokens},
        "sglang.srt.speculative.draft_free_kv_dispatch": {"finalize_verify_outputs": verify.finalize_verify_outputs},
        # committed verify rows into req_to_token (SPEC/draft_free_kv_info.py:32-82)
        "sglang.srt.speculative.draft_free_kv_info": {
            "_assign_fixed_verify_cache_locs_func": verify.assign_fixed_verify_cache_locs},
        # vocabulary bitmask (SRT/constrained/triton_ops/bitmask_ops.py:84-141), and the grammar
        # backend's own bindings: it imports the Triton function, or on ROCm
        # sgl_kernel.apply_token_bitmask_inplace_cuda, by name at import time
        # (SRT/constrained/xgrammar_backend.py:43-48) and calls them at :112-117 and :239-244
        "sglang.srt.constrained.triton_ops.bitmask_ops": {
            "apply_token_bitmask_inplace_triton": penalties.apply_token_bitmask_inplace},
        "sglang.srt.constrained.xgrammar_backend": {
            "apply_token_bitmask_inplace_triton": penalties.apply_token_bitmask_inplace,
            "apply_token_bitmask_inplace_cuda": penalties.apply_token_bitmask_inplace},
        # summary state (SPEC/global16_raw256_incremental.py:400-584; the GQA-5
        # adapter's wrappers are covered by the same functions)
        "sglang.srt.speculative.global16_raw256_incremental": {
            "cache_position_scores": summary.cache_position_scores,
            "merge_accepted_positions_": summary.merge_accepted_positions_},
        # the Qwen3-14B GQA-5 adapter (src/longspark/patches/gqa5_attention.py): its install()
        # (:109-112) rebinds the two functions above to its module-level wrappers and, for other
        # group sizes, those wrappers fall back to the functions it captured at import (:13-14).
        # Replacing all four names makes a later gqa5_attention.install() bind these ops again,
        # whichever of the two installs runs first.
        "longspark.patches.gqa5_attention": {
            "cache_position_scores": summary.cache_position_scores,
            "merge_accepted_positions_": summary.merge_accepted_positions_,
            "_original_scores": summary.cache_position_scores,
            "_original_merge": summary.merge_accepted_positions_},
        # prefill summary initialisation (SPEC/global16_raw256.py:668-784), a method of the
        # verify context class: dotted names replace a class attribute
        "sglang.srt.speculative.global16_raw256": {
            "Global16Raw256VerifyContext.run_prefill_global_attention": summary.run_prefill_global_attention},
        # drafter attention over the three views (SPEC/global16_raw256_draft_all_attention.py:283-416;
        # SPEC/global16_raw256.py:119-128 imports it at call time)
        "sglang.srt.speculative.global16_raw256_draft_all_attention": {
            "fused_global_local_raw_attention": draft_attention.fused_global_local_raw_attention,
            "can_use_fused_global_local_raw_attention": draft_attention.can_use_fused_global_local_raw_attention},
        # recent window (SPEC/global16_raw256_draft_fused.py:372-413, engine/draft.py:14-21)
        "sglang.srt.speculative.global16_raw256_draft_fused": {
            "build_raw256_page_table": kvwindow.build_raw256_page_table,
            # the default drafter path's merge after its window attention (:314-479)
            "fused_global_local_raw_merge": draft_attention.fused_global_local_raw_merge,
            "can_use_fused_global_local_raw_merge": draft_attention.can_use_fused_global_local_raw_merge},
        "longspark.engine.draft": {"ring_page_table": kvwindow.ring_page_table},
        "longspark.engine.state_export": {"gather_selected_kv": _gather_selected_kv_pool},
    }


def _gather_selected_kv_pool(pool, layer_ids, locations, *, tp, rank, group, workspace):
    """Signature of src/longspark/engine/state_export.py:14 (``pool.get_kv_buffer(layer)``
    per layer); one rank only -- a tensor-parallel export keeps the reference path."""
    if tp != 1:
        raise ValueError("gather_selected_kv replacement covers the single-rank export only")
    from . import kvwindow

    if not layer_ids or locations.ndim != 1 or locations.numel() == 0:
        raise ValueError("KV export requires selected layers and nonempty 1D locations")
    keys, values = zip(*(pool.get_kv_buffer(layer) for layer in layer_ids))
    return kvwindow.gather_selected_kv(list(keys), list(values), locations)


def install(modules: Optional[Iterable[str]] = None) -> Tuple[List[str], List[str]]:
    """Replace the attributes of every importable target module.

    Returns (patched module names, skipped module names).  ``modules`` limits
    the install to the given names.
    """
    table = replacements()
    names = list(table) if modules is None else list(modules)
    patched, skipped = [], []
    for name in names:
        try:
            mod = importlib.import_module(name)
        except ImportError:
            skipped.append(name)
            continue
        for attr, fn in table[name].items():
            owner, *path = [mod, *attr.split(".")]
            for part in path[:-1]:
                owner = getattr(owner, part)
            setattr(owner, path[-1], fn)
        patched.append(name)
    return patched, skipped
