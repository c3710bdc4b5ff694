"""The installer replaces the reference call sites by module attribute, as the
reference's own patches do (src/longspark/patches/__init__.py:15-33)."""

import sys
import types

from longspark_amd import accept, patches, summary, kvwindow, verify


def test_install_replaces_attributes_of_importable_modules(monkeypatch):
    names = ["sglang.srt.speculative.global16_raw256_incremental", "longspark.engine.draft",
             "longspark.engine.sampling", "sglang.srt.speculative.reject_sampling",
             "sglang.srt.speculative.dspark_components.dspark_accept"]
    for n in names:
        parts = n.split(".")
        for i in range(1, len(parts) + 1):
            mod = ".".join(parts[:i])
            if mod not in sys.modules:
                monkeypatch.setitem(sys.modules, mod, types.ModuleType(mod))
    patched, skipped = patches.install(names + ["not.a.module"])
    assert patched == names and skipped == ["not.a.module"]
    inc = sys.modules[names[0]]
    assert inc.cache_position_scores is summary.cache_position_scores
    assert inc.merge_accepted_positions_ is summary.merge_accepted_positions_
    assert sys.modules[names[1]].ring_page_table is kvwindow.ring_page_table
    assert sys.modules[names[2]].decide_acceptance is verify.decide_acceptance
    assert sys.modules[names[3]].chain_speculative_sampling_triton is accept.chain_speculative_sampling_triton
    assert sys.modules[names[4]].accept_draft_tokens is accept.accept_draft_tokens
    assert sys.modules[names[4]].AcceptSampling is accept.AcceptSampling


def test_every_replacement_target_is_listed_once():
    table = patches.replacements()
    assert len(table) >= 8
    for mod, attrs in table.items():
        assert attrs and all(callable(f) for f in attrs.values()), mod


def test_install_replaces_a_class_method(monkeypatch):
    name = "sglang.srt.speculative.global16_raw256"
    parts = name.split(".")
    for i in range(1, len(parts) + 1):
        mod = ".".join(parts[:i])
        if mod not in sys.modules:
            monkeypatch.setitem(sys.modules, mod, types.ModuleType(mod))

    class Global16Raw256VerifyContext:
        def run_prefill_global_attention(self, **kw):
            raise AssertionError("reference body still installed")

    monkeypatch.setattr(sys.modules[name], "Global16Raw256VerifyContext", Global16Raw256VerifyContext,
                        raising=False)
    patched, _ = patches.install([name])
    assert patched == [name]
    assert Global16Raw256VerifyContext.run_prefill_global_attention is summary.run_prefill_global_attention


def _fake_modules(monkeypatch, names):
    for n in names:
        parts = n.split(".")
        for i in range(1, len(parts) + 1):
            mod = ".".join(parts[:i])
            if mod not in sys.modules:
                monkeypatch.setitem(sys.modules, mod, types.ModuleType(mod))


# A stand-in with the structure of src/longspark/patches/gqa5_attention.py:
# it captures the incremental module's functions at import (:11-14), defines
# its own wrappers, and its install() (:109-112) rebinds the incremental
# module's attributes to those wrappers, looked up in its globals at call time.
_GQA5_STANDIN = '''
from sglang.srt.speculative import global16_raw256_incremental as original
_original_scores = original.cache_position_scores
_original_merge = original.merge_accepted_positions_
def cache_position_scores(**kw):
    raise AssertionError("GQA-5 Triton wrapper reached")
def merge_accepted_positions_(**kw):
    raise AssertionError("GQA-5 Triton wrapper reached")
def install():
    original.cache_position_scores = cache_position_scores
    original.merge_accepted_positions_ = merge_accepted_positions_
'''


def test_install_survives_the_gqa5_adapter_install(monkeypatch):
    inc_name = "sglang.srt.speculative.global16_raw256_incremental"
    gq_name = "longspark.patches.gqa5_attention"
    _fake_modules(monkeypatch, [inc_name, "longspark.patches"])
    inc = sys.modules[inc_name]
    inc.cache_position_scores = lambda **kw: "reference scores"
    inc.merge_accepted_positions_ = lambda **kw: "reference merge"
    gq = types.ModuleType(gq_name)
    monkeypatch.setitem(sys.modules, gq_name, gq)
    exec(_GQA5_STANDIN, gq.__dict__)
    # the documented order: this package's install first, then the reference's
    # apply_runtime_patches() runs gqa5_attention.install() (patches/__init__.py:15-19)
    patched, _ = patches.install([inc_name, gq_name])
    assert patched == [inc_name, gq_name]
    gq.install()
    assert inc.cache_position_scores is summary.cache_position_scores
    assert inc.merge_accepted_positions_ is summary.merge_accepted_positions_
    assert gq._original_scores is summary.cache_position_scores
    assert gq._original_merge is summary.merge_accepted_positions_
    # and the other order gives the same binding
    gq.install()
    patches.install([inc_name, gq_name])
    assert inc.cache_position_scores is summary.cache_position_scores


def test_install_binds_the_grammar_backend_bitmask(monkeypatch):
    from longspark_amd import penalties
    name = "sglang.srt.constrained.xgrammar_backend"
    _fake_modules(monkeypatch, [name])
    patched, _ = patches.install([name])
    mod = sys.modules[name]
    assert patched == [name]
    assert mod.apply_token_bitmask_inplace_cuda is penalties.apply_token_bitmask_inplace
    assert mod.apply_token_bitmask_inplace_triton is penalties.apply_token_bitmask_inplace
