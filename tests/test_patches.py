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
