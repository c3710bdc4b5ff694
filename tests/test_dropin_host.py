"""Host-side logic of the drop-ins (no GPU): configuration parsing and the
pointer-array cache's lifetime rules."""

import gc

import pytest
import torch

from longspark_amd import draft_attention, kvwindow


def test_draft_attention_block_from_environment(monkeypatch):
    env = "DFK_GLOBAL16_DRAFT_ATTENTION_CONFIGS"
    monkeypatch.delenv(env, raising=False)
    assert draft_attention._configured_raw_block(128) == 64
    monkeypatch.setenv(env, '{"128": [128, 8, 2], "default": [32, 4, 1]}')
    assert draft_attention._configured_raw_block(128) == 128
    assert draft_attention._configured_raw_block(7) == 32
    monkeypatch.setenv(env, '{"128": [64, 8, 3]}')
    assert draft_attention._configured_raw_block(128) == 64
    for bad, msg in (('[1, 2]', "JSON object"), ('{"0": [64, 4, 2]}', "positive integers"),
                     ('{"default": [48, 4, 2]}', "Unsupported")):
        monkeypatch.setenv(env, bad)
        with pytest.raises(ValueError, match=msg):
            draft_attention._configured_raw_block(1)


class _CpuPointers(kvwindow.LayerPointers):
    """The cache with host arrays, so its bookkeeping runs without a GPU."""

    capture = False

    def _capturing(self):
        return self.capture

    @staticmethod
    def _make_array(addrs, device):
        return torch.tensor(addrs, dtype=torch.int64)


def test_pointer_arrays_live_as_long_as_their_pools():
    lp = _CpuPointers(sweep_every=2)
    pool = torch.zeros(3, 8, 2, 4)
    views = [pool[i] for i in range(3)]
    a1 = lp.get(views, None)
    # fresh views of the same pool find the same array (the owner is the pool)
    assert lp.get([pool[i] for i in range(3)], None) is a1
    assert lp.get(pool, None) is not None
    # many other live pools never evict a live entry
    others = [torch.zeros(2, 4, 2, 4) for _ in range(10)]
    for o in others:
        lp.get(o, None)
    assert lp.get(views, None) is a1
    n_live = len(lp)
    # once pools die, their entries are swept
    del others, o
    gc.collect()
    for _ in range(4):
        lp.get(torch.zeros(1, 4, 2, 4), None)
        gc.collect()
    assert len(lp) < n_live
    assert lp.get(views, None) is a1


def test_pointer_array_needs_prepare_before_capture():
    lp = _CpuPointers()
    pool = torch.zeros(2, 4, 2, 4)
    lp.prepare(pool)
    lp.capture = True
    assert lp.get(pool, None) is not None          # prepared: found while capturing
    with pytest.raises(RuntimeError, match="prepare"):
        lp.get(torch.zeros(2, 4, 2, 4), None)      # not prepared: a copy cannot be captured
