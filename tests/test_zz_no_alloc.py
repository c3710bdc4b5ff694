"""The allocation-free greedy verify (``ls_verify_greedy_noalloc``) through
the C ABI: the same outputs as ``ls_verify_greedy`` with a workspace, on two
calls in a row, the second with a smaller input; and a call beyond the
built-in buffer is rejected before any launch."""

import ctypes

import pytest
import torch

from longspark_amd import _lib, verify, workloads

pytestmark = pytest.mark.gpu


def _noalloc(logits, cand, width, cutoff=None):
    dev = logits.device
    batch = cand.shape[0]
    acc = torch.full((batch,), -7, dtype=torch.int32, device=dev)
    bonus = torch.full((batch,), -7, dtype=torch.int64, device=dev)
    truth = torch.full((batch * width,), -7, dtype=torch.int32, device=dev)
    trim = torch.full((batch,), -7, dtype=torch.int32, device=dev)
    _lib.call("ls_verify_greedy_noalloc", logits.data_ptr(), _lib.dtype_code(logits), logits.stride(0),
              cand.data_ptr(), _lib.dtype_code(cand), cand.stride(0), cand.stride(1), 1, batch, width,
              logits.shape[1], _lib.ptr(cutoff), acc.data_ptr(), bonus.data_ptr(), truth.data_ptr(), trim.data_ptr(),
              _lib.stream_of(dev))
    return acc, bonus, truth, trim


@pytest.mark.parametrize("first,second", [((128, 16), (8, 16)), ((64, 8), (3, 8))])
def test_noalloc_matches_workspace_entry(dev, first, second):
    for i, (batch, width) in enumerate((first, second)):
        print(f"noalloc greedy call {i}: B={batch} K={width}", flush=True)
        logits, cand = workloads.greedy_inputs(batch, width, seed=100 + i, device=dev)
        cutoff = torch.randint(1, width + 1, (batch,), dtype=torch.int32, device=dev) if i else None
        got = _noalloc(logits, cand, width, cutoff)
        ref = verify.verify_greedy(logits=logits, candidates=cand, width=width, cutoff_verify_lens=cutoff,
                                   return_truth=True)
        torch.cuda.synchronize()
        acc, bonus, trim, truth = ref
        assert torch.equal(got[0], acc) and torch.equal(got[1], bonus)
        assert torch.equal(got[2], truth) and torch.equal(got[3], trim)


def test_noalloc_rejects_oversized_calls(dev):
    logits = torch.empty(1, 8, dtype=torch.bfloat16, device=dev)
    cand = torch.zeros(1, 2, dtype=torch.int32, device=dev)
    out = torch.empty(1, dtype=torch.int64, device=dev)
    rc = _lib.lib().ls_verify_greedy_noalloc(logits.data_ptr(), _lib.LS_BF16, 8, cand.data_ptr(), _lib.LS_I32, 2,
                                             1, 1, 65536, 64, 8, None, out.data_ptr(), out.data_ptr(), None, None,
                                             _lib.stream_of(dev))
    assert rc == _lib.LS_ERR_WORKSPACE
    assert b"built-in buffer" in _lib.lib().ls_last_error()
