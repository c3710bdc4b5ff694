"""The vocabulary bitmask in place on the GPU vs the oracle's
``apply_token_bitmask`` (SRT/constrained/triton_ops/bitmask_ops.py:60-141).

Cases: config 2's masks (32 requests x 16 rows x 151,936 bf16, about 30% of
bits set) through ``apply_token_bitmask_inplace`` (``ls_apply_token_bitmask``)
and through ``adjust_logits_`` (``ls_adjust_logits``); fp32 and fp16 logits;
``indices`` as a list and as a tensor (a subset, out of order, with a
repeat); a mask narrower than the vocabulary; a vocabulary that is not a
multiple of 32; rows whose start is not 16-byte aligned; 1-D inputs; the
reference's assertion messages.  Bit-exact.
"""

import pytest
import torch

from oracle import verify as ov
from longspark_amd import penalties, workloads

pytestmark = pytest.mark.gpu


def _expected(logits, mask, indices=None):
    ref = logits.clone().float()
    rows = range(logits.shape[0]) if indices is None else sorted(set(int(i) for i in indices))
    for r in rows:
        row = ref[r:r + 1]
        ov.apply_token_bitmask(row, mask[r:r + 1])
        ref[r:r + 1] = row
    return ref.to(logits.dtype)


def _same(a, b):
    return torch.equal(a.view(torch.int16 if a.element_size() == 2 else torch.int32),
                       b.view(torch.int16 if b.element_size() == 2 else torch.int32))


@pytest.mark.parametrize("entry", ["apply_token_bitmask_inplace", "adjust_logits_"])
def test_config2_masks(dev, entry):
    d = workloads.stochastic_inputs(32, 16, seed=12, temperature=0.8, top_p=0.9, min_p=0.05, mask_density=0.3)
    logits, mask = d["logits"], d["vocab_mask"]
    print(f"bitmask {entry}: {tuple(logits.shape)} bf16, mask {tuple(mask.shape)}", flush=True)
    x = logits.to(dev)
    if entry == "apply_token_bitmask_inplace":
        penalties.apply_token_bitmask_inplace(x, mask.to(dev))
    else:
        penalties.adjust_logits_(x, rows_per_request=1, vocab_mask=mask.to(dev))
    torch.cuda.synchronize()
    assert _same(x.cpu(), _expected(logits, mask))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_dtypes_and_indices(dev, dtype):
    g = torch.Generator().manual_seed(3)
    rows, vocab = 12, 151936
    logits = (3 * torch.randn(rows, vocab, generator=g)).to(dtype)
    mask = workloads.random_bitmask(rows, vocab, density=0.4, seed=4)
    idx_list = [7, 2, 11, 2, 5]
    for indices in (idx_list, torch.tensor(idx_list, dtype=torch.int64)):
        x = logits.to(dev)
        ind = indices.to(dev) if isinstance(indices, torch.Tensor) else indices
        penalties.apply_token_bitmask_inplace(x, mask.to(dev), ind)
        torch.cuda.synchronize()
        assert _same(x.cpu(), _expected(logits, mask, idx_list)), type(indices)


def test_narrow_mask_odd_vocab_and_unaligned_rows(dev):
    g = torch.Generator().manual_seed(5)
    # vocabulary 1000 (not a multiple of 32) with a mask of 20 words (640 columns)
    logits = torch.randn(6, 1000, generator=g).to(torch.bfloat16)
    mask = workloads.random_bitmask(6, 640, density=0.5, seed=6)
    x = logits.to(dev)
    penalties.apply_token_bitmask_inplace(x, mask.to(dev))
    torch.cuda.synchronize()
    got = x.cpu()
    assert _same(got, _expected(logits, mask))
    assert _same(got[:, 640:], logits[:, 640:])
    # full-width mask over an odd vocabulary: the last word covers 8 columns
    mask = workloads.random_bitmask(6, 1000, density=0.5, seed=7)
    x = logits.to(dev)
    penalties.apply_token_bitmask_inplace(x, mask.to(dev))
    torch.cuda.synchronize()
    assert _same(x.cpu(), _expected(logits, mask))
    # rows that start 2 bytes past a 16-byte boundary (a column-offset view)
    base = torch.randn(4, 4097, generator=g).to(torch.bfloat16)
    mask = workloads.random_bitmask(4, 4096, density=0.3, seed=8)
    xb = base.to(dev)
    view = xb[:, 1:]
    penalties.apply_token_bitmask_inplace(view, mask.to(dev))
    torch.cuda.synchronize()
    exp = base.clone()
    exp[:, 1:] = _expected(base[:, 1:].contiguous(), mask)
    assert _same(xb.cpu(), exp)


def test_one_dimensional_inputs_and_assertions(dev):
    logits = torch.randn(4096).to(torch.bfloat16)
    mask = workloads.random_bitmask(1, 4096, density=0.5, seed=9)[0]
    x = logits.to(dev)
    penalties.apply_token_bitmask_inplace(x, mask.to(dev))
    torch.cuda.synchronize()
    assert _same(x.cpu()[None], _expected(logits[None], mask[None]))
    with pytest.raises(AssertionError, match="bitmask must be of type int32"):
        penalties.apply_token_bitmask_inplace(x, mask.to(dev).to(torch.int64))
    with pytest.raises(AssertionError, match="Bitmask width too large"):
        penalties.apply_token_bitmask_inplace(x, torch.zeros(129, dtype=torch.int32, device=dev))
    with pytest.raises(AssertionError, match="batch size mismatch"):
        penalties.apply_token_bitmask_inplace(torch.zeros(3, 64, device=dev),
                                              torch.zeros(2, 2, dtype=torch.int32, device=dev))
