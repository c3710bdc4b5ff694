"""Greedy verify on the GPU vs the CPU oracle: bit-exact accept lengths, bonus
tokens and row argmaxes.

Cases: the greedy workload at batch 1 (block 16) and batch 128 (block 16) on
the full 151,936 vocabulary; every logits dtype; both candidate layouts
([B, K] with the current token first, and the split engine's drafted-only
[B, K-1]); int32 and int64 candidates; rows with exact ties and all -inf
rows; an odd vocabulary (rows not 16-byte aligned); tiny vocabularies; the
cutoff-layout cap.
"""

import pytest
import torch

from oracle import verify as ov
from longspark_amd import verify, workloads

pytestmark = pytest.mark.gpu


def run_case(dev, logits, cand, width, first_col=1, cutoff=None):
    print(f"greedy case rows={logits.shape[0]} vocab={logits.shape[1]} dtype={logits.dtype} "
          f"cand={tuple(cand.shape)}/{cand.dtype} first_col={first_col}", flush=True)
    acc, bon, trim, truth = verify.verify_greedy(
        logits=logits if logits.is_cuda else logits.to(dev), candidates=cand.to(dev), width=width,
        cand_first_col=first_col, cutoff_verify_lens=None if cutoff is None else cutoff.to(dev),
        return_truth=True)
    torch.cuda.synchronize()
    logits, cand = logits.cpu(), cand.cpu()
    ref_truth = ov.greedy_truth(logits.float())
    assert torch.equal(truth.cpu().long(), ref_truth), "row argmax differs"
    full = cand if first_col == 1 else torch.cat([torch.zeros_like(cand[:, :1]), cand], 1)
    ref_len, ref_bonus = ov.compute_correct_drafts_and_bonus(full.long(), ref_truth.view(-1, width))
    ref_trim = torch.zeros_like(ref_len)
    if cutoff is not None:
        cap = (cutoff.to(torch.int32) - 1).clamp(0, width - 1)
        capped = torch.minimum(ref_len, cap)
        ref_trim = ref_len - capped
        ref_len = capped
        ref_bonus = ref_truth.view(-1, width)[torch.arange(full.shape[0]), capped.long()]
    assert torch.equal(acc.cpu(), ref_len)
    assert torch.equal(bon.cpu(), ref_bonus)
    assert torch.equal(trim.cpu(), ref_trim)
    return acc.cpu()


@pytest.mark.parametrize("batch", [1, 128])
def test_greedy_workload_full_vocab(dev, batch):
    logits, cand = workloads.greedy_inputs(batch, 16, seed=100 + batch)
    # Force long accepted prefixes in half the requests so every length occurs.
    truth = ov.greedy_truth(logits.float()).view(batch, 16)
    for b in range(0, batch, 2):
        n = b % 16
        cand[b, 1:1 + n] = truth[b, :n].to(torch.int32)
    run_case(dev, logits, cand, 16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cand_dtype", [torch.int32, torch.int64])
def test_greedy_dtypes_and_layouts(dev, dtype, cand_dtype):
    g = torch.Generator().manual_seed(11)
    b, k, v = 5, 8, 4096 + 64
    logits = (torch.randint(-3, 4, (b * k, v), generator=g).float()).to(dtype)  # heavy ties
    cand = torch.randint(0, v, (b, k), generator=g).to(cand_dtype)
    truth = ov.greedy_truth(logits.float()).view(b, k)
    cand[:, 1:5] = truth[:, :4].to(cand_dtype)
    run_case(dev, logits, cand, k, first_col=1)
    run_case(dev, logits, cand[:, 1:].contiguous(), k, first_col=0)


def test_greedy_ties_and_neg_inf_rows(dev):
    b, k, v = 2, 4, 30000
    logits = torch.full((b * k, v), -5.0)
    logits[0, [17, 400, 29999]] = 3.0            # tie across slices -> 17
    logits[1, :] = float("-inf")                  # all -inf -> 0
    logits[2, [29999, 12000]] = 1.0               # -> 12000
    logits[3, 0] = 0.5
    logits[4:] = torch.randn(4, v)
    cand = torch.tensor([[0, 17, 0, 12000], [1, 2, 3, 4]], dtype=torch.int32)
    acc = run_case(dev, logits.to(torch.bfloat16), cand, k)
    assert int(acc[0]) == 3


@pytest.mark.parametrize("vocab", [1, 7, 33, 151937])
def test_greedy_unaligned_and_tiny_vocab(dev, vocab):
    g = torch.Generator().manual_seed(vocab)
    b, k = 3, 6
    logits = torch.randn(b * k, vocab, generator=g).to(torch.bfloat16)
    cand = torch.randint(0, vocab, (b, k), generator=g).to(torch.int32)
    truth = ov.greedy_truth(logits.float()).view(b, k)
    cand[:, 1:3] = truth[:, :2].to(torch.int32)
    run_case(dev, logits, cand, k)


def test_greedy_strided_rows_and_cutoff(dev):
    g = torch.Generator().manual_seed(5)
    b, k, v = 4, 8, 10000
    base = torch.randn(b * k, v + 24, generator=g).to(torch.bfloat16).to(dev)
    logits = base[:, :v]  # row stride v + 24 (16-byte aligned rows)
    assert logits.stride(0) == v + 24
    cand = torch.randint(0, v, (b, k), generator=g).to(torch.int64)
    truth = ov.greedy_truth(logits.float().cpu()).view(b, k)
    cand[:, 1:] = truth[:, :-1]  # all accepted before the cap
    cutoff = torch.tensor([1, 3, 8, 20], dtype=torch.int64)
    run_case(dev, logits, cand, k, cutoff=cutoff)


def test_greedy_repeated_calls_reuse_workspace(dev):
    logits, cand = workloads.greedy_inputs(16, 16, seed=9)
    ld, cd = logits.to(dev), cand.to(dev)
    first = verify.verify_greedy(logits=ld, candidates=cd, width=16)
    for _ in range(5):
        again = verify.verify_greedy(logits=ld, candidates=cd, width=16)
        assert all(torch.equal(a, b) for a, b in zip(first, again))
    small_l, small_c = workloads.greedy_inputs(2, 16, seed=10)
    run_case(dev, small_l, small_c, 16)
