"""The custom operators are registered and their fake implementations give
the right output shapes and dtypes (no GPU: fake tensors only)."""

import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from longspark_amd import ops


def test_every_operator_is_registered():
    for name in ops.OPS:
        assert hasattr(torch.ops.longspark_amd, name), name


def test_fake_shapes():
    V, B, K = 151936, 4, 16
    with FakeTensorMode():
        dev = "cuda"
        logits = torch.empty(B * K, V, dtype=torch.bfloat16, device=dev)
        cand = torch.empty(B, K, dtype=torch.int32, device=dev)
        acc, bonus, trim = torch.ops.longspark_amd.verify_greedy(logits, cand, K)
        assert (acc.shape, acc.dtype, bonus.dtype, trim.dtype) == ((B,), torch.int32, torch.int64, torch.int32)
        hist = torch.empty(B, 2048, dtype=torch.int32, device=dev)
        bits, rank, add, distinct, nonpos = torch.ops.longspark_amd.penalty_tables(hist, V)
        assert bits.shape == (B, 4748) and add.shape == (B, 2048) and nonpos.shape == (B,)
        f = lambda *s: torch.empty(*s, device=dev)  # noqa: E731
        acc, bonus, trim = torch.ops.longspark_amd.verify_sample(
            logits, cand, K, f(B), f(B, K - 1), f(B), draft_token_probs=f(B, K - 1), draft_logits=f(B, K - 1, V),
            pen_bits=bits, pen_rank=rank, pen_add=add, pen_nonpositive=nonpos)
        assert acc.shape == (B,) and bonus.dtype == torch.int64
        probs = torch.ops.longspark_amd.softmax_temp(logits, f(B), K)
        assert probs.shape == (B * K, V) and probs.dtype == torch.float32
        mask = torch.empty(B * K, 4748, dtype=torch.int32, device=dev)
        assert torch.ops.longspark_amd.apply_token_bitmask(logits, mask) is None
