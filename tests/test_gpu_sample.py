"""Drafter proposal step (``sample_step_tokens_with_q``) on the GPU vs the oracle.

Rows of fp32 and bf16 logits at the full 151,936 vocabulary (vector path),
an odd vocabulary with a row stride wider than it (element path), masked
(-inf) entries, per-row temperatures, invalid rows, scaled logits near the
float range (the exact-quotient path), and the workspace path that draws its
own noise.  Tokens bit-exact except where the two largest keys
p / E lie within 1e-6 of each other (fp64 keys); q within 1e-5 relative of the
fp64 value of p at the kernel's token.
"""

import pytest
import torch

from oracle import verify as ov
from longspark_amd import sample, workloads

pytestmark = pytest.mark.gpu


def check(logits, temps, noise, tokens, q):
    tok_r, q_r, valid = ov.sample_step_tokens_with_q(logits.cpu(), temps.cpu(), noise.cpu(),
                                                     compute_dtype=torch.float64)
    tokens, q = tokens.cpu(), q.cpu()
    assert bool(valid.all())
    x = logits.cpu().double()
    s = torch.where(torch.isfinite(x), x / temps.cpu().double()[:, None], torch.full_like(x, float("-inf")))
    p = torch.softmax(s, dim=-1)
    keys = p / noise.cpu().double()
    for r in range(tokens.numel()):
        if int(tokens[r]) != int(tok_r[r]):
            a, b = float(keys[r, tokens[r]]), float(keys[r, tok_r[r]])
            assert abs(a - b) <= 1e-6 * b, (r, int(tokens[r]), int(tok_r[r]), a, b)
        want = float(p[r, tokens[r]])
        assert abs(float(q[r]) - want) <= 1e-5 * want, (r, float(q[r]), want)


@pytest.mark.parametrize("dtype,vocab,stride_pad", [(torch.float32, workloads.VOCAB, 0),
                                                    (torch.bfloat16, workloads.VOCAB, 0),
                                                    (torch.float32, 5001, 3), (torch.bfloat16, 5001, 5)])
def test_sample_step_matches_oracle(dev, dtype, vocab, stride_pad):
    rows = 12
    g = torch.Generator().manual_seed(vocab + stride_pad)
    base = 4.0 * torch.randn(rows, vocab + stride_pad, generator=g)
    base[2, ::3] = float("-inf")                       # masked entries
    base[3, : vocab // 2] = float("-inf")
    logits = base.to(dtype)[:, :vocab]                 # row stride vocab + pad
    temps = torch.linspace(0.3, 1.7, rows)
    noise = torch.empty(rows, vocab).exponential_(1, generator=g)
    print(f"sample_step {dtype} V={vocab} pad={stride_pad}", flush=True)
    tokens, q = sample.sample_step_tokens_with_q(step_logits=logits.to(dev), temperatures=temps.to(dev),
                                                 exp_noise=noise.to(dev), check=True)
    torch.cuda.synchronize()
    assert tokens.dtype == torch.int64 and q.dtype == torch.float32
    check(logits, temps, noise, tokens, q)


def test_sample_step_invalid_rows(dev):
    inf = float("inf")
    vocab = 3000
    x = torch.randn(6, vocab)
    x[1, 17] = float("nan")
    x[2, 2999] = inf
    x[3] = -inf
    temps = torch.tensor([1.0, 1.0, 1.0, 1.0, 0.0, 1.0])
    noise = torch.empty(6, vocab).exponential_(1, generator=torch.Generator().manual_seed(3))
    noise[5, 100] = 0.0
    print("sample_step invalid rows", flush=True)
    tokens, q = sample.sample_step_tokens_with_q(step_logits=x.to(dev), temperatures=temps.to(dev),
                                                 exp_noise=noise.to(dev))
    torch.cuda.synchronize()
    tok_r, q_r, valid = ov.sample_step_tokens_with_q(x, temps, noise)
    assert valid.tolist() == [True, False, False, False, False, False]
    assert torch.equal(tokens.cpu()[1:], torch.zeros(5, dtype=torch.int64))
    assert bool(torch.isnan(q.cpu()[1:]).all()) and not bool(torch.isnan(q.cpu()[0]))
    with pytest.raises(RuntimeError, match="invalid probability row"):
        sample.sample_step_tokens_with_q(step_logits=x.to(dev), temperatures=temps.to(dev),
                                         exp_noise=noise.to(dev), check=True)


def test_sample_step_scaled_logit_near_the_float_range(dev):
    """Entries whose product l * (1/T) reaches 1e37 take the exact quotient l / T
    (only in the wave that holds them): a huge finite scaled logit stays valid
    and wins its row, one that overflows makes the row invalid."""
    vocab = workloads.VOCAB
    g = torch.Generator().manual_seed(11)
    x = 3.0 * torch.randn(3, vocab, generator=g)
    x[0, 1234] = 2.0e37          # l / T = 2.2e37: finite, far above every other entry
    x[1, 5] = 3.0e38             # l / T = 6e38: +inf, an invalid row
    temps = torch.tensor([0.9, 0.5, 1.1])
    noise = torch.empty(3, vocab).exponential_(1, generator=g)
    print("sample_step scaled logits near the float range", flush=True)
    tokens, q = sample.sample_step_tokens_with_q(step_logits=x.to(dev), temperatures=temps.to(dev),
                                                 exp_noise=noise.to(dev))
    torch.cuda.synchronize()
    tok_r, q_r, valid = ov.sample_step_tokens_with_q(x, temps, noise)
    assert valid.tolist() == [True, False, True]
    tokens, q = tokens.cpu(), q.cpu()
    assert int(tokens[0]) == 1234 and int(tok_r[0]) == 1234 and abs(float(q[0]) - 1.0) <= 1e-6
    assert int(tokens[1]) == 0 and bool(torch.isnan(q[1]))
    check(x[2:], temps[2:], noise[2:], tokens[2:], q[2:])


def test_sample_step_workspace_draws_noise(dev):
    rows, vocab = 8, 20000
    logits = (3.0 * torch.randn(rows, vocab, generator=torch.Generator().manual_seed(9))).to(dev)
    temps = torch.full((rows,), 0.8, device=dev)
    ws = sample.create_sample_step_workspace(batch=rows, vocab=vocab, device=dev)
    print("sample_step workspace noise", flush=True)
    torch.cuda.manual_seed(77)
    tokens, q = sample.sample_step_tokens_with_q(step_logits=logits, temperatures=temps, workspace=ws)
    torch.cuda.synchronize()
    torch.cuda.manual_seed(77)
    noise = torch.empty(rows, vocab, device=dev).exponential_(1)
    assert torch.equal(noise, ws.exp_noise)
    check(logits, temps, noise, tokens, q)
    with pytest.raises(ValueError, match="workspace batch"):
        sample.sample_step_tokens_with_q(step_logits=logits[:4], temperatures=temps[:4], workspace=ws)
    with pytest.raises(TypeError):
        sample.sample_step_tokens_with_q(step_logits=logits.half(), temperatures=temps)
