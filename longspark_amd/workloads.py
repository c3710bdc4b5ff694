"""Seeded synthetic inputs for the verify-and-refresh workloads.

The workloads are the reference path's benchmark configurations:
  greedy      -- greedy chain verification, logits ~ N(0, 3^2) bf16 with the
                 drafted token boosted by +8 with probability 0.7;
  stochastic  -- rejection-sampling verification with temperature / top-k /
                 top-p (and optionally min-p, penalties over a Zipf history and
                 a packed vocabulary bitmask); draft logits = target + N(0, 1)
                 in fp32, drafted tokens sampled from the draft distribution q;
  kv window   -- paged bf16 K/V pools with a random page permutation;
  summary     -- learned summary queries, state, and new K/V rows.
Every generator takes a seed and a device; the same seed gives the same
inputs on every device (generation runs on the CPU generator unless
``gen_device`` says otherwise).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

VOCAB = 151936


def _gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(int(seed))


def greedy_inputs(batch: int, width: int = 16, vocab: int = VOCAB, *, seed: int = 0,
                  dtype=torch.bfloat16, device="cpu", gen_device="cpu", sigma: float = 3.0,
                  boost: float = 8.0, p_boost: float = 0.7):
    """Target logits ``[batch*width, vocab]`` and candidates ``[batch, width]`` int32.

    ``candidates[:, 0]`` is the current token and ``candidates[:, 1:]`` the
    drafted tokens, uniform over the vocabulary.  Row j of a request verifies
    drafted token j+1; its logit gets ``+boost`` with probability ``p_boost``.
    """
    g = _gen(seed, gen_device)
    logits = torch.randn(batch, width, vocab, generator=g, device=gen_device) * sigma
    cand = torch.randint(0, vocab, (batch, width), generator=g, device=gen_device, dtype=torch.int64)
    hit = (torch.rand(batch, width - 1, generator=g, device=gen_device) < p_boost).float() * boost
    logits[:, :-1].scatter_add_(2, cand[:, 1:, None], hit[..., None])
    logits = logits.to(dtype).reshape(batch * width, vocab)
    return logits.to(device), cand.to(torch.int32).to(device)


def zipf_history(batch: int, length: int, vocab: int = VOCAB, *, s: float = 1.1, seed: int = 0,
                 device="cpu") -> torch.Tensor:
    """``[batch, length]`` int32 token ids drawn Zipf(s) over ranks 1..vocab,
    rank r mapped to a per-request random token id."""
    g = _gen(seed, "cpu")
    ranks = torch.arange(1, vocab + 1, dtype=torch.float64)
    w = ranks.pow(-s)
    w = w / w.sum()
    draws = torch.multinomial(w.expand(batch, -1), length, replacement=True, generator=g)
    perm = torch.stack([torch.randperm(vocab, generator=g) for _ in range(batch)])
    return perm.gather(1, draws).to(torch.int32).to(device)


def random_bitmask(rows: int, vocab: int = VOCAB, *, density: float = 0.3, seed: int = 0,
                   force_tokens: Optional[torch.Tensor] = None, force_prob: float = 0.8,
                   device="cpu") -> torch.Tensor:
    """Packed int32 bitmask ``[rows, ceil(vocab/32)]`` with about ``density`` of bits set.

    When ``force_tokens [rows]`` is given, that token's bit is set with
    probability ``force_prob`` and cleared otherwise.
    """
    g = _gen(seed, "cpu")
    words = (vocab + 31) // 32
    bits = torch.rand(rows, words * 32, generator=g) < density
    if force_tokens is not None:
        keep = torch.rand(rows, generator=g) < force_prob
        bits[torch.arange(rows), force_tokens.long().cpu()] = keep
    weights = (torch.ones(32, dtype=torch.int64) << torch.arange(32))
    packed = (bits.view(rows, words, 32).to(torch.int64) * weights).sum(-1)
    packed = torch.where(packed >= 2**31, packed - 2**32, packed)
    return packed.to(torch.int32).to(device)


@dataclass
class SamplingParams:
    """Per-request sampling parameters as ``[B]`` tensors (top_k >= V, top_p >= 1
    and min_p <= 0 disable the respective filter)."""
    temperatures: torch.Tensor
    top_ks: torch.Tensor
    top_ps: torch.Tensor
    min_ps: torch.Tensor

    @staticmethod
    def uniform(batch: int, *, temperature=1.0, top_k=VOCAB, top_p=1.0, min_p=0.0, device="cpu"):
        return SamplingParams(
            temperatures=torch.full((batch,), float(temperature), dtype=torch.float32, device=device),
            top_ks=torch.full((batch,), int(top_k), dtype=torch.int32, device=device),
            top_ps=torch.full((batch,), float(top_p), dtype=torch.float32, device=device),
            min_ps=torch.full((batch,), float(min_p), dtype=torch.float32, device=device),
        )

    def to(self, device):
        return SamplingParams(*(t.to(device) for t in (self.temperatures, self.top_ks, self.top_ps,
                                                        self.min_ps)))


def sampling_distribution(logits: torch.Tensor, temperature: float, top_k: int, top_p: float,
                          min_p: float) -> torch.Tensor:
    """Dense ``[rows, V]`` fp32 distribution after temperature / top-k / top-p /
    min-p, built with plain torch ops (used to draw synthetic drafted tokens)."""
    rows, vocab = logits.shape
    scaled = logits.float() / temperature
    if top_k < vocab:
        vals, idx = torch.topk(scaled, top_k, dim=-1)
    else:
        vals, idx = torch.sort(scaled, dim=-1, descending=True)
    p = torch.softmax(vals, dim=-1)
    if top_p < 1.0:
        cum = p.cumsum(-1)
        p = torch.where(cum - p > top_p, torch.zeros_like(p), p)
        p = p / p.sum(-1, keepdim=True)
    if min_p > 0.0:
        p = torch.where(p < p[:, :1] * min_p, torch.zeros_like(p), p)
        p = p / p.sum(-1, keepdim=True)
    return torch.zeros(rows, vocab, device=logits.device).scatter_(1, idx, p)


def stochastic_inputs(batch: int, width: int = 16, vocab: int = VOCAB, *, seed: int = 0, temperature: float = 0.7,
                      top_k: int = VOCAB, top_p: float = 1.0, min_p: float = 0.0, history_len: int = 0,
                      repetition: float = 1.0, presence: float = 0.0, frequency: float = 0.0,
                      mask_density: Optional[float] = None, dtype=torch.bfloat16, device="cpu", gen_device="cpu",
                      boost_drafted: bool = False, p_boost: float = 0.7, boost: float = 8.0):
    """Inputs of one stochastic verify round.

    Target logits as in :func:`greedy_inputs`; draft logits = target + N(0, 1)
    in fp32; q = the draft distribution under the same temperature / top-k /
    top-p / min-p; drafted tokens are drawn from q; uniforms U(0, 1).
    Optional: a Zipf(1.1) history of ``history_len`` tokens per request with
    repetition / presence / frequency values, and a per-row packed bitmask
    with about ``mask_density`` of the bits set (the drafted token's bit set
    with probability 0.8).  Returns a dict of tensors on ``device``.

    Where the +``boost`` lands: by default (``boost_drafted=False``) the
    target logits are boosted at uniform random candidates before the draft
    is built, and those candidates are then replaced by the tokens drawn from
    q, so the boost marks no drafted token and almost every request rejects
    at its first position.  With ``boost_drafted=True`` the target and draft
    are built unboosted, the tokens are drawn from q, and then row j's target
    logit of drafted token j gets +``boost`` with probability ``p_boost``
    (rounded to the logits' dtype again): the drafted token is boosted, as
    the workload text says, so requests accept long prefixes, reject late or
    accept every drafted token.
    """
    logits, cand = greedy_inputs(batch, width, vocab, seed=seed, dtype=dtype, device=gen_device,
                                 gen_device=gen_device, p_boost=0.0 if boost_drafted else p_boost, boost=boost)
    g = width - 1
    gen = _gen(seed + 1, gen_device)
    target = logits.float().view(batch, width, vocab)
    draft = target[:, :g] + torch.randn(batch, g, vocab, generator=gen, device=gen_device)
    q = sampling_distribution(draft.reshape(-1, vocab), temperature, top_k, top_p, min_p)
    drafted = torch.multinomial(q, 1, generator=gen).view(batch, g)
    cand = cand.to(torch.int64)
    cand[:, 1:] = drafted
    dtp = q.view(batch, g, vocab).gather(2, drafted[..., None]).squeeze(-1).contiguous()
    uniforms = torch.rand(batch, g, generator=gen, device=gen_device)
    final = torch.rand(batch, generator=gen, device=gen_device)
    if boost_drafted:
        hit = (torch.rand(batch, g, generator=gen, device=gen_device) < p_boost).float() * boost
        target = target.clone()
        target[:, :g].scatter_add_(2, drafted[..., None], hit[..., None])
        logits = target.to(dtype).reshape(batch * width, vocab)
    out = dict(logits=logits, candidates=cand.to(torch.int32), draft_logits=draft.contiguous(),
               draft_token_probs=dtp, uniforms=uniforms, final_uniforms=final,
               params=SamplingParams.uniform(batch, temperature=temperature, top_k=top_k, top_p=top_p,
                                             min_p=min_p, device=gen_device))
    if history_len > 0:
        out["history"] = zipf_history(batch, history_len, vocab, seed=seed + 2, device=gen_device)
        out["repetition"] = torch.full((batch,), repetition, device=gen_device)
        out["presence"] = torch.full((batch,), presence, device=gen_device)
        out["frequency"] = torch.full((batch,), frequency, device=gen_device)
    if mask_density is not None:
        force = torch.cat([cand[:, 1:], cand[:, :1]], dim=1).reshape(-1)  # row j verifies cand[j+1]
        out["vocab_mask"] = random_bitmask(batch * width, vocab, density=mask_density, seed=seed + 3,
                                           force_tokens=force, device=gen_device)
    for k, v in list(out.items()):
        out[k] = v.to(device) if isinstance(v, (torch.Tensor, SamplingParams)) else v
    return out


# --------------------------------------------------------------------------
# the benchmark workloads' inputs (shared by bench.py and the parity tests)
# --------------------------------------------------------------------------

#: Sampling configuration of the fused-verify benchmark at batch 128 x block 16.
VERIFY_BENCH_CFG = dict(temperature=0.7, top_k=50, top_p=0.95, history_len=2048, repetition=1.05)
VERIFY_BENCH_SEED = 2025


def verify_bench_inputs(device, batch: int = 128, width: int = 16, vocab: int = VOCAB, *,
                        boost_drafted: bool = False, p_boost: float = 0.7):
    """The fused-verify benchmark's inputs: :func:`stochastic_inputs` with
    ``VERIFY_BENCH_CFG`` and seed 2025, generated on ``device``."""
    return stochastic_inputs(batch, width, vocab, seed=VERIFY_BENCH_SEED, device=device, gen_device=device,
                             boost_drafted=boost_drafted, p_boost=p_boost, **VERIFY_BENCH_CFG)


def window_pool(device, *, batch=8, layers=36, heads=8, dim=128, page_size=16, context=131072, window=256,
                rotate=4, seed=31):
    """Paged K/V pools for the recent-window gather at one fixed context.

    The pool holds ``batch * context`` tokens per layer (K and V; 154.6 GB at
    8 x 131,072 x 36 layers x 8 heads x 128 bf16) with every request's pages
    placed by one random permutation.  Only the pages of the last ``rotate``
    windows are filled (N(0, 1) bf16); the rest is allocated but never read.
    ``seq_sets[j]`` are the sequence lengths ``context - j * window``, whose
    windows are disjoint.  Returns a dict with ``k``, ``v`` (lists of
    ``[N, heads, dim]``), ``table`` (``[batch, pages]`` int32), ``seq_sets``
    and ``touched_rows`` (the filled pool rows).
    """
    g = torch.Generator(device=device).manual_seed(seed)
    pages_per = context // page_size
    total_pages = batch * pages_per
    perm = torch.randperm(total_pages, generator=g, device=device).to(torch.int32)
    table = perm.view(batch, pages_per)
    seq_sets = [torch.full((batch,), context - j * window, dtype=torch.int64, device=device) for j in range(rotate)]
    n = total_pages * page_size
    k = [torch.empty(n, heads, dim, dtype=torch.bfloat16, device=device) for _ in range(layers)]
    v = [torch.empty(n, heads, dim, dtype=torch.bfloat16, device=device) for _ in range(layers)]
    first = (context - rotate * window) // page_size
    touched = table[:, first:].reshape(-1).long()
    rows = (touched[:, None] * page_size + torch.arange(page_size, device=device)[None, :]).reshape(-1)
    for t in k + v:
        t[rows] = torch.randn(rows.numel(), heads, dim, generator=g, device=device).to(torch.bfloat16)
    return dict(k=k, v=v, table=table, seq_sets=seq_sets, touched_rows=rows, page_size=page_size, window=window)


#: Geometry of the full verify-and-refresh round (Qwen3-14B).
FULL_ROUND = dict(batch=128, width=16, layers=40, q_heads=40, kv_heads=8, dim=128, rows=52, page=16, window=256)


def full_round_refresh_inputs(device, *, batch=128, width=16, layers=40, q_heads=40, kv_heads=8, dim=128, rows=52,
                              page=16, window=256, seed=91):
    """Refresh-side inputs of the full round: contexts U[8K, 32K], a page
    table over a pool that holds the pages the windows touch plus as many
    distractor pages (other table entries alias random pool pages: 128
    contexts of this size do not fit in HBM), K/V pools per layer, the
    committed rows' locations (the last ``width`` positions of each context),
    summary queries ``[layers, q_heads, rows, dim]`` bf16 and the fp32 summary
    state and LSE."""
    g = torch.Generator(device=device).manual_seed(seed)
    ctx = torch.randint(8192, 32769, (batch,), generator=g, device=device)
    pages_per = 32768 // page
    win_pages = window // page + 1
    pool_pages = 2 * batch * win_pages
    table = torch.randint(0, pool_pages, (batch, pages_per), generator=g, device=device, dtype=torch.int32)
    own = torch.randperm(pool_pages, generator=g, device=device)[:batch * win_pages].view(batch, win_pages)
    cols = ((ctx - window) // page)[:, None] + torch.arange(win_pages, device=device)[None, :]
    table.scatter_(1, cols.clamp(max=pages_per - 1), own.to(torch.int32))
    n = pool_pages * page
    k = [torch.randn(n, kv_heads, dim, generator=g, device=device).to(torch.bfloat16) for _ in range(layers)]
    v = [torch.randn(n, kv_heads, dim, generator=g, device=device).to(torch.bfloat16) for _ in range(layers)]
    pos = ctx[:, None] - width + torch.arange(width, device=device)[None, :]
    locs = table.gather(1, (pos // page)).long() * page + pos % page
    query = torch.randn(layers, q_heads, rows, dim, generator=g, device=device).to(torch.bfloat16)
    state = torch.randn(batch, layers, q_heads, rows, dim, generator=g, device=device)
    lse = torch.randn(batch, layers, q_heads, rows, generator=g, device=device)
    return dict(seq=ctx, table=table, k=k, v=v, locs=locs, query=query, state=state, lse=lse, page=page,
                window=window)
