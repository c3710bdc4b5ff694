"""Pin the oracle's greedy verification (CPU only).

Checks: brute-force python loops on small random inputs (first-index argmax,
first-mismatch prefix), constructed ties, all-accepted / first-mismatch
special cases, and agreement between the [B, K] and split-engine layouts.
"""

import random

import torch

from oracle import verify as ov


def brute_argmax(row):
    best, idx = row[0], 0
    for i, v in enumerate(row):
        if v > best:
            best, idx = v, i
    return idx


def brute_accept(cand, truth):
    n = 0
    while n < len(truth) - 1 and cand[n + 1] == truth[n]:
        n += 1
    return n, truth[n]


def test_greedy_matches_brute_force_random():
    rng = random.Random(7)
    for trial in range(200):
        b, k, v = rng.randint(1, 4), rng.randint(2, 6), rng.randint(1, 9)
        # few distinct values -> many ties
        logits = torch.tensor([[rng.choice([-1.0, 0.0, 0.5, 2.0]) for _ in range(v)] for _ in range(b * k)])
        truth_rows = [brute_argmax(r) for r in logits.tolist()]
        cand = torch.tensor([[rng.randrange(v) for _ in range(k)] for _ in range(b)])
        # make some drafts match the truth so long prefixes occur
        for bi in range(b):
            for j in range(k - 1):
                if rng.random() < 0.6:
                    cand[bi, j + 1] = truth_rows[bi * k + j]
        lens, bonus, trim = ov.accept_greedy(cand, logits, k)
        for bi in range(b):
            n, bon = brute_accept(cand[bi].tolist(), truth_rows[bi * k:(bi + 1) * k])
            assert int(lens[bi]) == n and int(bonus[bi]) == bon
        assert trim.eq(0).all()


def test_greedy_special_cases():
    v, k = 11, 5
    logits = torch.zeros(k, v)
    truth = [3, 7, 7, 0, 10]
    for j, t in enumerate(truth):
        logits[j, t] = 5.0
    all_match = torch.tensor([[9, 3, 7, 7, 0]])
    lens, bonus, _ = ov.accept_greedy(all_match, logits, k)
    assert int(lens) == k - 1 and int(bonus) == 10
    first_bad = torch.tensor([[9, 4, 7, 7, 0]])
    lens, bonus, _ = ov.accept_greedy(first_bad, logits, k)
    assert int(lens) == 0 and int(bonus) == 3
    # exact ties resolve to the first maximal index
    tied = torch.zeros(1, v)
    tied[0, [2, 5, 9]] = 1.0
    assert int(ov.greedy_truth(tied)) == 2
    # all -inf row -> index 0
    assert int(ov.greedy_truth(torch.full((1, v), float("-inf")))) == 0


def test_split_layout_matches_block_layout():
    g = torch.Generator().manual_seed(3)
    b, k, v = 6, 8, 50
    logits = torch.randint(0, 4, (b * k, v), generator=g).float()
    cand = torch.randint(0, v, (b, k), generator=g)
    truth = ov.greedy_truth(logits).view(b, k)
    cand[:, 1:4] = truth[:, 0:3]
    lens, bonus, _ = ov.accept_greedy(cand, logits, k)
    acc, bon = ov.greedy_verify_split(cand[:, 1:], logits.view(b, k, v))
    assert torch.equal(acc, lens.long()) and torch.equal(bon, bonus)
