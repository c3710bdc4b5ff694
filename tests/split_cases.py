"""Hand-worked cases of the split engine's two-phase rejection sampling,
src/longspark/engine/sampling.py:19-57 (``decide_acceptance`` then
``finish_sampling`` with host uniforms).

Every expected value below was worked out by hand from the rules the
reference states in code, not computed by a formula here:
  * acceptance at position j is the strict test ``u_j * q_j < p_j[cand_j]``,
    and the length is the number of leading accepted positions;
  * requests with length < gamma are the rejected rows, listed in request
    order with their rejection positions;
  * ``target_rows[b]`` is the target row at index ``lengths[b]`` (the bonus
    row, index gamma, when every drafted token is accepted);
  * a rejected request draws from ``max(p - q, 0)`` normalised, unless that
    mass is <= 1e-8, when it draws from p itself;
  * the token is the count of CDF entries at or below u, clamped to V - 1.
All probabilities are sums of powers of two, so every fp32 operation on them
is exact and the cases pin the comparisons themselves (equality rejects,
equality of u and a CDF entry moves past that entry, the 1e-8 threshold).
"""

from __future__ import annotations

import torch

# ---------------------------------------------------------------------------
# decide_acceptance: 4 requests, gamma = 3, vocabulary 4.
#   request 0: position 0 accepted (0.25 < 0.5), position 1 has u*q == p
#              (0.25 == 0.25): rejected -> length 1
#   request 1: every position accepted -> length 3 = gamma, target row 3
#   request 2: position 0 rejected (0.375 >= 0.25); positions 1-2 would
#              accept but the prefix stops at 0 -> length 0
#   request 3: positions 0, 1 accepted; position 2: u*q = 0.5*1.0 = 0.5 > p = 0.125
#              -> length 2
# ---------------------------------------------------------------------------

GAMMA = 3
VOCAB = 4


def decide_case():
    p = torch.zeros(4, GAMMA + 1, VOCAB)
    # request 0: rows 0, 1 (row j verifies candidate j); row 1 is the target row
    p[0, 0] = torch.tensor([0.125, 0.5, 0.25, 0.125])
    p[0, 1] = torch.tensor([0.25, 0.25, 0.25, 0.25])
    p[0, 2] = torch.tensor([0.5, 0.25, 0.125, 0.125])
    p[0, 3] = torch.tensor([0.0, 0.0, 0.5, 0.5])
    # request 1: accepted everywhere; row 3 is the bonus row
    p[1, 0] = torch.tensor([1.0, 0.0, 0.0, 0.0])
    p[1, 1] = torch.tensor([0.0, 1.0, 0.0, 0.0])
    p[1, 2] = torch.tensor([0.0, 0.0, 1.0, 0.0])
    p[1, 3] = torch.tensor([0.125, 0.125, 0.25, 0.5])
    # request 2
    p[2, 0] = torch.tensor([0.25, 0.25, 0.25, 0.25])
    p[2, 1] = torch.tensor([0.5, 0.5, 0.0, 0.0])
    p[2, 2] = torch.tensor([0.5, 0.5, 0.0, 0.0])
    p[2, 3] = torch.tensor([0.25, 0.25, 0.25, 0.25])
    # request 3
    p[3, 0] = torch.tensor([0.0, 0.0, 0.0, 1.0])
    p[3, 1] = torch.tensor([0.0, 0.0, 0.5, 0.5])
    p[3, 2] = torch.tensor([0.125, 0.125, 0.25, 0.5])
    p[3, 3] = torch.tensor([0.25, 0.25, 0.25, 0.25])
    cand = torch.tensor([[1, 2, 0],
                         [0, 1, 2],
                         [3, 0, 1],
                         [3, 2, 0]], dtype=torch.int64)
    q = torch.tensor([[0.5, 0.5, 0.5],
                      [1.0, 1.0, 1.0],
                      [0.75, 0.5, 0.5],
                      [0.5, 0.5, 1.0]])
    u = torch.tensor([[0.5, 0.5, 0.5],
                      [0.875, 0.875, 0.875],
                      [0.5, 0.5, 0.5],
                      [0.5, 0.5, 0.5]])
    expected = dict(lengths=[1, 3, 0, 2], rejected_rows=[0, 2, 3], rejection_positions=[1, 0, 2],
                    target_row_index=[1, 3, 0, 2])
    return p, cand, q, u, expected


# ---------------------------------------------------------------------------
# finish_sampling on the decision above (rejected rows 0, 2, 3; request 1
# accepted everything and draws from its bonus row p[1, 3]).
#   request 0: target row p[0,1] = [.25,.25,.25,.25], q row [.5,0,.25,.25]
#              residual [0,.25,0,0] -> normalised [0,1,0,0], CDF [0,1,1,1];
#              u = 0.5: entries <= u: only CDF[0] = 0 -> token 1
#   request 1: p[1,3] = [.125,.125,.25,.5], CDF [.125,.25,.5,1.0];
#              u = 0.5: CDF entries <= 0.5 are 3 (equality counts) -> token 3
#   request 2: target row p[2,0] = [.25,.25,.25,.25], q row equal to it:
#              residual 0 <= 1e-8 -> falls back to p, CDF [.25,.5,.75,1];
#              u = 0.6 -> 2 entries <= u -> token 2
#   request 3: target row p[3,2] = [.125,.125,.25,.5], q row [0,.25,.25,.5]:
#              residual [.125,0,0,0] -> [1,0,0,0], CDF [1,1,1,1];
#              u = 0.999 -> token 0
# ---------------------------------------------------------------------------

def finish_case():
    q_rows = torch.tensor([[0.5, 0.0, 0.25, 0.25],
                           [0.25, 0.25, 0.25, 0.25],
                           [0.0, 0.25, 0.25, 0.5]])
    u = torch.tensor([0.5, 0.5, 0.6, 0.999])
    return q_rows, u, [1, 3, 2, 0]


# ---------------------------------------------------------------------------
# The 1e-8 residual-mass threshold and the clamp to V - 1, on single-request
# decisions with a given target row (one rejected request at position 0).
#   mass 2**-27 (7.45e-9 <= 1e-8): falls back to p = [.125,.875] -> u = 0.5 -> token 1
#   mass 2**-26 (1.49e-8 >  1e-8): residual [2**-26, 0] normalised [1, 0] -> token 0
#   unnormalised row (an accepted request whose bonus row sums to 0.875):
#   CDF [.25,.5,.75,.875], u = 0.9 -> all 4 entries <= u -> clamped to 3
# ---------------------------------------------------------------------------

def threshold_cases():
    p = torch.tensor([0.125, 0.875])
    below = torch.tensor([0.125 - 2.0 ** -27, 0.875 + 2.0 ** -27])
    above = torch.tensor([0.125 - 2.0 ** -26, 0.875 + 2.0 ** -26])
    assert float(p[0] - below[0]) == 2.0 ** -27 and float(p[0] - above[0]) == 2.0 ** -26  # exact in fp32
    clamp_row = torch.tensor([0.25, 0.25, 0.25, 0.125])
    return [
        ("mass 2^-27 falls back to p", p, below, 0.5, 1),
        ("mass 2^-26 uses the residual", p, above, 0.5, 0),
    ], (clamp_row, 0.9, 3)
