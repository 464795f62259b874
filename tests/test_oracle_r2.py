"""R2 near-equal-probability fixture on the CPU (speccheck/moe_ref.py:338).

The softmax's ids are fixed by the logits except where two distinct logits give probabilities
within a couple of f32 ulps; there they depend on the last bit of each exp and of the reciprocal of
the sum, which differ between torch builds and CPUs. These tests check that the fixture has such
rows, and that the fragile-row classifier is sound: two valid f32 softmax evaluations (torch's
kernel, and correctly rounded exps summed in another order) agree on the ids of every row outside
the class."""
import numpy as np
import torch

import r2_fixture as F


def _softmax_cr(rows: torch.Tensor) -> torch.Tensor:
    """max-subtracted f32 softmax with correctly rounded exps (f64 exp, one rounding), summed as 64
    lane partials of 4 then a halving tree, times the reciprocal: a valid f32 evaluation that shares
    no code with torch's."""
    l = rows.float()
    a = l - l.max(-1, keepdim=True).values
    e = torch.from_numpy(np.exp(a.double().numpy()).astype(np.float32))
    acc = e.view(-1, 4, 64).sum(1)
    n = 64
    while n > 1:
        n //= 2
        acc = acc[:, :n] + acc[:, n:2 * n]
    return e * (1.0 / acc[:, :1])


def test_fixture_has_near_equal_distinct_probabilities():
    rows = F.logit_rows(2048, seed=5)
    st = F.near_equal_stats(rows)
    assert st["distinct_equal_prob_pairs"] > 1000 and st["distinct_1ulp_pairs"] > 1000, st
    frag = F.fragile_rows(rows)
    assert 0.2 < frag.float().mean() < 1.0


def test_ids_outside_fragile_rows_do_not_depend_on_the_exp():
    rows = F.logit_rows(2048, seed=5)
    _, it = torch.topk(torch.softmax(rows.float(), dim=-1), 8, dim=-1)
    _, ic = torch.topk(_softmax_cr(rows), 8, dim=-1)
    differ = (it != ic).any(-1)
    frag = F.fragile_rows(rows)
    assert not (differ & ~frag).any(), "ids differ on a row the classifier calls robust"
    # the class is not empty of real differences: the two evaluations disagree somewhere inside it
    assert differ.any()
