"""Near-equal-probability rows for the R2 softmax (speccheck/moe_ref.py:338; tie evidence
prototype/moe_router/results.md:73-88). Test data only.

Distinct bf16 logits normally give probabilities many f32 ulps apart: two neighbours at a logit of
magnitude 2^e differ by 2^(e-7), so their probabilities differ by a factor 1 + 2^(e-7). Only logits
within about 2^-16 of each other land within one f32 ulp, and then whether two probabilities come
out equal depends on the last bit of each exp and of the shared reciprocal. These rows put 12
candidates at or near zero (from a pool of 0 and +-2^-k, k = 14..32, and their multiples by 3), so
that distinct logits in the top 9 sit 0-8 ulps apart, exact repeats included; the other 244 logits
are far below (about -2), so only the near-zero group competes for the top 8.
"""
from __future__ import annotations

import torch

E = 256
N_NEAR = 12


def near_zero_pool() -> torch.Tensor:
    v = [0.0]
    for k in range(14, 33):
        for m in (1.0, 3.0):
            v += [m * 2.0 ** -k, -m * 2.0 ** -k]
    return torch.tensor(v, dtype=torch.float32).to(torch.bfloat16)


def logit_rows(n_rows: int, seed: int) -> torch.Tensor:
    """[n_rows, E] bf16 logits: 12 near-zero candidates at random expert positions, the rest
    ~ N(-2, 0.5) in bf16."""
    g = torch.Generator().manual_seed(seed)
    pool = near_zero_pool()
    rows = (torch.randn(n_rows, E, generator=g) * 0.5 - 2.0).to(torch.bfloat16)
    for r in range(n_rows):
        pos = torch.randperm(E, generator=g)[:N_NEAR]
        rows[r, pos] = pool[torch.randint(0, len(pool), (N_NEAR,), generator=g)]
    return rows


def near_equal_stats(rows: torch.Tensor) -> dict:
    """Among each row's top 9 (torch CPU softmax + topk), count pairs of DISTINCT logits whose
    probabilities are equal, and pairs one f32 ulp apart."""
    p = torch.softmax(rows.float(), dim=-1)
    vals, ids = torch.topk(p, 9, dim=-1)
    lg = torch.gather(rows.float(), 1, ids)
    bits = vals.view(torch.int32)
    n_eq = n_1ulp = 0
    for i in range(9):
        for j in range(i + 1, 9):
            distinct = lg[:, i] != lg[:, j]
            d = (bits[:, i] - bits[:, j]).abs()
            n_eq += int((distinct & (d == 0)).sum())
            n_1ulp += int((distinct & (d == 1)).sum())
    return {"distinct_equal_prob_pairs": n_eq, "distinct_1ulp_pairs": n_1ulp}


def fragile_rows(rows: torch.Tensor, ulps: int = 2) -> torch.Tensor:
    """bool [n_rows]: rows whose top 9 (torch CPU softmax + topk) hold two DISTINCT logits with
    probabilities at most `ulps` f32 ulps apart, equal included. Outside these rows every valid f32
    evaluation of the softmax orders the candidates the same way (distinct probabilities further
    apart than the evaluation error, equal logits equal everywhere), so the ids are fixed; inside
    them the ids depend on the last bit of each exp and of the shared reciprocal."""
    p = torch.softmax(rows.float(), dim=-1)
    vals, ids = torch.topk(p, 9, dim=-1)
    lg = torch.gather(rows.float(), 1, ids)
    bits = vals.view(torch.int32)
    out = torch.zeros(rows.shape[0], dtype=torch.bool)
    for i in range(9):
        for j in range(i + 1, 9):
            out |= (lg[:, i] != lg[:, j]) & ((bits[:, i] - bits[:, j]).abs() <= ulps)
    return out
