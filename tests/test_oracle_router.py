"""Pins of the router oracle (CPU only): the libstdc++ topk model vs torch.topk, the device's
rank-based partition vs the sequential partition, the correctly rounded R1 vs exact rationals."""
import random
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from oracle import topk_model as TM


def _tie_rows(n_rows, seed):
    rng = random.Random(seed)
    rows = []
    for i in range(n_rows):
        kind = i % 3
        if kind == 0:
            nd = rng.randint(1, 20)
            rows.append([float(rng.randint(0, nd)) for _ in range(256)])
        elif kind == 1:
            lg = (torch.randn(256, generator=torch.Generator().manual_seed(seed * 1000 + i)) * 0.9)
            rows.append(torch.softmax(lg.to(torch.bfloat16).float(), -1).tolist())
        else:
            lg = torch.randn(256, generator=torch.Generator().manual_seed(seed * 1000 + i))
            lg = torch.round(lg * 8) / 8
            rows.append(torch.softmax(lg, -1).tolist())
    return rows


def test_topk_model_matches_torch_on_tie_laden_rows():
    rows = _tie_rows(1500, seed=3)
    t = torch.tensor(rows, dtype=torch.float32)
    _, ids = torch.topk(t, 8, dim=-1)
    for r, row in enumerate(t.tolist()):
        got, _ = TM.torch_cpu_topk(row, 8)
        assert got == ids[r].tolist(), r


def test_topk_model_heap_select_branch_matches_torch():
    for start in (None, -40.0):
        vals = TM.adversarial_row(256, 8, start=start)
        got, heap = TM.torch_cpu_topk(vals, 8)
        assert heap
        assert got == torch.topk(torch.tensor(vals), 8).indices.tolist()


def test_lower_index_rule_is_not_torchs_order():
    """Negative control: 'ties by lower index' (the moe_ref.py:342 comment) disagrees with torch
    on tie-laden rows, so a kernel using it would fail the device tests."""
    rows = _tie_rows(300, seed=5)
    t = torch.tensor(rows)
    _, ids = torch.topk(t, 8, dim=-1)
    lower = torch.tensor([sorted(range(256), key=lambda i: (-row[i], i))[:8] for row in rows])
    assert (lower != ids).any(dim=-1).sum() > 10


# ---------------------------------------------------------------- the device's partition model
def _rank_partition(v, a, b, pivot):
    """Python model of wave_partition (router.hip): A = positions in [a,b) with value <= pivot
    (left stops) ascending, B = positions with value >= pivot (right stops) descending; swap
    A[m] <-> B[m] while A[m] < B[m]; return min(A[M], B[M-1])."""
    A = [p for p in range(a, b) if not v[p] > pivot]
    B = [p for p in range(b - 1, a - 1, -1) if not pivot > v[p]]
    M = 0
    while M < min(len(A), len(B)) and A[M] < B[M]:
        M += 1
    out = list(v)
    for m in range(M):
        out[A[m]], out[B[m]] = v[B[m]], v[A[m]]
    cands = []
    if M < len(A):
        cands.append(A[M])
    if M >= 1:
        cands.append(B[M - 1])
    return out, min(cands)


def _rank_partition_ballots(v, a, b, pivot):
    """Same, computed the way the kernel does: per-position counts from prefix sums only."""
    n = len(v)
    isA = [a <= p < b and not v[p] > pivot for p in range(n)]
    isB = [a <= p < b and not pivot > v[p] for p in range(n)]
    cA = np.cumsum([0] + isA)           # cA[p] = # A positions < p
    totB = sum(isB)
    cB = np.cumsum([0] + isB)
    rankA = [int(cA[p]) for p in range(n)]
    rankB = [int(totB - cB[p + 1]) for p in range(n)]     # # B positions > p
    swA = [isA[p] and rankB[p] > rankA[p] for p in range(n)]
    swB = [isB[p] and rankA[p] > rankB[p] for p in range(n)]
    M = sum(swA)
    assert M == sum(swB)
    pa, pb = {}, {}
    for p in range(n):
        if swA[p]:
            pa[rankA[p]] = p
        if swB[p]:
            pb[rankB[p]] = p
    out = list(v)
    for p in range(n):
        if swA[p]:
            out[p] = v[pb[rankA[p]]]
        if swB[p]:
            out[p] = v[pa[rankB[p]]]
    cells = [p for p in range(n) if isA[p] and rankA[p] == M] + \
            [p for p in range(n) if isB[p] and rankB[p] == M - 1]
    return out, min(min(cells), b)


def test_rank_partition_equals_sequential_unguarded_partition():
    rng = random.Random(7)
    for trial in range(3000):
        n = 256
        nd = rng.choice([2, 3, 5, 20, 1000])
        v = [float(rng.randint(0, nd)) for _ in range(n)]
        lo = rng.randint(0, 200)
        hi = rng.randint(lo + 4, n)
        row = TM._Row(v)
        mid = lo + (hi - lo) // 2
        row.median_to_first(lo, lo + 1, mid, hi - 1)
        vv = [v[i] for i in row.q]
        cut_seq = row.partition(lo + 1, hi, lo)
        seq_vals = [v[i] for i in row.q]
        got, cut = _rank_partition(vv, lo + 1, hi, vv[lo])
        got2, cut2 = _rank_partition_ballots(vv, lo + 1, hi, vv[lo])
        assert cut == cut_seq == cut2, trial
        assert got == seq_vals == got2, trial


# --------------------------------------------------------------------------------------- R1
def _exact_logits(x, w, bias=None):
    out = []
    for t in range(x.shape[0]):
        row = []
        for e in range(w.shape[0]):
            acc = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x[t].tolist(), w[e].tolist()))
            if bias is not None:
                acc += Fraction(float(bias[e]))
            row.append(O._round_to_bf16_exact(acc))
        out.append(row)
    return torch.tensor(out, dtype=torch.float32).to(torch.bfloat16)


def test_r1_matches_exact_rational_rounding():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 64, generator=g)
    w = (torch.randn(16, 64, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(16, generator=g)
    for bias in (None, b):
        got, _ = O.r1_logits(x, w, bias)
        assert torch.equal(got.view(torch.int16), _exact_logits(x, w, bias).view(torch.int16))


def test_r1_midpoints_go_through_the_exact_path():
    """1 + 2^-8 is a bf16 midpoint: ties to even -> 1.0; 1 + 2^-8 + 2^-40 -> 1 + 2^-7; a
    midpoint between odd and even neighbours (1 + 3*2^-8) -> 1 + 2^-6 (even)."""
    x = torch.tensor([[1.0, 2.0 ** -8, 0.0], [1.0, 2.0 ** -8, 2.0 ** -40], [1.0, 3 * 2.0 ** -8, 0.0]])
    w = torch.ones(4, 3, dtype=torch.bfloat16)
    got, n_exact = O.r1_logits(x, w)
    assert n_exact == 8        # two exact midpoints, four experts each
    assert got[0].float().tolist() == [1.0] * 4
    assert got[1].float().tolist() == [1.0 + 2.0 ** -7] * 4
    assert got[2].float().tolist() == [1.0 + 2.0 ** -6] * 4


def test_r1_is_not_torch_bf16_linear():
    """The f64 -> bf16 single rounding differs from rounding an f32 sum on some logits: the
    oracle must not silently be F.linear-then-cast."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(256, 2048, generator=g)
    w = (torch.randn(256, 2048, generator=g) * 0.02).to(torch.bfloat16)
    got, _ = O.r1_logits(x, w)
    f32 = (x @ w.float().T).to(torch.bfloat16)
    assert (got.view(torch.int16) != f32.view(torch.int16)).sum() > 0


def test_route_invariants():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(32, 2048, generator=g)
    w = (torch.randn(256, 2048, generator=g) * 0.02).to(torch.bfloat16)
    r = O.route(x, w, 8)
    wf = r["topk_weights_f32"]
    assert torch.all((wf.sum(-1) - 1).abs() <= 8 * 2.0 ** -24)
    assert torch.all(wf[:, :-1] >= wf[:, 1:])
    assert torch.all((r["router_probs"] > 0) & (r["router_probs"] <= 1))
    # closed form: the renormalised weights are softmax over the 8 selected logits
    sel = torch.gather(r["router_logits"].float(), 1, r["topk_ids"])
    assert torch.allclose(wf, torch.softmax(sel.double(), -1).float(), rtol=1e-5, atol=0)
