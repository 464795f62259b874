"""Pins of the oracle's post-attention RMSNorm (engine/m3_forward.py:303-307), CPU only.

The oracle defines r = f32(1 / sqrt(mean(x^2) + eps)) evaluated in f64 and rounded once. These
checks fix that definition from outside the oracle's own formula: an exact decimal evaluation of
the scale, closed forms on constant rows, exact power-of-two invariance, and closeness to the
reference's own f32 torch formula.
"""
from decimal import Decimal, getcontext

import numpy as np
import torch

from oracle import moe_oracle as O

H = 2048


def _f32(v: float) -> float:
    return float(np.float32(v))


def _exact_scale(row: torch.Tensor, eps: float) -> float:
    """1/sqrt(sum(x^2)/H + eps) to 60 digits, then rounded to f32 (round-half-even through the
    f64 nearest, which is exact at this precision for all but measure-zero inputs)."""
    getcontext().prec = 60
    ss = sum(Decimal(float(v)) * Decimal(float(v)) for v in row.tolist())
    val = Decimal(1) / (ss / Decimal(row.numel()) + Decimal(eps)).sqrt()
    return _f32(float(val))


def test_scale_is_the_correctly_rounded_exact_value():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(6, H, generator=g) * torch.tensor([1e-3, 0.5, 1.0, 3.0, 40.0, 1e3]).view(6, 1)
    w = torch.ones(H)
    for eps in (1e-6, 0.0):
        xn = O.rmsnorm_a(x, w, eps)
        for t in range(x.shape[0]):
            r = np.float32(_exact_scale(x[t], eps))
            want = (x[t].numpy().astype(np.float32) * r).astype(np.float32)
            assert np.array_equal(xn[t].numpy().view(np.uint32), want.view(np.uint32)), (eps, t)


def test_association_is_x_times_r_then_times_w():
    """Form A is (x * r) * w (engine/m3_forward.py:303-307), two f32 roundings in that order. With
    r from the exact decimal scale and w not a power of two, the bits are fixed, and the other
    association x * (r * w) differs on a share of the elements (negative control)."""
    g = torch.Generator().manual_seed(14)
    x = torch.randn(4, H, generator=g) * 1.7
    w = (1.0 + 0.3 * torch.randn(H, generator=g)).float()
    eps = 1e-6
    xn = O.rmsnorm_a(x, w, eps)
    wn = w.numpy().astype(np.float32)
    n_other = 0
    for t in range(x.shape[0]):
        r = np.float32(_exact_scale(x[t], eps))
        xr = (x[t].numpy().astype(np.float32) * r).astype(np.float32)
        want = (xr * wn).astype(np.float32)
        assert np.array_equal(xn[t].numpy().view(np.uint32), want.view(np.uint32)), t
        other = (x[t].numpy().astype(np.float32) * (r * wn).astype(np.float32)).astype(np.float32)
        n_other += int((other.view(np.uint32) != want.view(np.uint32)).sum())
    assert n_other > 0.05 * x.numel()


def test_constant_rows_closed_form():
    w = torch.linspace(0.5, 1.5, H)
    # x = 2^k: r = 2^-k exactly, so the output is exactly sign(x) * w
    for c in (2.0 ** -6, 1.0, 4.0, -8.0):
        xn = O.rmsnorm_a(torch.full((1, H), c), w, 0.0)
        assert torch.equal(xn[0], w * (1.0 if c > 0 else -1.0)), c
    # x = 3: r = f32(1/3), output = f32(3 * f32(1/3)) * w
    r = np.float32(_f32(1.0 / 3.0))
    xn = O.rmsnorm_a(torch.full((1, H), 3.0), w, 0.0)
    want = (np.float32(3.0) * r) * w.numpy()
    assert np.array_equal(xn[0].numpy(), want.astype(np.float32))


def test_power_of_two_scaling_is_exact():
    g = torch.Generator().manual_seed(12)
    x = torch.randn(4, H, generator=g)
    w = 1.0 + 0.1 * torch.randn(H, generator=g)
    base = O.rmsnorm_a(x, w, 0.0)
    for k in (-20, -3, 5, 30):
        assert torch.equal(O.rmsnorm_a(x * 2.0 ** k, w, 0.0), base), k


def test_close_to_the_reference_f32_formula():
    """The reference's own arithmetic (torch f32 mean and rsqrt) differs only in the last bits."""
    g = torch.Generator().manual_seed(13)
    x = torch.randn(8, H, generator=g) * 2.0
    w = 1.0 + 0.1 * torch.randn(H, generator=g)
    eps = 1e-6
    ref = (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)) * w
    ours = O.rmsnorm_a(x, w, eps)
    ulp = torch.finfo(torch.float32).eps
    assert ((ours - ref).abs() <= 3 * ulp * ref.abs() + 1e-30).all()


def test_residual_step_is_x_plus_block_of_the_normalized_input():
    """residual_step = x1 + moe_block(rmsnorm_a(x1)) with the block evaluated on the normed rows."""
    import test_oracle_block as TB
    lw = TB._layer(5)
    g = torch.Generator().manual_seed(14)
    x1 = torch.randn(3, TB.H, generator=g) * 3.0
    w = 1.0 + 0.1 * torch.randn(TB.H, generator=g)
    st = O.residual_step(x1, lw, w, 1e-6)
    blk = O.moe_block(O.rmsnorm_a(x1, w, 1e-6), lw)
    assert torch.equal(st["x_out"], x1 + blk["combined_out"])
    assert torch.equal(st["topk_ids"], blk["topk_ids"])
