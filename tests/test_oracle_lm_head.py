"""The lm_head oracle pinned: the reference's quoted band factors, its index rule, the Q8_0 decode
on hand-built blocks with closed-form values, and the f64 dot against an exact rational sum."""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ggml_quant as GQ
from oracle import lm_head_oracle as LO


def test_gamma_values_match_the_reference_quotes():
    # prototype/lm_head/HANDOFF.md:13-15 quotes gamma_2047 and gamma_4095 for K = 2048
    assert LO.gamma_of_index(2047) == pytest.approx(1.22025596e-04, rel=1e-8)
    assert LO.gamma_of_index(4095) == pytest.approx(2.4414061e-04, rel=1e-7)
    # ... and names 1.22085215e-04 as gamma_2048, the superseded index = K form
    assert LO.gamma_of_index(2048) == pytest.approx(1.22085215e-04, rel=1e-8)


def test_band_index_follows_the_measured_products():
    assert LO.gamma_index(2048, 0) == 2047
    assert LO.gamma_index(2048, 1) == 4095
    with pytest.raises(ValueError):
        LO.gamma_index(2048, None)
    rng = np.random.default_rng(0)
    # bf16 x bf16 products have <= 16 significant bits: exact in binary32 -> K - 1
    hb = LO.bf16_to_f32(rng.integers(0x3C00, 0x4000, size=(1, 2048), dtype=np.uint16))
    wb = LO.bf16_to_f32(rng.integers(0x3C00, 0x4000, size=(3, 2048), dtype=np.uint16))
    assert LO.lm_head(hb, wb)[2] == 2047
    # a full-width f32 hidden vector makes products inexact -> 2K - 1
    hf = rng.standard_normal((1, 2048)).astype(np.float32)
    assert LO.lm_head(hf, wb)[2] == 4095


def _q8_block(d: float, q) -> np.ndarray:
    b = np.zeros(34, dtype=np.uint8)
    b[0:2] = np.array([d], dtype=np.float16).view(np.uint8)
    b[2:34] = np.asarray(q, dtype=np.int8).view(np.uint8)
    return b


def test_q8_0_hand_blocks():
    q = np.arange(-16, 16)                                 # every sign, zero included
    blk = np.concatenate([_q8_block(0.5, q), _q8_block(-3.0, np.full(32, -128)),
                          _q8_block(2.0 ** -20, np.full(32, 127))])
    v = LO.dequant_q8_0(blk, 96)
    assert np.array_equal(v[:32], 0.5 * q.astype(np.float32))
    assert np.all(v[32:64] == 384.0)                       # -3 * -128
    assert np.all(v[64:] == np.float32(127 * 2.0 ** -20))  # subnormal-range f16 d stays exact
    # negative control: a decoder that forgot the sign (uint8 quants) is caught by these values
    wrong = 0.5 * blk[2:34].astype(np.float32)
    assert not np.array_equal(v[:32], wrong)


def test_q8_0_packer_roundtrip(pkg):
    w = torch.randn(8, 2048, generator=torch.Generator().manual_seed(4)) * 0.05
    qb = pkg.quant.quantize(w, pkg.quant.FMT_Q8_0).numpy()
    assert qb.shape == (8, 2176)
    dec = np.stack([LO.dequant_q8_0(r, 2048) for r in qb])
    err = np.abs(dec - w.numpy()).max()
    step = np.abs(w.numpy()).reshape(8, 64, 32).max(-1) / 127.0
    assert err <= 0.5 * step.max() * 1.01 + 1e-7          # round to nearest on the f16 step


def test_dot_against_exact_rationals():
    rng = np.random.default_rng(1)
    h = rng.standard_normal((2, 2048)).astype(np.float32)
    w = rng.standard_normal((3, 2048)).astype(np.float32)
    logits, band, n = LO.lm_head(h, w)
    for b in range(2):
        for j in range(3):
            exact = sum(Fraction(float(x)) * Fraction(float(y)) for x, y in zip(h[b], w[j]))
            assert abs(Fraction(float(logits[b, j])) - exact) <= Fraction(2.0 ** -40) * abs(exact) + Fraction(1, 10 ** 30)
            assert band[b, j] > 0 and n == 4095


def test_table_rows_formats(pkg):
    w = torch.randn(5, 2048, generator=torch.Generator().manual_seed(6)) * 0.02
    q6 = pkg.quant.quantize(w, pkg.quant.FMT_Q6_K).numpy()
    rows = np.array([4, 0, 2])
    got = LO.table_rows(q6, GQ.GGML_Q6_K, rows, 2048)
    for i, r in enumerate(rows):
        assert np.array_equal(got[i], GQ.dequant_q6k(q6[r], 2048))
    bf = w.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = LO.table_rows(bf, LO.FMT_BF16, rows, 2048)
    assert np.array_equal(got, w.to(torch.bfloat16).float().numpy()[rows])


def test_q8_0_oracle_shared_conversion(pkg):
    """from_device turns Q8_0 shared rows into the exact f32 values d * q the block oracle reads."""
    from oracle import moe_oracle as O
    lw = pkg.synth.make_layer(seed=3, device="cpu", n_experts=64, top_k=2, i_s=512,
                              shared_fmt=pkg.quant.FMT_Q8_0)
    ow = O.from_device(lw)
    assert ow.shared_gate.dtype == torch.float32 and tuple(ow.shared_gate.shape) == (512, 2048)
    assert tuple(ow.shared_down.shape) == (2048, 512)
    row = lw.shared_down[5].numpy()
    assert np.array_equal(ow.shared_down[5].numpy(), LO.dequant_q8_0(row, 512))
