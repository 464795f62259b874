"""Untied lm_head GEMV (moe_lm_head) against the oracle: every output within the reference's band
gamma_n * sum_k |h_k w_k| of the exact dot (prototype/lm_head/gate.py:214-240), for Q6_K, Q8_0
and bf16 tables, dense and gather, 1..8 tokens, and the full 248320-row Q6_K table."""
import numpy as np
import pytest
import torch

from oracle import ggml_quant as GQ
from oracle import lm_head_oracle as LO

pytestmark = pytest.mark.gpu

H = 2048


def _table(pkg, fmt, V, seed):
    w = torch.randn(V, H, generator=torch.Generator().manual_seed(seed)) * 0.02
    if fmt == pkg._lib.MOE_FMT_BF16:
        t = w.to(torch.bfloat16)
        dec = t.float().numpy()
    else:
        t = pkg.quant.quantize(w, fmt)
        flat = t.numpy().reshape(-1)
        dec = (GQ.dequant_q6k(flat, V * H) if fmt == pkg._lib.MOE_FMT_Q6_K
               else LO.dequant_q8_0(flat, V * H)).reshape(V, H)
    return t, dec


def _check(got, h, dec_rows, tag):
    logits, band, n = LO.lm_head(h, dec_rows)
    g = got.cpu().double().numpy()
    ratio = np.abs(g - logits) / band
    print(f"{tag}: band index {n}, worst |got - exact| / band = {ratio.max():.3e}", flush=True)
    assert np.isfinite(g).all(), tag
    assert (ratio <= 1.0).all(), (tag, ratio.max())


@pytest.mark.parametrize("fmt_name", ["Q6_K", "Q8_0", "BF16"])
@pytest.mark.parametrize("B,hdt", [(1, torch.float32), (3, torch.float32), (8, torch.bfloat16)])
def test_lm_head_dense(pkg, dev, fmt_name, B, hdt):
    fmt = getattr(pkg._lib, "MOE_FMT_" + fmt_name)
    V = 5003                                           # not a multiple of the 16-row iteration
    t, dec = _table(pkg, fmt, V, seed=11)
    h = torch.randn(B, H, generator=torch.Generator().manual_seed(12 + B)).to(hdt)
    got = pkg.abi.lm_head(h.to(dev), t.to(dev), fmt)
    torch.cuda.synchronize()
    assert got.shape == (B, V)
    _check(got, h.float().numpy(), dec, f"dense {fmt_name} B={B} {hdt}")


@pytest.mark.parametrize("fmt_name", ["Q6_K", "Q8_0", "BF16"])
def test_lm_head_gather(pkg, dev, fmt_name):
    """Row ids with repeats, in any order, and ids outside [0, V) (NaN for those outputs)."""
    fmt = getattr(pkg._lib, "MOE_FMT_" + fmt_name)
    V = 1500
    t, dec = _table(pkg, fmt, V, seed=21)
    g = torch.Generator().manual_seed(22)
    ids = torch.randint(0, V, (301,), generator=g, dtype=torch.int32)
    ids[7] = ids[100]
    ids[50], ids[51], ids[52] = -1, V, V + 1000
    h = torch.randn(2, H, generator=g)
    got = pkg.abi.lm_head(h.to(dev), t.to(dev), fmt, row_ids=ids.to(dev))
    torch.cuda.synchronize()
    bad = np.array([50, 51, 52])
    assert torch.isnan(got[:, bad]).all()
    keep = np.setdiff1d(np.arange(301), bad)
    _check(got[:, keep], h.numpy(), dec[ids.numpy()[keep]], f"gather {fmt_name}")
    assert torch.equal(got[:, 7], got[:, 100])


def test_lm_head_full_vocab_q6k(pkg, dev):
    """The artifact's shape: 248320 x 2048 Q6_K (417 MB), one token. The reference side is the
    library's bit-exact dequant of the same bytes with an f64 GEMV on the GPU."""
    V = 248320
    g = torch.Generator(device=dev).manual_seed(31)
    t = pkg.quant.quantize(torch.randn(V, H, generator=g, device=dev) * 0.02, pkg._lib.MOE_FMT_Q6_K)
    h = torch.randn(1, H, generator=g, device=dev)
    got = pkg.abi.lm_head(h, t, pkg._lib.MOE_FMT_Q6_K)
    w = pkg.abi.dequant(t.reshape(-1), pkg._lib.MOE_FMT_Q6_K, V * H).view(V, H).double()
    exact = (h.double() @ w.T)
    band = LO.gamma_of_index(2 * H - 1) * (h.double().abs() @ w.abs().T)
    ratio = ((got.double() - exact).abs() / band).max().item()
    print(f"full vocab Q6_K: worst |got - exact| / band = {ratio:.3e}", flush=True)
    assert ratio <= 1.0
    # rows beyond the first iterations' stride pattern: a few spot rows against the CPU oracle
    rows = np.array([0, 15, 16, 123457, V - 1])
    dec = np.stack([GQ.dequant_q6k(t[r].cpu().numpy(), H) for r in rows])
    _check(got[:, rows], h.cpu().numpy(), dec, "full vocab Q6_K spot rows")


def test_lm_head_refusals(pkg, dev):
    t = torch.zeros(16, 1680, dtype=torch.uint8, device=dev)
    h = torch.zeros(1, 1024, device=dev)
    with pytest.raises(pkg.abi.Refused):
        pkg.abi.lm_head(h, t, pkg._lib.MOE_FMT_Q6_K)                  # H != 2048
    h = torch.zeros(9, 2048, device=dev)
    with pytest.raises(pkg.abi.Refused):
        pkg.abi.lm_head(h, t, pkg._lib.MOE_FMT_Q6_K)                  # B > 8
    with pytest.raises(pkg.abi.Refused):
        pkg.abi.lm_head(h[:1], t, pkg._lib.MOE_FMT_Q4_K)              # not a table format
