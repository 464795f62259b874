"""Device super-block decode is bit-exact against the oracle decoders (moe_dequant entry point)."""
import numpy as np
import pytest
import torch

from oracle import ggml_quant as GQ

pytestmark = pytest.mark.gpu


def _bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    """f32 bit equality, with any NaN matching any NaN (random bytes can encode NaN scales)."""
    na, nb = np.isnan(a), np.isnan(b)
    if not np.array_equal(na, nb):
        return False
    return np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


def _random_blocks(nb, nbytes, seed, sane_scale_at=None):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(nb, nbytes), dtype=np.uint8)
    if sane_scale_at is not None:
        # keep half the blocks' f16 scales finite and moderate, so most values are ordinary
        for off in sane_scale_at:
            h = (rng.standard_normal(nb // 2) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
            raw[: nb // 2, off:off + 2] = h
    return raw


@pytest.mark.parametrize("fmt,nbytes,scales", [(GQ.GGML_Q4_K, 144, (0, 2)), (GQ.GGML_Q5_K, 176, (0, 2)),
                                                (GQ.GGML_Q6_K, 210, (208,))])
def test_dequant_random_bytes_bitexact(pkg, dev, fmt, nbytes, scales):
    nb = 4096
    raw = _random_blocks(nb, nbytes, seed=fmt, sane_scale_at=scales)
    want = GQ.dequant(raw, fmt, nb * 256)
    got = pkg.abi.dequant(torch.from_numpy(raw.reshape(-1)).to(dev), fmt, nb * 256).cpu().numpy()
    assert _bits_equal(got, want)


@pytest.mark.parametrize("fmt", [GQ.GGML_Q4_K, GQ.GGML_Q5_K, GQ.GGML_Q6_K])
def test_dequant_quantized_weights_bitexact_f32_and_bf16(pkg, dev, fmt):
    g = torch.Generator().manual_seed(5)
    w = torch.randn(512, 2048, generator=g) * 0.02
    q = pkg.quant.quantize(w, fmt)
    want = GQ.dequant(q.numpy(), fmt, w.numel())
    qd = q.reshape(-1).to(dev)
    got = pkg.abi.dequant(qd, fmt, w.numel()).cpu().numpy()
    assert _bits_equal(got, want)
    got_bf = pkg.abi.dequant(qd, fmt, w.numel(), out_dtype=torch.bfloat16).cpu()
    assert torch.equal(got_bf.view(torch.int16), torch.from_numpy(want).to(torch.bfloat16).view(torch.int16))


def test_dequant_q4k_hand_block(pkg, dev):
    """prototype/q4k_dequant/q4k_dequant.hip:435-462: d = dmin = 1, every 6-bit field 63;
    q = 0 -> -63 (0xC27C0000), q = 15 -> 882 (0x445C8000)."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x3C]
    blk[4:16] = 0xFF
    got0 = pkg.abi.dequant(torch.from_numpy(blk.copy()).to(dev), GQ.GGML_Q4_K, 256).cpu().numpy()
    blk[16:] = 0xFF
    got15 = pkg.abi.dequant(torch.from_numpy(blk.copy()).to(dev), GQ.GGML_Q4_K, 256).cpu().numpy()
    assert (got0.view(np.uint32) == 0xC27C0000).all()
    assert (got15.view(np.uint32) == 0x445C8000).all()


def test_dequant_refuses_bad_args(pkg, dev):
    blk = torch.zeros(144, dtype=torch.uint8, device=dev)
    with pytest.raises(pkg.Refused) as ei:
        pkg.abi.dequant(blk, 99, 256)
    assert ei.value.tag == "unsupported-format"


def test_dequant_q5k_hand_block(pkg, dev):
    """d = dmin = 1, every 6-bit field 63: all q = 0 -> -63, all q = 31 -> 1890; one qh bit
    (bit 3 of qh[5], element 101's 5th bit) with zero nibbles and mins -> only element 101 = 1008."""
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x3C]
    blk[4:16] = 0xFF
    got = pkg.abi.dequant(torch.from_numpy(blk.copy()).to(dev), GQ.GGML_Q5_K, 256).cpu().numpy()
    assert np.all(got == -63.0)
    blk[16:] = 0xFF
    got = pkg.abi.dequant(torch.from_numpy(blk.copy()).to(dev), GQ.GGML_Q5_K, 256).cpu().numpy()
    assert np.all(got == 1890.0)
    one = np.zeros(176, dtype=np.uint8)
    one[0:2] = [0x00, 0x3C]
    one[4:8] = 63                                     # sc[0..3] = 63, all mins 0
    one[12:16] = 0x0F                                 # sc[4..7] low bits 15 ...
    one[0 + 4:4 + 4] |= 0xC0                          # ... high bits 3 -> 63
    one[16 + 5] = 1 << 3
    got = pkg.abi.dequant(torch.from_numpy(one).to(dev), GQ.GGML_Q5_K, 256).cpu().numpy()
    assert np.nonzero(got)[0].tolist() == [101] and got[101] == 1008.0
    assert np.array_equal(got, GQ.dequant_q5k(one, 256))
