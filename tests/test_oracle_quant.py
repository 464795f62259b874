"""Pins of the oracle's Q4_K / Q5_K / Q6_K decoders (CPU only). Each check is chosen so a plausible
mistake fails it: a swapped scale/min field, a wrong nibble or sub-block index, a dropped min
term, a wrong Q6_K bit shift, a double rounding."""
import numpy as np
import pytest

from oracle import ggml_quant as GQ


def test_f16_decode_exhaustive():
    """All 65,536 binary16 patterns -> the IEEE value (Python's struct 'e' as the independent
    reference; NaNs compared as NaN)."""
    import struct
    bits = np.arange(65536, dtype=np.uint16)
    got = GQ.f16_to_f64(bits)
    ref = np.array([struct.unpack("<e", struct.pack("<H", int(b)))[0] for b in bits])
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])
    # hand-worked points (prototype/q4k_dequant/q4k_dequant.hip:365-381)
    assert GQ.f16_to_f64(np.array([0x7BFF], dtype=np.uint16))[0] == 65504.0
    assert GQ.f16_to_f64(np.array([0x0001], dtype=np.uint16))[0] == 2.0 ** -24
    assert GQ.f16_to_f64(np.array([0x03FF], dtype=np.uint16))[0] == 1023 * 2.0 ** -24


def _bit_unpack(scales: bytes, j: int):
    """Independent route: read the 96-bit field as a bit string. j < 4: sc = bits [8j, 8j+6),
    m = bits [32+8j, 32+8j+6). j >= 4: low 4 bits from byte 8+(j-4) (sc low nibble, m high
    nibble), high 2 bits from the top 2 bits of byte j-4 (sc) / byte j (m)."""
    b = list(scales)
    bit = lambda i: (b[i // 8] >> (i % 8)) & 1
    if j < 4:
        sc = sum(bit(8 * j + i) << i for i in range(6))
        m = sum(bit(32 + 8 * j + i) << i for i in range(6))
    else:
        k = j - 4
        sc = sum(bit(8 * (8 + k) + i) << i for i in range(4)) | (bit(8 * k + 6) << 4) | (bit(8 * k + 7) << 5)
        m = sum(bit(8 * (8 + k) + 4 + i) << i for i in range(4)) | (bit(8 * j + 6) << 4) | (bit(8 * j + 7) << 5)
    return sc, m


def test_scale_min_every_byte_pair_vs_bit_unpack():
    """Every field j depends on two bytes; sweep both over all 256 x 256 values."""
    v = np.arange(256, dtype=np.uint8)
    a, b = np.meshgrid(v, v, indexing="ij")
    a, b = a.reshape(-1), b.reshape(-1)
    for j in range(8):
        s = np.zeros((a.size, 12), dtype=np.uint8)
        if j < 4:
            s[:, j], s[:, j + 4] = a, b
        else:
            s[:, j + 4], s[:, j - 4] = a, b           # low nibbles / sc high bits
        sc, m = GQ.q4k_scale_min(s)
        for idx in (0, 1, 255, 256 * 171 + 3, 65535, 256 * 64 + 200):
            assert (sc[idx, j], m[idx, j]) == _bit_unpack(bytes(s[idx]), j)
        # m high bits for j >= 4 come from byte j: sweep that byte too
        if j >= 4:
            s2 = np.zeros((a.size, 12), dtype=np.uint8)
            s2[:, j + 4], s2[:, j] = a, b
            sc2, m2 = GQ.q4k_scale_min(s2)
            want = np.array([_bit_unpack(bytes(r), j) for r in s2[::257]])
            assert np.array_equal(np.stack([sc2[::257, j], m2[::257, j]], 1), want)


def test_scale_min_reference_vectors():
    """prototype/q4k_dequant/q4k_dequant.hip:383-433, hand-worked get_scale_min_k4 vectors."""
    q = np.array([[1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12]], dtype=np.uint8)
    sc, m = GQ.q4k_scale_min(q)
    assert sc[0].tolist() == [1, 2, 3, 4, 9, 10, 11, 12]
    assert m[0].tolist() == [5, 6, 7, 8, 0, 0, 0, 0]
    q[0, 0], q[0, 4], q[0, 3] = 0x41, 0x45, 0x84
    sc, m = GQ.q4k_scale_min(q)
    assert (sc[0, 4], m[0, 4]) == (25, 16)
    assert (sc[0, 7], m[0, 7]) == (44, 0)


def _hand_block(qs_byte: int) -> np.ndarray:
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]      # d = 1.0
    blk[2:4] = [0x00, 0x3C]      # dmin = 1.0
    blk[4:16] = 0xFF             # every 6-bit field 63
    blk[16:] = qs_byte
    return blk


def test_q4k_hand_block_kats():
    """prototype/q4k_dequant/q4k_dequant.hip:435-462: q = 0 -> -63 (0xC27C0000),
    q = 15 -> 882 (0x445C8000); dropping the min would give 945 (0x446C4000)."""
    v0 = GQ.dequant_q4k(_hand_block(0x00), 256)
    v15 = GQ.dequant_q4k(_hand_block(0xFF), 256)
    assert (v0.view(np.uint32) == 0xC27C0000).all()
    assert (v15.view(np.uint32) == 0x445C8000).all()
    assert not (v15.view(np.uint32) == 0x446C4000).any()


def test_q4k_subblock_witness_element_33():
    """prototype/q4k_dequant/q4k_dequant_kernels.h:199-203: d = 1, dmin = 0, scales[1] = 63 (so
    sc[1] = 63, every other 6-bit field 0), a low nibble 15 in qs[32g] and a high nibble 15 in
    qs[32g+1]: only element 33 (high nibble of byte 1 = sub-block 1) is non-zero, = 945. A
    decoder that put high nibbles in the same sub-block as low ones would light element 1."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[5] = 63
    for g in range(4):
        blk[16 + 32 * g] = 0x0F
        blk[16 + 32 * g + 1] = 0xF0
    v = GQ.dequant_q4k(blk, 256)
    nz = np.nonzero(v)[0].tolist()
    assert nz == [33] and v[33] == 945.0


def _pack_q4k_fields(d, dmin, sc, m, q):
    """Encoder route from the fields (tools/audit_published_quant.py:1007-1040 shape)."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.array([d], dtype=np.float16).view(np.uint8)
    blk[2:4] = np.array([dmin], dtype=np.float16).view(np.uint8)
    s = np.zeros(12, dtype=np.int64)
    for j in range(4):
        s[j] = sc[j] & 63
        s[j + 4] = m[j] & 63
    for j in range(4, 8):
        s[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (m[j] >> 4) << 6
    blk[4:16] = s.astype(np.uint8)
    for g in range(4):
        for l in range(32):
            blk[16 + 32 * g + l] = q[64 * g + l] | (q[64 * g + 32 + l] << 4)
    return blk


def test_q4k_fields_roundtrip_vs_affine_definition():
    """value(e) = d*sc[e//32]*q[e] - dmin*m[e//32] from the fields, 200 random blocks."""
    rng = np.random.default_rng(0)
    for _ in range(200):
        d = float(np.float16(rng.uniform(1e-4, 0.1)))
        dmin = float(np.float16(rng.uniform(1e-4, 0.1)))
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        got = GQ.dequant_q4k(_pack_q4k_fields(d, dmin, sc, m, q), 256)
        want = np.array([np.float32(d * sc[e // 32] * q[e] - dmin * m[e // 32]) for e in range(256)],
                        dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q4k_f32_route_equals_f64_route_when_scales_are_close():
    """The single f32 rounding equals the reference's f64-then-f32 route (tools/gguf_fast_dequant.py
    :115-125) whenever the f64 difference is exact; realistic blocks (packed weights)."""
    import torch
    import importlib.util, sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("q_", root / "qwen3.6-35b-a3b_amd" / "quant.py")
    Q = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(Q)
    w = torch.randn(64, 2048, generator=torch.Generator().manual_seed(1)) * 0.02
    raw = Q.quantize(w, Q.FMT_Q4_K).numpy().reshape(-1, 144)
    got = GQ.dequant_q4k(raw, raw.shape[0] * 256)
    d = GQ.f16_to_f64(raw[:, 0:2].copy().view(np.uint16).reshape(-1))
    dmin = GQ.f16_to_f64(raw[:, 2:4].copy().view(np.uint16).reshape(-1))
    sc, m = GQ.q4k_scale_min(raw[:, 4:16])
    qs = raw[:, 16:].reshape(-1, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).astype(np.float64)
    f64 = (d.reshape(-1, 1, 1, 1) * sc.reshape(-1, 4, 2, 1)) * q - dmin.reshape(-1, 1, 1, 1) * m.reshape(-1, 4, 2, 1)
    assert np.array_equal(got, f64.reshape(-1).astype(np.float32))


def _pack_q6k_fields(d, sc, q):
    """tools/audit_published_quant.py:1083-1103 packing order (ql / qh / int8 scales / d)."""
    blk = np.zeros(210, dtype=np.uint8)
    for half in range(2):
        j = 128 * half
        for l in range(32):
            blk[64 * half + l] = (q[j + l] & 15) | ((q[j + l + 64] & 15) << 4)
            blk[64 * half + l + 32] = (q[j + l + 32] & 15) | ((q[j + l + 96] & 15) << 4)
            blk[128 + 32 * half + l] = ((q[j + l] >> 4) | ((q[j + l + 32] >> 4) << 2)
                                        | ((q[j + l + 64] >> 4) << 4) | ((q[j + l + 96] >> 4) << 6))
    blk[192:208] = np.array(sc, dtype=np.int8).view(np.uint8)
    blk[208:210] = np.array([d], dtype=np.float16).view(np.uint8)
    return blk


def test_q6k_fields_roundtrip_vs_affine_definition():
    """value(e) = d * sc[e//16] * (q[e] - 32); the reference has no hand-worked Q6_K KAT, so the
    packer route of tools/audit_published_quant.py:1083-1114 is the pin."""
    rng = np.random.default_rng(1)
    for _ in range(200):
        d = float(np.float16(rng.uniform(-0.01, 0.01)))
        sc = rng.integers(-128, 128, 16)
        q = rng.integers(0, 64, 256)
        got = GQ.dequant_q6k(_pack_q6k_fields(d, sc, q), 256)
        want = np.array([np.float32(d * sc[e // 16] * (q[e] - 32)) for e in range(256)], dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q6k_products_exact_in_f32():
    """d*sc*(q-32) needs <= 23 significant bits: the f32 product equals the exact f64 one for every
    (sc, q) pair and a sweep of f16 d values (normal and subnormal)."""
    sc = np.arange(-128, 128, dtype=np.float64)[:, None]
    qq = (np.arange(64, dtype=np.float64) - 32)[None, :]
    for dbits in list(range(1, 1024, 97)) + list(range(0x0400, 0x7BFF, 1531)):
        d = GQ.f16_to_f64(np.array([dbits], dtype=np.uint16))[0]
        exact = (d * sc) * qq
        f32 = (np.float32(d) * sc.astype(np.float32)) * qq.astype(np.float32)
        assert np.array_equal(exact.astype(np.float32), f32)
        assert np.array_equal(exact, f32.astype(np.float64))


def test_q6k_negative_control_wrong_shift_is_caught():
    """A decoder that took the high bits with shift k instead of 2k would differ: the round trip
    above must be able to fail."""
    rng = np.random.default_rng(2)
    q = rng.integers(0, 64, 256)
    blk = _pack_q6k_fields(0.5, rng.integers(1, 100, 16), q)
    good = GQ.dequant_q6k(blk, 256)
    bad = blk.copy()
    bad[128:192] = np.roll(bad[128:192], 1)
    assert not np.array_equal(GQ.dequant_q6k(bad, 256), good)


def _pack_q5k_fields(d, dmin, sc, m, q):
    """Encoder route for Q5_K from the fields (the packing order of tools/audit_published_quant.py
    :1047-1072): the Q4_K scale bytes, the low 4 bits of q as Q4_K nibbles, and the 5th bit of
    element 64n + j at bit 2n of qh[j], of element 64n + 32 + j at bit 2n + 1."""
    blk = np.zeros(176, dtype=np.uint8)
    head = _pack_q4k_fields(d, dmin, sc, m, np.asarray(q) & 15)
    blk[0:16] = head[0:16]
    blk[48:176] = head[16:144]
    for n in range(4):
        for j in range(32):
            if q[64 * n + j] > 15:
                blk[16 + j] |= 1 << (2 * n)
            if q[64 * n + 32 + j] > 15:
                blk[16 + j] |= 2 << (2 * n)
    return blk


def test_q5k_fields_roundtrip_vs_affine_definition():
    """value(e) = d*sc[e//32]*q[e] - dmin*m[e//32], q in [0, 31], rounded once to f32
    (tools/audit_published_quant.py:1036-1044 `expect_k`), 200 random blocks."""
    rng = np.random.default_rng(5)
    for _ in range(200):
        d = float(np.float16(rng.uniform(1e-4, 0.1)))
        dmin = float(np.float16(rng.uniform(1e-4, 0.1)))
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 32, 256)
        got = GQ.dequant_q5k(_pack_q5k_fields(d, dmin, sc, m, q), 256)
        want = np.array([np.float32(d * sc[e // 32] * q[e] - dmin * m[e // 32]) for e in range(256)],
                        dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q5k_hand_blocks():
    """Closed forms with d = dmin = 1 and every 6-bit field 63: q = 0 -> -63, q = 31 -> 1890
    (63 * 31 - 63), and a single qh bit: bit 3 of qh[5] is element 32*3 + 5 = 101's 5th bit, so
    with all nibbles 0 and all mins 0 exactly that element reads 63 * 16 = 1008."""
    blk = np.zeros(176, dtype=np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x3C]
    blk[4:16] = 0xFF
    assert np.all(GQ.dequant_q5k(blk, 256) == -63.0)
    blk[16:] = 0xFF
    assert np.all(GQ.dequant_q5k(blk, 256) == 1890.0)
    one = np.zeros(176, dtype=np.uint8)
    one[0:2] = [0x00, 0x3C]
    one[4:16] = _pack_q4k_fields(1.0, 0.0, [63] * 8, [0] * 8, [0] * 256)[4:16]
    one[16 + 5] = 1 << 3
    v = GQ.dequant_q5k(one, 256)
    assert np.nonzero(v)[0].tolist() == [101] and v[101] == 1008.0


def test_q5k_negative_control_wrong_high_bit_is_caught():
    """A decoder that took the 5th bit from the wrong qh byte (or bit) would differ: the round
    trip above must be able to fail."""
    rng = np.random.default_rng(6)
    q = rng.integers(0, 32, 256)
    blk = _pack_q5k_fields(0.5, 0.25, rng.integers(1, 64, 8), rng.integers(0, 64, 8), q)
    good = GQ.dequant_q5k(blk, 256)
    bad = blk.copy()
    bad[16:48] = np.roll(bad[16:48], 1)
    assert not np.array_equal(GQ.dequant_q5k(bad, 256), good)
    bad2 = blk.copy()
    bad2[16:48] = (bad2[16:48].astype(np.int64) << 1 & 0xFF).astype(np.uint8)
    assert not np.array_equal(GQ.dequant_q5k(bad2, 256), good)


def test_q5k_packer_roundtrip_and_f64_route():
    """The package's Q5_K packer: its bytes decode (oracle) to the f64 route's values rounded once,
    and the fit is the finer one a 5-bit code gives."""
    import torch
    import importlib.util
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("q_", root / "qwen3.6-35b-a3b_amd" / "quant.py")
    Q = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(Q)
    w = torch.randn(64, 2048, generator=torch.Generator().manual_seed(7)) * 0.02
    raw = Q.quantize(w, Q.FMT_Q5_K).numpy().reshape(-1, 176)
    got = GQ.dequant_q5k(raw, raw.shape[0] * 256)
    d = GQ.f16_to_f64(raw[:, 0:2].copy().view(np.uint16).reshape(-1))
    dmin = GQ.f16_to_f64(raw[:, 2:4].copy().view(np.uint16).reshape(-1))
    sc, m = GQ.q4k_scale_min(raw[:, 4:16])
    qh = raw[:, 16:48].astype(np.int64)
    qs = raw[:, 48:].reshape(-1, 4, 32).astype(np.int64)
    q = np.stack([qs & 15, qs >> 4], axis=2)
    for j in range(8):
        q[:, j // 2, j % 2, :] += 16 * ((qh >> j) & 1)
    assert q.max() > 15                               # the 5th bit is in use
    f64 = (d.reshape(-1, 1, 1, 1) * sc.reshape(-1, 4, 2, 1)) * q - dmin.reshape(-1, 1, 1, 1) * m.reshape(-1, 4, 2, 1)
    assert np.array_equal(got, f64.reshape(-1).astype(np.float32))
    # the 5th bit halves the quantisation step: the Q5_K fit's RMS error must be well under the
    # Q4_K fit's on the same weights (a misplaced 5th bit would not be)
    wv = w.numpy().reshape(-1).astype(np.float64)
    e5 = np.sqrt(np.mean((got.astype(np.float64) - wv) ** 2))
    r4 = Q.quantize(w, Q.FMT_Q4_K).numpy().reshape(-1, 144)
    e4 = np.sqrt(np.mean((GQ.dequant_q4k(r4, r4.shape[0] * 256).astype(np.float64) - wv) ** 2))
    assert e5 < 0.6 * e4 and e5 < 0.08 * np.sqrt(np.mean(wv ** 2)), (e5, e4)
