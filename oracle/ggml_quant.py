"""Q4_K / Q6_K super-block decoders (CPU, numpy) — test infrastructure, see oracle/__init__.py.

Restated from the GGUF block format as the reference reads it:
  * Q4_K: tools/gguf_reader.py:17-51 (layout), :165-175 (`qk_scale_min`), :248-268 (`_deq_q4_k`);
    tools/gguf_fast_dequant.py:75-125 (vectorized route, association `ds = d*sc` then
    `ds*q - dmin*m`, one cast to f32).
  * Q6_K: tools/gguf_reader.py:42-48, :299-322 (`_deq_q6_k`); tools/gguf_fast_dequant.py:126-145.
  * llama.cpp / ggml (commit d327bf1f, tag b11869, not vendored) defines both formats in
    ggml-common.h and ggml-quants.c (`dequantize_row_q4_K`, `dequantize_row_q6_K`,
    `get_scale_min_k4`); tools/gguf_reader.py:10-15 names that pin.

Exactness. Every factor of a Q4_K element (f16 d and dmin, 6-bit sc and m, 4-bit q) is exact in
f32 and so is each product (d*sc <= 17 significant bits, *q <= 21, dmin*m <= 17), so the value is
the f32 subtraction (d*sc)*q - dmin*m with its single rounding — the correctly rounded f32 of the
exact value, which is what `fma(d*sc, q, -(dmin*m))` gives on the device
(prototype/q4k_dequant/q4k_dequant_kernels.h:43-59). The reference's f64 route rounded to f32
(tools/gguf_fast_dequant.py:115-125) agrees whenever the f64 difference is exact, i.e. whenever
d and dmin are within 2^32 of each other (every realistic block; tests check both routes).
Q6_K: d*sc <= 11+7 bits, *(q-32) <= 5 more, so <= 23 bits: exact in f32 with no rounding at all.
"""
from __future__ import annotations

import numpy as np

QK_K = 256
Q4K_BYTES = 144      # 2 (d) + 2 (dmin) + 12 (scales) + 128 (qs)
Q5K_BYTES = 176      # 2 + 2 + 12 + 32 (qh) + 128 (qs)
Q6K_BYTES = 210      # 128 (ql) + 64 (qh) + 16 (int8 scales) + 2 (d, at byte 208)

# ggml_type ids (ggml/include/ggml.h enum, as listed in tools/gguf_reader.py)
GGML_Q4_K = 12
GGML_Q5_K = 13
GGML_Q6_K = 14
GGML_BF16 = 30                       # plain bf16 rows (ggml type id)
BLOCK_BYTES = {GGML_Q4_K: Q4K_BYTES, GGML_Q5_K: Q5K_BYTES, GGML_Q6_K: Q6K_BYTES}


def f16_to_f64(u16: np.ndarray) -> np.ndarray:
    """IEEE binary16 bit patterns -> float64 (exact for every finite pattern)."""
    return np.ascontiguousarray(u16, dtype=np.uint16).view(np.float16).astype(np.float64)


def _as_blocks(buf, block_bytes: int, n_elts: int) -> np.ndarray:
    raw = np.frombuffer(memoryview(buf), dtype=np.uint8) if not isinstance(buf, np.ndarray) \
        else buf.reshape(-1).view(np.uint8)
    nb = -(-int(n_elts) // QK_K)
    need = nb * block_bytes
    if raw.size < need:
        raise ValueError(f"short buffer: {n_elts} elements need {need} B, got {raw.size}")
    return raw[:need].reshape(nb, block_bytes)


def q4k_scale_min(scales: np.ndarray):
    """12 packed bytes -> (sc[8], m[8]) 6-bit ints; tools/gguf_reader.py:165-175.

        j < 4 : sc = s[j] & 63,                       m = s[j+4] & 63
        j >= 4: sc = (s[j+4] & 15) | ((s[j-4] >> 6) << 4)
                m  = (s[j+4] >> 4) | ((s[j]   >> 6) << 4)
    """
    s = np.asarray(scales, dtype=np.uint8).reshape(-1, 12).astype(np.int64)
    sc = np.empty((s.shape[0], 8), dtype=np.int64)
    m = np.empty((s.shape[0], 8), dtype=np.int64)
    sc[:, 0:4] = s[:, 0:4] & 63
    m[:, 0:4] = s[:, 4:8] & 63
    sc[:, 4:8] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:8] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def dequant_q4k(buf, n_elts: int) -> np.ndarray:
    """Q4_K blocks -> float32[n_elts]; element order as stored (gguf_reader.py:27-31):
    element e of a block: qs byte 32*(e>>6) + (e & 31), nibble (e>>5) & 1, sub-block e>>5."""
    raw = _as_blocks(buf, Q4K_BYTES, n_elts)
    d = f16_to_f64(raw[:, 0:2].copy().view(np.uint16).reshape(-1))
    dmin = f16_to_f64(raw[:, 2:4].copy().view(np.uint16).reshape(-1))
    sc, m = q4k_scale_min(raw[:, 4:16])
    qs = raw[:, 16:144].reshape(-1, 4, 32)
    q = np.stack([qs & 0xF, qs >> 4], axis=2).astype(np.float32)         # (nb, 4, 2, 32)
    # d*sc, (d*sc)*q and dmin*m are exact in f32; the subtraction is the single rounding.
    ds = (d.reshape(-1, 1, 1, 1) * sc.reshape(-1, 4, 2, 1)).astype(np.float32)
    dm = (dmin.reshape(-1, 1, 1, 1) * m.reshape(-1, 4, 2, 1)).astype(np.float32)
    vals = (ds * q) - dm
    return vals.reshape(-1)[:n_elts].astype(np.float32)


def dequant_q6k(buf, n_elts: int) -> np.ndarray:
    """Q6_K blocks -> float32[n_elts] (gguf_reader.py:42-48, 299-322). Element e = 128g+32k+l:
    q = ((ql[64g + 32(k&1) + l] >> 4(k>>1)) & 15) | (((qh[32g + l] >> 2k) & 3) << 4),
    value = d * sc[8g + 2k + (l>>4)] * (q - 32)."""
    raw = _as_blocks(buf, Q6K_BYTES, n_elts)
    ql = raw[:, 0:128].astype(np.int64)
    qh = raw[:, 128:192].astype(np.int64)
    sc = raw[:, 192:208].view(np.int8).astype(np.float64)
    d = f16_to_f64(raw[:, 208:210].copy().view(np.uint16).reshape(-1))
    g = np.arange(2).reshape(2, 1, 1)
    k = np.arange(4).reshape(1, 4, 1)
    l = np.arange(32).reshape(1, 1, 32)
    ql_idx = 64 * g + 32 * (k & 1) + l                                     # (2,4,32)
    qh_idx = 32 * g + 0 * k + l
    lo = (ql[:, ql_idx] >> (4 * (k >> 1))) & 0xF                           # (nb,2,4,32)
    hi = (qh[:, qh_idx] >> (2 * k)) & 3
    q = (lo | (hi << 4)).astype(np.float64) - 32.0
    sidx = (8 * g + 2 * k + (l >> 4))                                      # (2,4,32)
    s = sc[:, sidx]
    vals = (d.reshape(-1, 1, 1, 1) * s) * q
    return vals.reshape(-1)[:n_elts].astype(np.float32)


def dequant_q5k(buf, n_elts: int) -> np.ndarray:
    """Q5_K blocks -> float32 (gguf_reader.py:271-296): Q4_K layout plus a 5th bit; element e's
    high bit is bit (e>>5) of qh[e & 31]."""
    raw = _as_blocks(buf, Q5K_BYTES, n_elts)
    d = f16_to_f64(raw[:, 0:2].copy().view(np.uint16).reshape(-1))
    dmin = f16_to_f64(raw[:, 2:4].copy().view(np.uint16).reshape(-1))
    sc, m = q4k_scale_min(raw[:, 4:16])
    qh = raw[:, 16:48].astype(np.int64)                                    # (nb,32)
    qs = raw[:, 48:176].reshape(-1, 4, 32).astype(np.int64)
    q = np.stack([qs & 0xF, qs >> 4], axis=2)                              # (nb,4,2,32)
    bit = (qh[:, None, None, :] >> np.arange(8).reshape(1, 4, 2, 1)) & 1
    q = (q + 16 * bit).astype(np.float32)
    ds = (d.reshape(-1, 1, 1, 1) * sc.reshape(-1, 4, 2, 1)).astype(np.float32)
    dm = (dmin.reshape(-1, 1, 1, 1) * m.reshape(-1, 4, 2, 1)).astype(np.float32)
    return ((ds * q) - dm).reshape(-1)[:n_elts].astype(np.float32)


def dequant(buf, fmt: int, n_elts: int) -> np.ndarray:
    if fmt == GGML_Q4_K:
        return dequant_q4k(buf, n_elts)
    if fmt == GGML_Q6_K:
        return dequant_q6k(buf, n_elts)
    if fmt == GGML_Q5_K:
        return dequant_q5k(buf, n_elts)
    if fmt == GGML_BF16:
        # plain bf16 rows (ggml type 30): each 16-bit pattern is the top half of an f32
        u = np.frombuffer(np.ascontiguousarray(buf).tobytes(), dtype=np.uint16, count=n_elts)
        return (u.astype(np.uint32) << 16).view(np.float32)
    raise NotImplementedError(f"no decoder for ggml type {fmt}")


def dequant_matrix(qbytes: np.ndarray, fmt: int, rows: int, cols: int) -> np.ndarray:
    """A [rows, cols] weight matrix stored row-major as whole super-blocks per row."""
    if cols % QK_K:
        raise ValueError("row length must be a multiple of 256")
    return dequant(qbytes, fmt, rows * cols).reshape(rows, cols)
