"""Untied lm_head oracle (CPU, numpy) — test infrastructure, see oracle/__init__.py.

What it restates:
  * the table decode: Q6_K through ggml_quant.dequant_q6k (tools/gguf_reader.py:299-322), Q8_0 as
    tools/gguf_reader.py:238-245 (`_deq_q8_0`: value = f16(d) * int8(q), exact in f32: 11 + 8
    significant bits), bf16 by bit pattern;
  * the dot: logits[b, j] = sum_k h[b, k] * W[row_j, k] (prototype/lm_head/lm_head_kernels.h:474-512,
    `lmh_dot_batch`), here in f64 over the f32 dequantized weights, so the oracle's own rounding
    error (about K * 2^-53 relative) is far inside any f32 band;
  * the acceptance band of prototype/lm_head/gate.py:214-240 (`gamma_of_index`, `gamma_index`):
    |device - exact| <= gamma_n * sum_k |h_k w_k|, gamma_n = n u / (1 - n u), u = 2^-24, with
    n = K - 1 when every product h_k w_k is exact in binary32 and n = 2K - 1 when any is not —
    the index chosen by measuring the products, never typed.

Pins: the gamma values against the two the reference quotes (prototype/lm_head/HANDOFF.md:13-15,
gamma_2047 = 1.22025596e-04 and gamma_4095 = 2.4414061e-04); the Q8_0 decode against hand-built
blocks with closed-form values; the f64 dot against an exact rational sum on small cases
(tests/test_oracle_lm_head.py).
"""
from __future__ import annotations

import numpy as np

from . import ggml_quant as GQ

U32 = 2.0 ** -24
Q8_0_BYTES = 34
GGML_Q8_0 = 8
FMT_BF16 = 30


def gamma_of_index(n: int) -> float:
    """Higham's gamma_n = n u / (1 - n u) for binary32 (prototype/lm_head/gate.py:214-221)."""
    if n < 1 or n * U32 >= 1.0:
        raise ValueError(f"gamma_{n} is not a band factor")
    return n * U32 / (1.0 - n * U32)


def gamma_index(K: int, products_inexact: int) -> int:
    """K - 1 roundings for a K-term dot whose products are exact in binary32, 2K - 1 when any
    product is not (prototype/lm_head/gate.py:224-240)."""
    if products_inexact is None:
        raise ValueError("the band index needs a measured count")
    return K - 1 if products_inexact == 0 else 2 * K - 1


def dequant_q8_0(buf, n_elts: int) -> np.ndarray:
    """Q8_0 blocks (f16 d, 32 x int8) -> float32[n_elts], value = d * q (tools/gguf_reader.py:238-245)."""
    raw = np.frombuffer(bytes(np.asarray(buf, dtype=np.uint8).tobytes()), dtype=np.uint8)
    nb = -(-n_elts // 32)
    raw = raw[: nb * Q8_0_BYTES].reshape(nb, Q8_0_BYTES)
    d = GQ.f16_to_f64(raw[:, 0:2].copy().view(np.uint16).reshape(-1))
    q = raw[:, 2:34].copy().view(np.int8).astype(np.float64)
    return (d.reshape(-1, 1) * q).reshape(-1)[:n_elts].astype(np.float32)


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def table_rows(w: np.ndarray, fmt: int, rows: np.ndarray, H: int) -> np.ndarray:
    """f32 [len(rows), H]: the decoded table rows `rows` of W (uint8 [V, row_bytes] for Q6_K /
    Q8_0, uint16 [V, H] bf16 bits for BF16)."""
    out = np.empty((len(rows), H), dtype=np.float32)
    for i, r in enumerate(rows):
        if fmt == GQ.GGML_Q6_K:
            out[i] = GQ.dequant_q6k(w[r], H)
        elif fmt == GGML_Q8_0:
            out[i] = dequant_q8_0(w[r], H)
        elif fmt == FMT_BF16:
            out[i] = bf16_to_f32(w[r])
        else:
            raise NotImplementedError(fmt)
    return out


def lm_head(h: np.ndarray, wrows: np.ndarray):
    """(exact-ish logits f64 [B, n], band f64 [B, n], band index) for hidden vectors h (f32
    [B, H]) against decoded rows wrows (f32 [n, H])."""
    h64 = np.asarray(h, dtype=np.float32).astype(np.float64)
    w64 = np.asarray(wrows, dtype=np.float32).astype(np.float64)
    logits = h64 @ w64.T
    # f32 x f32 products are exact in f64 (<= 48 significant bits): count those binary32 rounds
    inexact = 0
    for r0 in range(0, w64.shape[0], 256):
        prod = h64[:, None, :] * w64[None, r0:r0 + 256, :]
        inexact += int(np.count_nonzero(prod.astype(np.float32).astype(np.float64) != prod))
    n = gamma_index(h64.shape[1], inexact)
    band = gamma_of_index(n) * np.abs(h64) @ np.abs(w64).T
    return logits, band, n
