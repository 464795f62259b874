"""GGUF K-quant packers: float weights -> Q4_K / Q5_K / Q6_K super-block bytes (torch, CPU or GPU).

These produce weight bytes in the exact GGUF layout the device kernels consume (the same bytes the
reference reads, tools/gguf_reader.py:17-51). The fit is a plain min/max fit of this package's own
(like the reference's `_qref_k` / `_qref_q6_K`, tools/gguf_reader.py:386-452, it is not llama.cpp's
iterative fit). Parity never depends on the packer: the device kernels and every checker consume
the same bytes. Written with torch tensor ops so the same code packs on the host (tests) and on
the device (the benchmark's 40 x 256 synthetic experts), chunked to bound temporaries.

Layouts written here:
  Q4_K (144 B / 256 elements): f16 d | f16 dmin | 12 B packed 6-bit (sc, m) x 8 | 128 B nibbles,
       element 64g + l (l < 32) in the low nibble of qs[32g + l], 64g + 32 + l in its high nibble.
  Q5_K (176 B / 256 elements): f16 d | f16 dmin | 12 B scales (as Q4_K) | qh[32] | 128 B nibbles;
       the Q4_K nibble layout for the low 4 bits of q in [0, 31], and the 5th bit of element e
       at bit e >> 5 of qh[e & 31] (tools/gguf_reader.py:271-296).
  Q6_K (210 B / 256 elements): ql[128] | qh[64] | int8 sc[16] | f16 d; element 128g + 32k + l has
       its low 4 bits in nibble (k >> 1) of ql[64g + 32(k & 1) + l] and its high 2 bits at bit 2k
       of qh[32g + l]; the stored value is q + 32 for q in [-32, 31].
"""
from __future__ import annotations

import numpy as np
import torch

QK_K = 256
Q4K_BYTES = 144
Q5K_BYTES = 176
Q6K_BYTES = 210
FMT_Q4_K = 12
FMT_Q5_K = 13
FMT_Q6_K = 14
FMT_BF16 = 30
FMT_Q8_0 = 8
Q8_0_BYTES = 34                      # f16 d + 32 x int8, per 32 elements
# bytes per 256 elements
BLOCK_BYTES = {FMT_Q4_K: Q4K_BYTES, FMT_Q5_K: Q5K_BYTES, FMT_Q6_K: Q6K_BYTES, FMT_Q8_0: 8 * Q8_0_BYTES,
               FMT_BF16: 2 * QK_K}


def _u8(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.uint8)


def _f16_bytes(t: torch.Tensor) -> torch.Tensor:
    """float tensor [...] -> uint8 [..., 2] (little-endian f16 bit pattern)."""
    return t.to(torch.float16).contiguous().view(torch.uint8).reshape(*t.shape, 2)


def pack_q4k_scales(sc: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """(sc, m) int[..., 8] in [0, 63] -> uint8[..., 12]; the inverse of get_scale_min_k4
    (tools/gguf_reader.py:165-175)."""
    sc = sc.to(torch.int32)
    m = m.to(torch.int32)
    s0 = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    s1 = (m[..., 0:4] & 63) | ((m[..., 4:8] >> 4) << 6)
    s2 = (sc[..., 4:8] & 15) | ((m[..., 4:8] & 15) << 4)
    return _u8(torch.cat([s0, s1, s2], dim=-1))


def _kquant_fit(w: torch.Tensor, qmax: int):
    """The min/max fit shared by Q4_K (qmax 15) and Q5_K (qmax 31): per super-block f16 d, dmin;
    per 32-element sub-block 6-bit sc, m; per element q in [0, qmax] with v ~ d*sc*q - dmin*m."""
    rows, cols = w.shape
    nb = cols // QK_K
    x = w.reshape(rows, nb, 8, 32).float()
    mn = torch.clamp(x.amin(dim=-1), max=0.0)                  # (rows, nb, 8)
    mx = x.amax(dim=-1)
    scale = (mx - mn) / float(qmax)
    minv = -mn
    d = (scale.amax(dim=-1) / 63.0).to(torch.float16).float()  # (rows, nb)
    dmin = (minv.amax(dim=-1) / 63.0).to(torch.float16).float()
    sc = torch.where(d[..., None] > 0, torch.round(scale / d[..., None].clamp_min(1e-30)),
                     torch.zeros_like(scale)).clamp(0, 63)
    mm = torch.where(dmin[..., None] > 0, torch.round(minv / dmin[..., None].clamp_min(1e-30)),
                     torch.zeros_like(minv)).clamp(0, 63)
    step = d[..., None] * sc
    off = dmin[..., None] * mm
    q = torch.where(step[..., None] > 0,
                    torch.round((x + off[..., None]) / step[..., None].clamp_min(1e-30)),
                    torch.zeros_like(x)).clamp(0, qmax).to(torch.int32)  # (rows, nb, 8, 32)
    return d, dmin, sc, mm, q


def _q4k_rows(w: torch.Tensor) -> torch.Tensor:
    rows, cols = w.shape
    nb = cols // QK_K
    d, dmin, sc, mm, q = _kquant_fit(w, 15)
    qg = q.reshape(rows, nb, 4, 2, 32)
    qs = _u8(qg[..., 0, :] | (qg[..., 1, :] << 4)).reshape(rows, nb, 128)
    out = torch.cat([_f16_bytes(d), _f16_bytes(dmin), pack_q4k_scales(sc, mm), qs], dim=-1)
    return out.reshape(rows, nb * Q4K_BYTES)


def _q5k_rows(w: torch.Tensor) -> torch.Tensor:
    rows, cols = w.shape
    nb = cols // QK_K
    d, dmin, sc, mm, q = _kquant_fit(w, 31)
    lo = q & 15
    qg = lo.reshape(rows, nb, 4, 2, 32)
    qs = _u8(qg[..., 0, :] | (qg[..., 1, :] << 4)).reshape(rows, nb, 128)
    # bit j of qh[l] is the 5th bit of element 32 j + l (sub-block j)
    hi = (q >> 4).reshape(rows, nb, 8, 32)
    qh = torch.zeros(rows, nb, 32, dtype=torch.int32, device=w.device)
    for j in range(8):
        qh |= hi[:, :, j, :] << j
    out = torch.cat([_f16_bytes(d), _f16_bytes(dmin), pack_q4k_scales(sc, mm), _u8(qh), qs], dim=-1)
    return out.reshape(rows, nb * Q5K_BYTES)


def _q6k_rows(w: torch.Tensor) -> torch.Tensor:
    rows, cols = w.shape
    nb = cols // QK_K
    x = w.reshape(rows, nb, 16, 16).float()
    scale = x.abs().amax(dim=-1) / 31.0                        # (rows, nb, 16)
    d = (scale.amax(dim=-1) / 127.0).to(torch.float16).float()
    sc = torch.where(d[..., None] > 0, torch.round(scale / d[..., None].clamp_min(1e-30)),
                     torch.zeros_like(scale)).clamp(-128, 127)
    step = d[..., None] * sc
    q = torch.where(step[..., None] != 0, torch.round(x / torch.where(step[..., None] != 0,
                                                                        step[..., None], 1.0)),
                    torch.zeros_like(x)).clamp(-32, 31).to(torch.int32) + 32
    q = q.reshape(rows, nb, 2, 4, 32)                          # (g, k, l)
    ql0 = (q[..., 0, :] & 15) | ((q[..., 2, :] & 15) << 4)
    ql1 = (q[..., 1, :] & 15) | ((q[..., 3, :] & 15) << 4)
    ql = _u8(torch.stack([ql0, ql1], dim=-2)).reshape(rows, nb, 128)
    qh = _u8((q[..., 0, :] >> 4) | ((q[..., 1, :] >> 4) << 2) | ((q[..., 2, :] >> 4) << 4)
             | ((q[..., 3, :] >> 4) << 6)).reshape(rows, nb, 64)
    scb = sc.to(torch.int8).view(torch.uint8)
    out = torch.cat([ql, qh, scb, _f16_bytes(d)], dim=-1)
    return out.reshape(rows, nb * Q6K_BYTES)


def _q8_0_rows(w: torch.Tensor) -> torch.Tensor:
    """Q8_0: per 32 elements d = f16(max|x| / 127), q = round(x / d) as int8 (the GGUF block
    tools/gguf_reader.py:238-245 decodes)."""
    rows, cols = w.shape
    nb = cols // 32
    x = w.reshape(rows, nb, 32).float()
    d = (x.abs().amax(dim=-1) / 127.0).to(torch.float16).float()
    q = torch.where(d[..., None] > 0, torch.round(x / d[..., None].clamp_min(1e-30)),
                    torch.zeros_like(x)).clamp(-127, 127).to(torch.int8).view(torch.uint8)
    out = torch.cat([_f16_bytes(d), q], dim=-1)
    return out.reshape(rows, nb * Q8_0_BYTES)


def _bf16_rows(w: torch.Tensor) -> torch.Tensor:
    """Plain bf16 rows (RNE) as their little-endian bytes: the BF16 weight records."""
    return w.to(torch.bfloat16).contiguous().view(torch.uint8).reshape(w.shape[0], -1)


def quantize(w, fmt: int, chunk_rows: int = 16384) -> torch.Tensor:
    """float[rows, cols] (torch or numpy; cols % 256 == 0) -> uint8[rows, row_bytes(fmt, cols)]
    on the same device as `w`."""
    if isinstance(w, np.ndarray):
        w = torch.from_numpy(np.ascontiguousarray(w, dtype=np.float32))
    if w.dim() != 2 or w.shape[1] % QK_K:
        raise ValueError(f"expected [rows, cols] with cols % 256 == 0, got {tuple(w.shape)}")
    fn = {FMT_Q4_K: _q4k_rows, FMT_Q5_K: _q5k_rows, FMT_Q6_K: _q6k_rows, FMT_Q8_0: _q8_0_rows,
          FMT_BF16: _bf16_rows}.get(fmt)
    if fn is None:
        raise ValueError(f"unsupported format {fmt}")
    rows = w.shape[0]
    out = torch.empty(rows, row_bytes(fmt, w.shape[1]), dtype=torch.uint8, device=w.device)
    for r0 in range(0, rows, chunk_rows):
        out[r0:r0 + chunk_rows] = fn(w[r0:r0 + chunk_rows])
    return out


def quantize_q4k(w) -> torch.Tensor:
    return quantize(w, FMT_Q4_K)


def quantize_q5k(w) -> torch.Tensor:
    return quantize(w, FMT_Q5_K)


def quantize_q6k(w) -> torch.Tensor:
    return quantize(w, FMT_Q6_K)


def row_bytes(fmt: int, cols: int) -> int:
    if cols % QK_K:
        raise ValueError("cols must be a multiple of 256")
    per = BLOCK_BYTES.get(fmt)
    if per is None:
        raise ValueError(f"unsupported format {fmt}")
    return cols // QK_K * per
