"""The MoE block on the CPU, in the engine / policy-A form — test infrastructure, see __init__.py.

Semantics follow speccheck/moe_ref.py with Form(accumulate="f32", order="expert_asc",
weight_cast="before", batching="grouped") applied to dequantized weights, which is the engine's
f32 compute basis with the R1 and R5 casts (engine/m3_forward.py:430-476,
engine/block_forward.py:614-681, specification/11-moe-block.md §11.2-§11.6):

  R1  logits[t,e] = bf16_rne( sum_j x[t,j] * Wr[e,j]  (+ bias[e]) )       correctly rounded
  R2  probs = softmax(f32(logits))                                         torch CPU
  R3  (vals, ids) = torch.topk(probs, K)                                   torch CPU tie order
  R4  wpre = vals / vals.sum(-1)                                           f32
  R5  w = bf16(wpre)                                                        cast BEFORE multiply
  expert(e, x) = down_e @ (silu(gate_e x) * up_e x), gate = rows 0..I-1 of gate_up (gate first)
  routed[t] = sum over k in ascending expert id of f32(w[t,k]) * expert_raw[t,k]    (f32)
  shared[t] = sigmoid(wsg . x) * down_s @ (silu(gate_s x) * up_s x)                 (f32)
  out = routed + shared

With a post-attention norm weight (the decoder layer's MoE half, engine/m3_forward.py:732-737):

  xn  = rmsnorm_a(x1, w) = (x1 * r) * w,  r = f32(1 / sqrt(mean(x1^2) + eps))  (f64, one rounding)
  x   = x1 + moe_block(xn)["combined_out"]

R1 is the one deliberate departure from the reference's own arithmetic: torch's bf16 F.linear sums
in a blocked, thread-dependent order (prototype/moe_router/results.md:36), so this oracle defines
R1 as the correctly rounded dot — f64 accumulation with a certified error bound, and an exact
rational recompute for every logit whose f64 value lies within that bound of a bf16 rounding
midpoint.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from fractions import Fraction

import numpy as np
import torch
import torch.nn.functional as F

from . import ggml_quant as GQ

U64 = 2.0 ** -53


@dataclass(frozen=True)
class Geometry:
    """checkpoints/Qwen3.6-35B-A3B.config.json text_config (speccheck/moe_ref.py:62-118)."""
    hidden_size: int = 2048
    num_experts: int = 256
    top_k: int = 8
    moe_intermediate_size: int = 512
    shared_expert_intermediate_size: int = 512


GEOM = Geometry()


@dataclass
class LayerWeights:
    """One MoE block's weights as bytes / bf16 tensors on the host.

    gate_up_q: uint8 [E, 2I, row_bytes(H)]  GGUF super-blocks, gate rows 0..I-1 then up rows
    down_q:    uint8 [E, H, row_bytes(I)]
    router, shared_*: torch.bfloat16; router_bias: torch.float32 [E] or None (added inside R1).
    """
    router: torch.Tensor
    gate_up_q: np.ndarray
    gate_up_fmt: int
    down_q: np.ndarray
    down_fmt: int
    shared_gate: torch.Tensor
    shared_up: torch.Tensor
    shared_down: torch.Tensor
    shared_scalar_gate: torch.Tensor
    router_bias: torch.Tensor | None = None

    def expert_f32(self, e: int):
        """(gate_up [2I,H], down [H,I]) float32, decoded from the stored bytes."""
        two_i, h = self.gate_up_q.shape[1], self.down_q.shape[1]
        i = two_i // 2
        gu = GQ.dequant_matrix(self.gate_up_q[e], self.gate_up_fmt, two_i, h)
        dn = GQ.dequant_matrix(self.down_q[e], self.down_fmt, h, i)
        return torch.from_numpy(gu), torch.from_numpy(dn)


# ------------------------------------------------------------------------------------ bf16 edges
def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _round_to_bf16_exact(v: Fraction) -> float:
    """Round an exact rational to the nearest bf16 value, ties to even; returns it as a float."""
    if v == 0:
        return 0.0
    sign = -1.0 if v < 0 else 1.0
    a = -v if v < 0 else v
    e = a.numerator.bit_length() - a.denominator.bit_length()      # 2^e <= a < 2^(e+2)
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    qe = max(e - 7, -133)                                          # bf16 quantum at a
    n = a / (Fraction(2) ** qe)
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    val = math.ldexp(float(fl), qe)
    if val > 3.3895313892515355e38:
        return sign * math.inf
    return sign * val


def _bf16_quantum(v: np.ndarray) -> np.ndarray:
    a = np.abs(v)
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    # guard log2 rounding at exact powers of two
    e = np.where(np.exp2(e) > a, e - 1, e)
    e = np.where(np.exp2(e + 1) <= a, e + 1, e)
    return np.exp2(np.maximum(e - 7, -133))


def round_f64_to_bf16(v: np.ndarray) -> np.ndarray:
    """f64 -> nearest bf16 (ties to even) as float64 values; direct, never via f32."""
    q = _bf16_quantum(v)
    return np.round(v / q) * q          # v/q and the product are exact; np.round is half-even


def midpoint_distance(s: np.ndarray) -> np.ndarray:
    """Distance from each f64 value to the nearest bf16 rounding midpoint (0 where s is 0: a
    zero sum is always recomputed exactly). Inside a binade the midpoints sit half a quantum q
    from the bf16 grid; just above a power of two 2^e (|s| < 2^e + q) the quantum below 2^e is
    q/2, so the midpoint 2^e - q/4 may be the nearer one. Below 2^-126 (qe = -133 on both sides)
    the quantum does not change."""
    a = np.abs(s)
    q = _bf16_quantum(s)
    r = a / q                                    # exact (division by a power of two)
    fl = np.floor(r)
    d = np.abs((r - fl) - 0.5)
    at_pow2 = (fl == 128.0) & (q > 2.0 ** -133)
    d = np.where(at_pow2, np.minimum(d, (r - fl) + 0.25), d)
    return np.where(a > 0, d * q, 0.0)


def r1_logits(x: torch.Tensor, w_router: torch.Tensor, bias: torch.Tensor | None = None):
    """R1, correctly rounded: returns (logits bf16 [T,E], n_exact_recomputes)."""
    xd = x.detach().double().numpy()
    wd = w_router.detach().double().numpy()
    s = xd @ wd.T
    a = np.abs(xd) @ np.abs(wd).T
    n = xd.shape[1]
    if bias is not None:
        bd = bias.detach().double().numpy()
        s = s + bd[None, :]
        a = a + np.abs(bd)[None, :]
        n += 1
    # |f64 result - exact| <= gamma_n * sum|p|, and the computed `a` is itself within gamma_n;
    # a factor 4 covers both with room to spare.
    bound = 4.0 * (n + 2) * U64 * a
    near = midpoint_distance(s) <= bound
    out = round_f64_to_bf16(s)
    idx = np.argwhere(near)
    for t, e in idx:
        acc = sum(Fraction(float(xd[t, j])) * Fraction(float(wd[e, j])) for j in range(xd.shape[1]))
        if bias is not None:
            acc += Fraction(float(bias[e]))
        out[t, e] = _round_to_bf16_exact(acc)
    return torch.from_numpy(out.astype(np.float32)).to(torch.bfloat16), int(len(idx))


# ---------------------------------------------------------------------------------- the router
def route(x: torch.Tensor, w_router: torch.Tensor, top_k: int, bias=None) -> dict:
    """R1-R5 (speccheck/moe_ref.py:318-363, engine/m3_forward.py:443-446)."""
    logits, n_exact = r1_logits(x, w_router, bias)
    probs = torch.softmax(logits.float(), dim=-1)                       # R2, f32
    vals, ids = torch.topk(probs, top_k, dim=-1)                        # R3, torch tie order
    wpre = vals / vals.sum(dim=-1, keepdim=True)                        # R4, f32
    wcast = wpre.to(torch.bfloat16)                                     # R5, before the multiply
    return {"router_logits": logits, "router_probs": probs, "topk_ids": ids,
            "topk_weights": wcast, "topk_weights_f32": wpre, "topk_probs_pre_renorm": vals,
            "n_exact_recomputes": n_exact}


def expert_apply(rows: torch.Tensor, gu: torch.Tensor, dn: torch.Tensor) -> torch.Tensor:
    """rows [n,H] f32 -> [n,H] through one expert (speccheck/moe_ref.py:367-392): gate first."""
    h = F.linear(rows, gu)
    gate, up = h.chunk(2, dim=-1)
    return F.linear(F.silu(gate) * up, dn)


def experts_and_combine(x: torch.Tensor, ids: torch.Tensor, w_bf16: torch.Tensor,
                        lw: LayerWeights) -> dict:
    """Grouped gather (moe_ref.py:395-451), ascending-id f32 combine (moe_ref.py:452-476)."""
    T, K = ids.shape
    H = x.shape[1]
    xf = x.float()
    raw = torch.zeros(T, K, H, dtype=torch.float32)
    for e_t in torch.unique(ids):                                       # ascending expert id
        e = int(e_t)
        tok, slot = torch.where(ids == e)
        gu, dn = lw.expert_f32(e)
        raw[tok, slot] = expert_apply(xf[tok], gu, dn)
    return {"expert_raw": raw, "routed_sum": routed_combine(raw, ids, w_bf16)}


def routed_combine(raw: torch.Tensor, ids: torch.Tensor, w_bf16: torch.Tensor) -> torch.Tensor:
    """routed[t] = sum over the token's K slots in ascending expert id of f32(w_bf16[t,k]) *
    raw[t,k], each product rounded to f32 before its add (speccheck/moe_ref.py:452-476: the
    expert_asc order, the cast-before weight, `prod = raw * w; acc += prod`)."""
    T, K, H = raw.shape
    w = w_bf16.to(torch.float32)
    order = torch.argsort(ids, dim=-1, stable=True)
    acc = torch.zeros(T, H, dtype=torch.float32)
    ar = torch.arange(T)
    for j in range(K):
        k = order[:, j]
        prod = raw[ar, k] * w[ar, k][:, None]
        acc = acc + prod
    return acc


def final_add(routed: torch.Tensor, gate_prob: torch.Tensor, shared_raw: torch.Tensor,
              residual: torch.Tensor | None = None) -> torch.Tensor:
    """combined = routed + gate_prob * shared_raw (speccheck/moe_ref.py:514-517), then
    x = x1 + combined (engine/m3_forward.py:737); every op rounded to f32 on its own."""
    combined = routed + gate_prob.reshape(-1, 1) * shared_raw
    return combined if residual is None else residual + combined


def shared_expert(x: torch.Tensor, lw: LayerWeights) -> dict:
    """speccheck/moe_ref.py:480-495 in f32; gate is one scalar per token (spec §11.6)."""
    xf = x.float()
    g = lw.shared_gate.float()
    u = lw.shared_up.float()
    d = lw.shared_down.float()
    raw = F.linear(F.silu(F.linear(xf, g)) * F.linear(xf, u), d)
    prob = torch.sigmoid(F.linear(xf, lw.shared_scalar_gate.float()))
    return {"shared_raw": raw, "shared_gate_prob": prob, "shared_out": prob * raw}


def moe_block(x: torch.Tensor, lw: LayerWeights, top_k: int = 8) -> dict:
    """The whole block; stage names follow speccheck/moe_ref.py:519-533."""
    if x.dim() == 3:
        x = x.reshape(-1, x.shape[-1])
    r = route(x, lw.router, top_k, lw.router_bias)
    e = experts_and_combine(x, r["topk_ids"], r["topk_weights"], lw)
    s = shared_expert(x, lw)
    out = {"input": x}
    out.update(r)
    out.update(e)
    out.update(s)
    out["combined_out"] = final_add(e["routed_sum"], s["shared_gate_prob"], s["shared_raw"])
    return out


# --------------------------------------------------------------------------------- comparators
def rmsnorm_a(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Post-attention RMSNorm, Form A with the artifact's (1 + w) already in w
    (engine/m3_forward.py:303-307): (x * r) * w in f32. This oracle evaluates the scale
    r = 1/sqrt(mean(x^2) + eps) in f64 (every square of an f32 is exact there) and rounds it once
    to f32; torch's f32 mean sums in a vectorized, unpinnable order and differs from it by at most
    a couple of f32 ulps of r."""
    xf = x.float()
    x64 = xf.double()
    ms = (x64 * x64).sum(-1, keepdim=True) / x.shape[-1]
    r = (1.0 / torch.sqrt(ms + float(eps))).float()
    return (xf * r) * w.float()


def residual_step(x1: torch.Tensor, lw: LayerWeights, norm_w: torch.Tensor, eps: float,
                  top_k: int = 8) -> dict:
    """The decoder layer's MoE half (engine/m3_forward.py:732-737): h = rmsnorm_a(x1, w);
    x = x1 + moe_block(h). Returns moe_block's stages (on h) plus "x_out"."""
    st = moe_block(rmsnorm_a(x1, norm_w, eps), lw, top_k)
    st["x_out"] = final_add(st["routed_sum"], st["shared_gate_prob"], st["shared_raw"], x1.float())
    return st


def ulp_of(v: float) -> float:
    """The width of one bf16 step above |v| (speccheck/moe_ref.py:551-567): 2^(floor(log2|v|) - 7),
    bf16 having 7 explicit mantissa bits; 0.0 at zero and for non-finite v."""
    v = abs(float(v))
    if v == 0 or not math.isfinite(v):
        return 0.0
    m, e = math.frexp(v)                 # v = m 2^e, 0.5 <= m < 1: floor(log2 v) = e - 1, exactly
    return math.ldexp(1.0, e - 1 - 7)


def metrics(a: torch.Tensor, b: torch.Tensor, name: str = "") -> dict:
    """speccheck/moe_ref.py:578-630 comparator fields (max_abs, max_abs_over_scale, mean_abs,
    1-cos, ndiff, n_gt_1ulp / n_gt_100ulp against one bf16 step at the reference's max |value|).
    Refuses a shape or dtype mismatch (both sides are widened to f64 explicitly, so a mixed pair
    would otherwise compare quietly), non-finite input, an all-zero reference and a zero norm."""
    if a.shape != b.shape:
        raise AssertionError(f"{name}: shape {tuple(a.shape)} vs {tuple(b.shape)}")
    if a.dtype != b.dtype:
        raise AssertionError(f"{name}: dtype {a.dtype} vs {b.dtype}")
    x = a.detach().to(torch.float64).flatten()
    y = b.detach().to(torch.float64).flatten()
    if not (torch.isfinite(x).all() and torch.isfinite(y).all()):
        raise AssertionError(f"{name}: non-finite input to metrics()")
    scale = y.abs().max().item()
    if scale == 0:
        raise AssertionError(f"{name}: the reference side is all zero")
    diff = (x - y).abs()
    denom = (x.norm() * y.norm()).item()
    if denom == 0:
        raise AssertionError(f"{name}: zero-norm side; cos is undefined")
    cos = (x @ y).item() / denom
    ulp_ref = ulp_of(scale)
    return {"name": name, "dtype": str(a.dtype), "n": int(x.numel()), "max_abs": diff.max().item(),
            "max_abs_over_scale": diff.max().item() / scale, "mean_abs": diff.mean().item(),
            "one_minus_cos": max(0.0, 1.0 - cos), "ndiff": int((diff > 0).sum().item()),
            "n_gt_1ulp": int((diff > ulp_ref).sum().item()),
            "n_gt_100ulp": int((diff > 100 * ulp_ref).sum().item()),
            "ref_absmax": scale, "ulp_of_refmax": ulp_ref}


def from_device(lw) -> LayerWeights:
    """Copy a device-side weight set (any object with the LayerWeights field names) to the host
    form this oracle reads; the bytes are the same bytes the kernels read. Separate gate and up
    records (an `up_q` field) are stacked gate first, the fused record's row order."""
    def host(t):
        return None if t is None else t.detach().cpu()
    gu = host(lw.gate_up_q).numpy()
    up = getattr(lw, "up_q", None)
    if up is not None:
        gu = np.concatenate([gu, host(up).numpy()], axis=1)

    def shared(t):
        # Q8_0 rows (uint8) decode to the exact f32 values d * q (tools/gguf_reader.py:238-245)
        if t.dtype != torch.uint8:
            return host(t)
        from .lm_head_oracle import dequant_q8_0
        b = host(t).numpy()
        n = b.shape[1] // 34 * 32
        return torch.from_numpy(dequant_q8_0(b.reshape(-1), b.shape[0] * n).reshape(b.shape[0], n))
    return LayerWeights(
        router=host(lw.router), gate_up_q=gu, gate_up_fmt=lw.gate_up_fmt,
        down_q=host(lw.down_q).numpy(), down_fmt=lw.down_fmt, shared_gate=shared(lw.shared_gate),
        shared_up=shared(lw.shared_up), shared_down=shared(lw.shared_down),
        shared_scalar_gate=host(lw.shared_scalar_gate), router_bias=host(lw.router_bias))
