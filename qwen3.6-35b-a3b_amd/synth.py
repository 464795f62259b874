"""Seeded synthetic weights and inputs of the real architecture, for tests and the benchmark
(the benchmark configurations: N(0, 0.02) weights quantized by quant.py, N(0, 1) activations).

Generation runs on whatever device is asked for (the benchmark generates its 40 x 256 Q4_K
experts on the GPU, chunk by chunk); every draw comes from a private torch.Generator seeded from
the config's seed, so a config is the same bytes every time on the same device type.
"""
from __future__ import annotations

import math

import torch

from . import quant as Q
from .weights import LayerWeights


def zipf_bias(n_experts: int, seed: int, s: float = 1.1, device="cpu") -> torch.Tensor:
    """Per-expert router logit bias b_e = ln(r_e^-s / sum_r r^-s) over a seeded permutation of
    the ranks 1..E: softmax of the bias alone is a Zipf(s) law, so routing is skewed."""
    g = torch.Generator(device="cpu").manual_seed(seed + 7919)
    ranks = torch.randperm(n_experts, generator=g).to(torch.float64) + 1.0
    w = ranks.pow(-s)
    return torch.log(w / w.sum()).to(torch.float32).to(device)


def make_layer(seed: int, device="cuda", gate_up_fmt: int = Q.FMT_Q4_K,
               down_fmt: int = Q.FMT_Q4_K, zipf: bool = False, n_experts: int = 256,
               hidden: int = 2048, i_e: int = 512, i_s: int = 512, top_k: int = 8,
               std: float = 0.02, chunk: int = 16, router_dtype=torch.bfloat16,
               scalar_gate_dtype=torch.bfloat16, split_gate_up: bool = False,
               shared_fmt: int = Q.FMT_BF16) -> LayerWeights:
    """Random-init weights of the block's architecture. router_dtype / scalar_gate_dtype f32 and
    split_gate_up give the shipped artifact's widths (F32 ffn_gate_inp and ffn_gate_inp_shexp,
    separate ffn_gate_exps / ffn_up_exps records; engine/block_forward.py:221-231); shared_fmt
    Q8_0 stores the shared expert as the artifact's Q8_0 ffn_*_shexp rows."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)

    def randn(*shape):
        return torch.randn(*shape, generator=g, device=dev, dtype=torch.float32) * std

    router = randn(n_experts, hidden).to(router_dtype)
    gu_row = Q.row_bytes(gate_up_fmt, hidden)
    dn_row = Q.row_bytes(down_fmt, i_e)
    gate_up = torch.empty(n_experts, 2 * i_e, gu_row, dtype=torch.uint8, device=dev)
    down = torch.empty(n_experts, hidden, dn_row, dtype=torch.uint8, device=dev)
    for e0 in range(0, n_experts, chunk):
        n = min(chunk, n_experts - e0)
        w = randn(n, 2 * i_e, hidden)
        gate_up[e0:e0 + n] = Q.quantize(w.reshape(-1, hidden), gate_up_fmt).view(n, 2 * i_e, gu_row)
        del w
        w = randn(n, hidden, i_e)
        down[e0:e0 + n] = Q.quantize(w.reshape(-1, i_e), down_fmt).view(n, hidden, dn_row)
        del w
    def shared(*shape):
        w = randn(*shape)
        return Q.quantize(w, Q.FMT_Q8_0) if shared_fmt == Q.FMT_Q8_0 else w.to(torch.bfloat16)

    lw = LayerWeights(
        router=router, gate_up_q=gate_up, gate_up_fmt=gate_up_fmt, down_q=down, down_fmt=down_fmt,
        shared_gate=shared(i_s, hidden), shared_up=shared(i_s, hidden),
        shared_down=shared(hidden, i_s),
        shared_scalar_gate=randn(1, hidden).to(scalar_gate_dtype),
        router_bias=zipf_bias(n_experts, seed, device=dev) if zipf else None,
        top_k=top_k, shared_fmt=shared_fmt)
    if split_gate_up:
        lw = lw.split_gate_up()
    lw.validate()
    return lw


def make_input(n_tokens: int, seed: int, device="cuda", dtype=torch.float32,
               hidden: int = 2048) -> torch.Tensor:
    """x ~ N(0, 1) f32 [T, H] from a private generator; cast to `dtype` (bf16 for prefill)."""
    g = torch.Generator(device=torch.device(device)).manual_seed(seed + 104729)
    x = torch.randn(n_tokens, hidden, generator=g, device=device, dtype=torch.float32)
    return x.to(dtype)


def rms_normalize(x: torch.Tensor) -> torch.Tensor:
    """Rows rescaled to RMS 1 (the block input is a post-attention RMSNorm output; used to chain
    layer outputs into the next layer's input in the decode benchmark). torch's fused rms_norm:
    one kernel on the GPU where the composed form (square, mean, add, rsqrt, multiply) took five,
    inside the benchmark's timed graph."""
    return torch.nn.functional.rms_norm(x.float(), (x.shape[-1],), eps=1e-6).to(x.dtype)


def make_norm_weight(seed: int, device="cuda", hidden: int = 2048, std: float = 0.1) -> torch.Tensor:
    """A post-attention RMSNorm weight as the artifact stores it (1 + w folded in): 1 + N(0, std)."""
    g = torch.Generator(device="cpu").manual_seed(seed + 15485863)
    return (1.0 + std * torch.randn(hidden, generator=g)).to(device)


def decode_active_bytes(lw: LayerWeights) -> int:
    """Bytes of the 8 routed + 1 shared active experts per token-layer (20,447,232 for Q4_K experts
    and a bf16 shared expert at H = 2048, I = I_s = 512)."""
    return lw.top_k * lw.routed_bytes_per_expert() + lw.shared_bytes()


def prefill_flops(T: int, lw: LayerWeights) -> float:
    """Routed + shared expert FLOPs of a T-token step (2 FLOP per MAC)."""
    per_expert = 3 * lw.i_e * lw.hidden
    shared = 3 * lw.i_s * lw.hidden
    return 2.0 * T * (lw.top_k * per_expert + shared)


def router_flops(T: int, lw: LayerWeights) -> float:
    return 2.0 * T * lw.n_experts * lw.hidden


_ = math
