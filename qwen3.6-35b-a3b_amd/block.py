"""The reference's MoE call surfaces, backed by the gfx950 library.

engine/block_forward.py:614-681 — moe_router / moe_shared / moe_routed / moe_block(g_row, W, cfg)
engine/m3_forward.py:430-476     — moe_block(g, E, layer) -> (out, {"used", "ids"})

Same names, argument meaning and stage dictionaries; every stage is computed on the GPU by the
HIP kernels behind the C-ABI, and routing values stay on the device (spec §11.7). `W` is a
weights.LayerWeights (it offers the reference handle's `get` / `expert_slice`); `cfg` is the
geometry dict of weights.load_geometry(). Errors raise abi.Refused(tag, msg).
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import abi


def _rows(g_row: torch.Tensor, cfg: dict) -> torch.Tensor:
    x = g_row.reshape(-1, cfg["d"])
    return x if x.is_contiguous() else x.contiguous()


def moe_router(g_row, W, cfg):
    """R1-R5 (engine/block_forward.py:614-636): router_logits bf16 [T,E], topk_ids int64 [T,K],
    topk_weights bf16 [T,K] (the R5 cast, before any multiply), topk_weights_f32 [T,K]."""
    x = _rows(g_row, cfg)
    r = abi.router_topk(x, W.router, cfg["top_k"], W.router_bias)
    return {"router_logits": r["router_logits"], "topk_ids": r["topk_ids"].long(),
            "topk_weights": r["topk_weights"], "topk_weights_f32": r["topk_weights_f32"]}


def moe_shared(g_row, W, cfg, path: int = L.MOE_PATH_AUTO):
    """Shared expert + scalar sigmoid gate (engine/block_forward.py:639-649)."""
    x = _rows(g_row, cfg)
    raw, prob = abi.shared_expert(x, W.shared_gate, W.shared_up, W.shared_down,
                                  W.shared_scalar_gate, path)
    prob = prob.view(-1, 1)
    return {"shared_raw": raw, "shared_gate_prob": prob, "shared_out": prob * raw}


def moe_routed(g_row, W, cfg, route, path: int = L.MOE_PATH_AUTO):
    """The K gathered experts and their ascending-id weighted sum (engine/block_forward.py:
    652-667): expert_raw [T,K,d] in top-k slot order, routed_sum [T,d]."""
    x = _rows(g_row, cfg)
    ids = route["topk_ids"].to(torch.int32).contiguous()
    grouping = abi.sort_permute(ids, W.n_experts)
    y = abi.experts(x, W.gate_up_q, W.gate_up_fmt, W.down_q, W.down_fmt, grouping, ids.shape[1],
                    path, up_q=W.up_q)
    T, H = x.shape
    zeros = torch.zeros(T, H, dtype=torch.float32, device=x.device)
    gp = torch.zeros(T, dtype=torch.float32, device=x.device)
    c = abi.combine(y, grouping, ids, route["topk_weights"].contiguous(), zeros, gp, stages=True)
    return {"expert_raw": c["expert_raw"], "routed_sum": c["routed_sum"]}


def moe_block(g_row, W, cfg, path: int = L.MOE_PATH_AUTO):
    """The whole block in §11.1's order (engine/block_forward.py:670-681), one library call."""
    x = _rows(g_row, cfg)
    st = abi.block_forward(x, W, path=path, stages=True)
    st["topk_ids"] = st["topk_ids"].long()
    st["shared_gate_prob"] = st["shared_gate_prob"].view(-1, 1)
    return st


class DeviceLayers:
    """The engine handle moe_block_m3 reads: one LayerWeights per decoder layer."""

    def __init__(self, layers):
        self.layers = list(layers)
        self.cfg = {"d": self.layers[0].hidden, "top_k": self.layers[0].top_k}

    def layer(self, i: int):
        return self.layers[i]


def moe_block_m3(g, E, layer, path: int = L.MOE_PATH_AUTO, out: torch.Tensor | None = None):
    """engine/m3_forward.py:430-476: g [B,T,d] -> (out [B,T,d] f32, {"used": n_hit_experts,
    "ids": [B,T,K] int64}). `used` is a 0-d device tensor: reading it is the caller's sync."""
    B, T, d = g.shape
    W = E.layer(layer)
    x = g.reshape(B * T, d).contiguous()
    st = abi.block_forward(x, W, path=path, stages={"topk_ids"}, out=out)
    ids = st["topk_ids"].long()
    used = torch.zeros(W.n_experts, dtype=torch.int32, device=x.device)
    used = used.index_fill_(0, ids.flatten(), 1).sum()
    return st["combined_out"].view(B, T, d), {"used": used, "ids": ids.view(B, T, -1)}
