"""One MoE block's weights, resident on one GPU, in the layout the kernels read.

Mirrors the reference's weight handle (engine/block_forward.py:347-483, `W.get(name)` and
`W.expert_slice('gate'|'up'|'down', e)`) and its geometry dict (engine/block_forward.py:504-531).

HBM layout (all 16-byte aligned, expert axis slowest, as GGUF stores it — engine/loader.py:338-390):
  router           bf16 [E, H]                      read whole every token
  router_bias      f32  [E] or None                 added inside R1 (synthetic skew only)
  gate_up_q        u8   [E, 2I, H/256 * blk]        gate rows 0..I-1 then up rows (spec §11.4)
  down_q           u8   [E, H, I/256 * blk]
  shared_gate/up   bf16 [I_s, H];  shared_down bf16 [H, I_s];  shared_scalar_gate bf16 [1, H]
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import quant as Q

GEOMETRY = {"d": 2048, "n_experts": 256, "top_k": 8, "i_e": 512, "i_s": 512,
            "act_dtype": torch.bfloat16, "threads": 8}


def load_geometry() -> dict:
    """checkpoints/Qwen3.6-35B-A3B.config.json text_config, as engine/block_forward.py:504-531
    returns it (d, n_experts, top_k, i_e, i_s, act_dtype, threads)."""
    return dict(GEOMETRY)


@dataclass
class LayerWeights:
    router: torch.Tensor
    gate_up_q: torch.Tensor
    gate_up_fmt: int
    down_q: torch.Tensor
    down_fmt: int
    shared_gate: torch.Tensor
    shared_up: torch.Tensor
    shared_down: torch.Tensor
    shared_scalar_gate: torch.Tensor
    router_bias: torch.Tensor | None = None
    top_k: int = 8

    @property
    def n_experts(self) -> int:
        return self.router.shape[0]

    @property
    def hidden(self) -> int:
        return self.router.shape[1]

    @property
    def i_e(self) -> int:
        return self.gate_up_q.shape[1] // 2

    @property
    def i_s(self) -> int:
        return self.shared_gate.shape[0]

    @property
    def device(self) -> torch.device:
        return self.router.device

    def routed_bytes_per_expert(self) -> int:
        return self.gate_up_q[0].numel() + self.down_q[0].numel()

    def shared_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in
                   (self.shared_gate, self.shared_up, self.shared_down))

    def validate(self) -> None:
        E, H = self.router.shape
        I = self.i_e
        want = {
            "gate_up_q": (self.gate_up_q, torch.uint8, (E, 2 * I, Q.row_bytes(self.gate_up_fmt, H))),
            "down_q": (self.down_q, torch.uint8, (E, H, Q.row_bytes(self.down_fmt, I))),
            "shared_gate": (self.shared_gate, torch.bfloat16, (self.i_s, H)),
            "shared_up": (self.shared_up, torch.bfloat16, (self.i_s, H)),
            "shared_down": (self.shared_down, torch.bfloat16, (H, self.i_s)),
            "shared_scalar_gate": (self.shared_scalar_gate, torch.bfloat16, (1, H)),
        }
        for name, (t, dt, shp) in want.items():
            if t.dtype != dt or tuple(t.shape) != tuple(shp) or not t.is_contiguous():
                raise ValueError(f"{name}: got {t.dtype} {tuple(t.shape)}, want {dt} {shp}")
        if self.router.dtype != torch.bfloat16:
            raise ValueError("router must be bf16")

    # ----------------------------------------------------- the reference's weight-handle surface
    def get(self, name: str) -> torch.Tensor:
        """Whole tensor by GGUF role name (engine/block_forward.py:412-428), blk.N. prefix allowed."""
        role = name.split(".")[-2] if name.endswith(".weight") else name
        table = {"ffn_gate_inp": self.router, "ffn_gate_shexp": self.shared_gate,
                 "ffn_up_shexp": self.shared_up, "ffn_down_shexp": self.shared_down,
                 "ffn_gate_inp_shexp": self.shared_scalar_gate}
        if role not in table:
            raise KeyError(f"no tensor for role {role!r} (routed experts: use expert_slice)")
        return table[role]

    def expert_slice(self, role: str, e: int) -> torch.Tensor:
        """One routed expert's matrix decoded on the device to f32 (engine/block_forward.py:430-468):
        'gate'/'up' -> [I, H], 'down' -> [H, I]."""
        from . import abi
        H, I = self.hidden, self.i_e
        if role in ("gate", "up"):
            rows = self.gate_up_q[e, :I] if role == "gate" else self.gate_up_q[e, I:]
            return abi.dequant(rows.contiguous(), self.gate_up_fmt, I * H).view(I, H)
        if role == "down":
            return abi.dequant(self.down_q[e].contiguous(), self.down_fmt, H * I).view(H, I)
        raise KeyError(role)
