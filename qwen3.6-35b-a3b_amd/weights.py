"""One MoE block's weights, resident on one GPU, in the layout the kernels read.

Mirrors the reference's weight handle (engine/block_forward.py:347-483, `W.get(name)` and
`W.expert_slice('gate'|'up'|'down', e)`) and its geometry dict (engine/block_forward.py:504-531).

HBM layout (all 16-byte aligned, expert axis slowest, as GGUF stores it — engine/loader.py:338-390):
  router           bf16 or f32 [E, H]               read whole every token (the artifact: f32)
  router_bias      f32  [E] or None                 added inside R1 (synthetic skew only)
  gate_up_q        u8   [E, 2I, H/256 * blk]        gate rows 0..I-1 then up rows (spec §11.4), or
                   u8   [E, I, H/256 * blk]         the gate rows alone when up_q is given
  up_q             u8   [E, I, H/256 * blk] or None the separate up tensor (the artifact's
                                                    ffn_up_exps beside ffn_gate_exps)
  down_q           u8   [E, H, I/256 * blk]         Q4_K, Q5_K (the artifact) or Q6_K
  shared_gate/up   bf16 [I_s, H];  shared_down bf16 [H, I_s]; or Q8_0 rows (uint8 [I_s, H/32*34],
                   [H, I_s/32*34]: the artifact's ffn_*_shexp) when shared_fmt is Q8_0
  shared_scalar_gate bf16 or f32 [1, H]             (the artifact: f32)
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
    up_q: torch.Tensor | None = None
    shared_fmt: int = Q.FMT_BF16

    @property
    def n_experts(self) -> int:
        return self.router.shape[0]

    @property
    def hidden(self) -> int:
        return self.router.shape[1]

    @property
    def i_e(self) -> int:
        return self.gate_up_q.shape[1] if self.up_q is not None else self.gate_up_q.shape[1] // 2

    @property
    def default_widths(self) -> bool:
        """bf16 router and scalar gate with a fused gate_up record: moe_block_forward's form."""
        return (self.up_q is None and self.router.dtype == torch.bfloat16
                and self.shared_scalar_gate.dtype == torch.bfloat16 and self.shared_fmt == Q.FMT_BF16)

    @property
    def i_s(self) -> int:
        return self.shared_gate.shape[0]

    @property
    def device(self) -> torch.device:
        return self.router.device

    def routed_bytes_per_expert(self) -> int:
        up = 0 if self.up_q is None else self.up_q[0].numel()
        return self.gate_up_q[0].numel() + up + self.down_q[0].numel()

    def shared_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in
                   (self.shared_gate, self.shared_up, self.shared_down))

    def validate(self) -> None:
        E, H = self.router.shape
        I = self.i_e
        rows = I if self.up_q is not None else 2 * I
        q8 = self.shared_fmt == Q.FMT_Q8_0
        if self.shared_fmt not in (Q.FMT_BF16, Q.FMT_Q8_0):
            raise ValueError(f"shared_fmt must be BF16 or Q8_0, got {self.shared_fmt}")
        sdt = torch.uint8 if q8 else torch.bfloat16
        scols = (lambda c: c // 32 * Q.Q8_0_BYTES) if q8 else (lambda c: c)
        want = {
            "gate_up_q": (self.gate_up_q, torch.uint8, (E, rows, Q.row_bytes(self.gate_up_fmt, H))),
            "down_q": (self.down_q, torch.uint8, (E, H, Q.row_bytes(self.down_fmt, I))),
            "shared_gate": (self.shared_gate, sdt, (self.i_s, scols(H))),
            "shared_up": (self.shared_up, sdt, (self.i_s, scols(H))),
            "shared_down": (self.shared_down, sdt, (H, scols(self.i_s))),
            "shared_scalar_gate": (self.shared_scalar_gate, self.shared_scalar_gate.dtype, (1, H)),
        }
        if self.up_q is not None:
            want["up_q"] = (self.up_q, torch.uint8, (E, I, Q.row_bytes(self.gate_up_fmt, H)))
        for name, (t, dt, shp) in want.items():
            if t.dtype != dt or tuple(t.shape) != tuple(shp) or not t.is_contiguous():
                raise ValueError(f"{name}: got {t.dtype} {tuple(t.shape)}, want {dt} {shp}")
        for name, t in (("router", self.router), ("shared_scalar_gate", self.shared_scalar_gate)):
            if t.dtype not in (torch.bfloat16, torch.float32):
                raise ValueError(f"{name} must be bf16 or f32, got {t.dtype}")

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
            if self.up_q is not None:
                rows = self.gate_up_q[e] if role == "gate" else self.up_q[e]
            else:
                rows = self.gate_up_q[e, :I] if role == "gate" else self.gate_up_q[e, I:]
            return abi.dequant(rows.contiguous(), self.gate_up_fmt, I * H).view(I, H)
        if role == "down":
            return abi.dequant(self.down_q[e].contiguous(), self.down_fmt, H * I).view(H, I)
        raise KeyError(role)

    def split_gate_up(self) -> "LayerWeights":
        """The same weights with gate and up as separate tensors (the artifact's ffn_gate_exps and
        ffn_up_exps records); the bytes are the same bytes."""
        import dataclasses
        I = self.i_e
        if self.up_q is not None:
            return self
        return dataclasses.replace(self, gate_up_q=self.gate_up_q[:, :I].contiguous(),
                                   up_q=self.gate_up_q[:, I:].contiguous())

    def c_struct(self, norm_w: torch.Tensor | None = None):
        """moe_layer_weights for moe_block_forward_w (pointers into these tensors)."""
        from . import _lib as L
        dt = lambda t: L.MOE_DT_F32 if t.dtype == torch.float32 else L.MOE_DT_BF16
        p = lambda t: None if t is None else t.data_ptr()
        return L.LayerWeightsC(
            p(self.router), dt(self.router), p(self.router_bias), p(self.gate_up_q), p(self.up_q),
            self.gate_up_fmt, p(self.down_q), self.down_fmt, p(self.shared_gate), p(self.shared_up),
            p(self.shared_down), self.shared_fmt, p(self.shared_scalar_gate),
            dt(self.shared_scalar_gate), p(norm_w))
