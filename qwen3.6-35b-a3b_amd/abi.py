"""Python face of the C-ABI: argument validation, workspace and stream plumbing, named refusals.

Every function here takes and returns torch tensors that live on one GPU and launches work on
the current HIP stream; none of them copies routing values to the host. Errors come back as
`Refused(tag, msg)`, the reference's error shape (engine/block_forward.py:109-114).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L


class Refused(Exception):
    """A call the library would not make. `tag` names the reason."""

    def __init__(self, tag: str, msg: str):
        super().__init__(f"{tag}: {msg}")
        self.tag = tag


def _check(rc: int, who: str) -> None:
    if rc != L.MOE_OK:
        text = L.lib.moe_last_error().decode(errors="replace")
        raise Refused(L.ERROR_NAMES.get(rc, f"error{rc}"), f"{who}: {text}")


def _p(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _need(t: torch.Tensor, name: str, dtype=None, shape=None, device=None):
    if not isinstance(t, torch.Tensor):
        raise Refused("bad-argument", f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise Refused("bad-argument", f"{name} must live on the GPU (got {t.device})")
    if device is not None and t.device != device:
        raise Refused("bad-argument", f"{name} is on {t.device}, expected {device}")
    if dtype is not None and t.dtype != dtype:
        raise Refused("bad-argument", f"{name} has dtype {t.dtype}, expected {dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise Refused("bad-argument", f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise Refused("bad-argument", f"{name} must be contiguous")
    return t


def _wdt(t: torch.Tensor, name: str) -> int:
    """bf16 or f32 weight vectors / matrices (router, scalar shared gate)."""
    if t.dtype == torch.float32:
        return L.MOE_DT_F32
    if t.dtype == torch.bfloat16:
        return L.MOE_DT_BF16
    raise Refused("bad-argument", f"{name} must be bfloat16 or float32, got {t.dtype}")


def _xdt(x: torch.Tensor) -> int:
    if x.dtype == torch.float32:
        return L.MOE_DT_F32
    if x.dtype == torch.bfloat16:
        return L.MOE_DT_BF16
    raise Refused("bad-argument", f"activations must be float32 or bfloat16, got {x.dtype}")


_WS_CACHE: dict = {}


def _ws_key(device: torch.device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return idx, torch.cuda.current_stream(torch.device("cuda", idx)).cuda_stream


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A cached scratch buffer of at least nbytes for (device, the current stream), allocated by
    torch (not the library) and initialised on that stream. Calls that share a workspace must be
    ordered on one stream, so each stream gets its own."""
    key = _ws_key(device)
    buf = _WS_CACHE.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _check(L.lib.moe_workspace_init(_p(buf), buf.numel(), ctypes.c_void_p(key[1])),
               "workspace_init")
        _WS_CACHE[key] = buf
    return buf


def workspace_bytes(T: int, H: int, I: int, E: int, K: int, I_s: int) -> int:
    return int(L.lib.moe_workspace_bytes(T, H, I, E, K, I_s))


def workspace_status(device) -> int:
    """moe_workspace_status of the current stream's workspace on `device`: the status bits since the
    last read (bit MOE_STATUS_SPIN_TIMEOUT: a bounded wait of the single-launch decode layer gave
    up, and the rows of the workgroups that gave up are NaN), then cleared. 0 when no workspace
    exists yet. Stream-ordered in the library; this helper then synchronises to return the value."""
    key = _ws_key(device)
    buf = _WS_CACHE.get(key)
    if buf is None:
        return 0
    out = torch.empty(1, dtype=torch.int32, device=device)
    _check(L.lib.moe_workspace_status(_p(buf), buf.numel(), _p(out), ctypes.c_void_p(key[1])),
           "workspace_status")
    return int(out.item())


def set_test_hook(device, on: bool) -> None:
    """Sets the current stream's workspace's test-hook word: while on, every bounded wait of the
    single-launch decode layer reports a timeout after completing (include/moe_gfx950.h)."""
    buf = workspace(device, L.SYNC_BYTES)
    buf[4 * L.TEST_HOOK_WORD:4 * L.TEST_HOOK_WORD + 4].view(torch.int32).fill_(1 if on else 0)


def device_error_bits(device) -> int:
    """The status bits of every workspace this module holds on `device`, OR-ed, each read and
    cleared (moe_workspace_status); 0 when every launch since the last read ran as designed.
    Synchronises the device first, so work on any stream (graph replays included) is counted."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    torch.cuda.synchronize(idx)
    st = ctypes.c_void_p(torch.cuda.current_stream(torch.device("cuda", idx)).cuda_stream)
    bufs = [b for (d, _), b in _WS_CACHE.items() if d == idx]
    if not bufs:
        return 0
    out = torch.zeros(len(bufs), dtype=torch.int32, device=device)
    for i, buf in enumerate(bufs):
        _check(L.lib.moe_workspace_status(_p(buf), buf.numel(), _p(out[i:i + 1]), st), "workspace_status")
    bits = 0
    for v in out.tolist():
        bits |= int(v)
    return bits


# ---------------------------------------------------------------------------------- entry points
def dequant(blocks: torch.Tensor, fmt: int, n_elts: int, out_dtype=torch.float32) -> torch.Tensor:
    """Bit-exact decode of `n_elts` elements of GGUF super-blocks -> f32 / bf16 [n_elts]."""
    _need(blocks, "blocks", torch.uint8)
    out = torch.empty(n_elts, dtype=out_dtype, device=blocks.device)
    odt = L.MOE_DT_F32 if out_dtype == torch.float32 else L.MOE_DT_BF16
    _check(L.lib.moe_dequant(_p(blocks), fmt, n_elts, _p(out), odt, _stream(blocks)), "dequant")
    return out


def router_topk(x: torch.Tensor, w_router: torch.Tensor, top_k: int,
                bias: torch.Tensor | None = None, want_probs: bool = False) -> dict:
    """R1-R5 (speccheck/moe_ref.py:318-363). Returns logits (bf16), ids (int32), w_f32, w_bf16.
    w_router is bf16 or f32 (the artifact's F32 ffn_gate_inp)."""
    _need(x, "x")
    T, H = x.shape
    E = w_router.shape[0]
    wdt = _wdt(w_router, "w_router")
    _need(w_router, "w_router", None, (E, H), x.device)
    if bias is not None:
        _need(bias, "logit_bias", torch.float32, (E,), x.device)
    dev = x.device
    logits = torch.empty(T, E, dtype=torch.bfloat16, device=dev)
    probs = torch.empty(T, E, dtype=torch.float32, device=dev) if want_probs else None
    ids = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    wf = torch.empty(T, top_k, dtype=torch.float32, device=dev)
    wb = torch.empty(T, top_k, dtype=torch.bfloat16, device=dev)
    ws = workspace(dev, int(L.lib.moe_router_workspace_bytes(T, H, E)))
    _check(L.lib.moe_router_topk(_p(x), _xdt(x), _p(w_router), wdt, _p(bias), T, H, E, top_k,
                                 _p(logits), _p(probs), _p(ids), _p(wf), _p(wb), _p(ws),
                                 ws.numel(), _stream(x)), "router_topk")
    return {"router_logits": logits, "router_probs": probs, "topk_ids": ids,
            "topk_weights": wb, "topk_weights_f32": wf}


def sort_permute(ids: torch.Tensor, n_experts: int) -> dict:
    """Stable grouping of (token, slot) pairs by expert id (torch.argsort(stable=True) order)."""
    _need(ids, "topk_ids", torch.int32)
    T, K = ids.shape
    dev = ids.device
    P = T * K
    off = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    srt = torch.empty(P, dtype=torch.int32, device=dev)
    pos = torch.empty(P, dtype=torch.int32, device=dev)
    hits = torch.empty(n_experts + 1, dtype=torch.int32, device=dev)
    # the sync words, then one int32 histogram row per 1024-pair chunk
    ws = workspace(dev, L.SYNC_BYTES + ((P + 1023) // 1024 * n_experts * 4 + 255) // 256 * 256)
    _check(L.lib.moe_sort_permute(_p(ids), T, K, n_experts, _p(off), _p(srt), _p(pos), _p(hits),
                                  _p(ws), ws.numel(), _stream(ids)), "sort_permute")
    return {"expert_offsets": off, "sorted_pairs": srt, "pair_pos": pos, "hit_list": hits}


def experts(x: torch.Tensor, gate_up_q: torch.Tensor, gate_up_fmt: int, down_q: torch.Tensor,
            down_fmt: int, grouping: dict, top_k: int, path: int = L.MOE_PATH_AUTO,
            up_q: torch.Tensor | None = None) -> torch.Tensor:
    """y [T*K, H] f32 in sorted-pair order (expert_raw before the routing weight). gate_up_q is the
    fused [E, 2I, ...] record, or the gate rows [E, I, ...] when up_q (the up rows) is given."""
    _need(x, "x")
    T, H = x.shape
    _need(gate_up_q, "gate_up_q", torch.uint8, device=x.device)
    _need(down_q, "down_q", torch.uint8, device=x.device)
    if up_q is not None:
        _need(up_q, "up_q", torch.uint8, tuple(gate_up_q.shape), x.device)
    E = gate_up_q.shape[0]
    I = gate_up_q.shape[1] if up_q is not None else gate_up_q.shape[1] // 2
    y = torch.empty(T * top_k, H, dtype=torch.float32, device=x.device)
    ws = workspace(x.device, workspace_bytes(T, H, I, E, top_k, I))
    _check(L.lib.moe_experts(_p(x), _xdt(x), _p(gate_up_q), _p(up_q), gate_up_fmt, _p(down_q), down_fmt,
                             _p(grouping["expert_offsets"]), _p(grouping["sorted_pairs"]),
                             _p(grouping["hit_list"]), T, H, I, E, top_k, path, _p(y), _p(ws),
                             ws.numel(), _stream(x)), "experts")
    return y


def shared_expert(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
                  w_scalar_gate: torch.Tensor, path: int = L.MOE_PATH_AUTO):
    """(shared_raw [T,H] f32, gate_prob [T] f32). The expert's rows are bf16 ([I_s,H], [I_s,H],
    [H,I_s]) or Q8_0 bytes (uint8 [I_s,H/32*34], [I_s,H/32*34], [H,I_s/32*34]: the artifact's
    ffn_*_shexp); w_scalar_gate is bf16 or f32 (the artifact's F32 ffn_gate_inp_shexp)."""
    _need(x, "x")
    T, H = x.shape
    Is = w_gate.shape[0]
    q8 = w_gate.dtype == torch.uint8
    sfmt = L.MOE_FMT_Q8_0 if q8 else L.MOE_FMT_BF16
    cols = (lambda c: c // 32 * 34) if q8 else (lambda c: c)
    for n, t, shp in (("w_gate", w_gate, (Is, cols(H))), ("w_up", w_up, (Is, cols(H))),
                      ("w_down", w_down, (H, cols(Is)))):
        _need(t, n, torch.uint8 if q8 else torch.bfloat16, shp, x.device)
    gdt = _wdt(w_scalar_gate, "w_scalar_gate")
    _need(w_scalar_gate, "w_scalar_gate", None, (1, H), x.device)
    raw = torch.empty(T, H, dtype=torch.float32, device=x.device)
    prob = torch.empty(T, dtype=torch.float32, device=x.device)
    ws = workspace(x.device, workspace_bytes(T, H, Is, 256, 8, Is))
    _check(L.lib.moe_shared_expert(_p(x), _xdt(x), _p(w_gate), _p(w_up), _p(w_down),
                                   sfmt, _p(w_scalar_gate), gdt, T, H, Is, path, _p(raw),
                                   _p(prob), _p(ws), ws.numel(), _stream(x)), "shared_expert")
    return raw, prob


def combine(y: torch.Tensor, grouping: dict, ids: torch.Tensor, w_bf16: torch.Tensor,
            shared_raw: torch.Tensor, gate_prob: torch.Tensor, stages: bool = False) -> dict:
    """Ascending-expert-id weighted combine + gated shared expert."""
    T, K = ids.shape
    H = y.shape[1]
    dev = y.device
    out = torch.empty(T, H, dtype=torch.float32, device=dev)
    routed = torch.empty(T, H, dtype=torch.float32, device=dev) if stages else None
    shared_out = torch.empty(T, H, dtype=torch.float32, device=dev) if stages else None
    raw = torch.empty(T, K, H, dtype=torch.float32, device=dev) if stages else None
    _check(L.lib.moe_combine(_p(y), _p(grouping["pair_pos"]), _p(ids), _p(w_bf16),
                             _p(shared_raw), _p(gate_prob), T, K, H, _p(out), _p(routed),
                             _p(shared_out), _p(raw), _stream(y)), "combine")
    return {"combined_out": out, "routed_sum": routed, "shared_out": shared_out, "expert_raw": raw}


def _need_layer(lw, H: int, dev, tag: str) -> None:
    """Device, dtype and leading-shape checks of a LayerWeights passed by descriptor."""
    E = lw.router.shape[0]
    _wdt(lw.router, tag + "router")
    _need(lw.router, tag + "router", None, (E, H), dev)
    _wdt(lw.shared_scalar_gate, tag + "shared_scalar_gate")
    _need(lw.shared_scalar_gate, tag + "shared_scalar_gate", None, (1, H), dev)
    sdt = torch.uint8 if lw.shared_fmt == L.MOE_FMT_Q8_0 else torch.bfloat16
    for n in ("shared_gate", "shared_up", "shared_down"):
        _need(getattr(lw, n), tag + n, sdt, device=dev)
    for n in ("gate_up_q", "down_q"):
        _need(getattr(lw, n), tag + n, torch.uint8, device=dev)
    if lw.up_q is not None:
        _need(lw.up_q, tag + "up_q", torch.uint8, tuple(lw.gate_up_q.shape), dev)
    if lw.router_bias is not None:
        _need(lw.router_bias, tag + "router_bias", torch.float32, (E,), dev)


def block_forward(x: torch.Tensor, lw, path: int = L.MOE_PATH_AUTO, stages=False,
                  out: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                  norm_w: torch.Tensor | None = None, norm_eps: float = 1e-6,
                  next_layer=None, next_norm_w: torch.Tensor | None = None) -> dict:
    """The whole block in one library call (moe_block_forward). `lw` is a LayerWeights;
    `stages` is False, True (every stage output) or a set of stage names to return;
    out = residual + MoE(input) when `residual` (f32 [T,H], may be `out` or `x` itself) is given.
    input = x, or the post-attention RMSNorm of x when `norm_w` (f32 [H], the artifact's 1+w) is
    given: engine/m3_forward.py:732-737 is then block_forward(x1, lw, norm_w=w, residual=x1).
    `next_layer` (a LayerWeights, optional) is the layer this stream runs next and `next_norm_w`
    its norm weight: its router rows and that norm weight are warmed into L2 by the single-launch
    decode layer (moe_block_forward_prefetch); results do not depend on them. Weights in other
    widths than the bf16 router / fused gate_up / bf16 scalar gate (the artifact's F32 router and
    scalar gate, separate gate and up tensors) go through moe_block_forward_w."""
    _need(x, "x")
    T, H = x.shape
    if norm_w is not None:
        _need(norm_w, "norm_w", torch.float32, (H,), x.device)
    E, K, I, Is = lw.n_experts, lw.top_k, lw.i_e, lw.i_s
    dev = x.device
    if out is None:
        out = torch.empty(T, H, dtype=torch.float32, device=dev)
    if residual is not None:
        _need(residual, "residual", torch.float32, (T, H), dev)
    shapes = {"router_logits": ((T, E), torch.bfloat16), "topk_ids": ((T, K), torch.int32),
              "topk_weights": ((T, K), torch.bfloat16),
              "topk_weights_f32": ((T, K), torch.float32),
              "routed_sum": ((T, H), torch.float32), "shared_out": ((T, H), torch.float32),
              "shared_gate_prob": ((T,), torch.float32),
              "expert_raw": ((T, K, H), torch.float32)}
    want = set(shapes) if stages is True else (set(stages) if stages else set())
    st = {n: torch.empty(*shapes[n][0], dtype=shapes[n][1], device=dev) for n in want}
    ws = workspace(dev, workspace_bytes(T, H, I, E, K, Is))
    g = st.get
    if not lw.default_widths or (next_layer is not None and not next_layer.default_widths):
        _need_layer(lw, H, dev, "")
        if next_layer is not None:
            _need_layer(next_layer, H, dev, "next ")
            if next_norm_w is not None:
                _need(next_norm_w, "next_norm_w", torch.float32, (H,), dev)
        W = lw.c_struct(norm_w)
        N = next_layer.c_struct(next_norm_w) if next_layer is not None else None
        _check(L.lib.moe_block_forward_w(
            _p(x), _xdt(x), T, H, I, E, K, Is, ctypes.byref(W), float(norm_eps), path, _p(residual),
            _p(out), _p(g("router_logits")), _p(g("topk_ids")), _p(g("topk_weights")),
            _p(g("topk_weights_f32")), _p(g("routed_sum")), _p(g("shared_out")),
            _p(g("shared_gate_prob")), _p(g("expert_raw")), _p(ws), ws.numel(), _stream(x),
            None if N is None else ctypes.byref(N)), "block_forward")
        st["combined_out"] = out
        return st
    args = (
        _p(x), _xdt(x), T, H, I, E, K, Is, _p(norm_w), float(norm_eps), _p(lw.router), _p(lw.router_bias), _p(lw.gate_up_q),
        lw.gate_up_fmt, _p(lw.down_q), lw.down_fmt, _p(lw.shared_gate), _p(lw.shared_up),
        _p(lw.shared_down), _p(lw.shared_scalar_gate), path, _p(residual), _p(out),
        _p(g("router_logits")),
        _p(g("topk_ids")), _p(g("topk_weights")), _p(g("topk_weights_f32")), _p(g("routed_sum")),
        _p(g("shared_out")), _p(g("shared_gate_prob")), _p(g("expert_raw")), _p(ws), ws.numel(),
        _stream(x))
    if next_layer is None:
        _check(L.lib.moe_block_forward(*args), "block_forward")
    else:
        nl = next_layer
        _need(nl.router, "next router", device=dev)
        if next_norm_w is not None:
            _need(next_norm_w, "next_norm_w", torch.float32, (H,), dev)
        hint = L.NextLayer(nl.router.data_ptr(), None if next_norm_w is None else next_norm_w.data_ptr())
        _check(L.lib.moe_block_forward_prefetch(*args, ctypes.byref(hint)), "block_forward")
    st["combined_out"] = out
    return st


def lm_head(h: torch.Tensor, table: torch.Tensor, fmt: int,
            row_ids: torch.Tensor | None = None) -> torch.Tensor:
    """Untied lm_head GEMV (moe_lm_head): logits f32 [B, n] = h [B, 2048] (f32 or bf16, B <= 8)
    against the table rows (all V rows, or row_ids int32 [n] for the gather form).
    table: uint8 [V, row_bytes] for MOE_FMT_Q6_K / MOE_FMT_Q8_0, bfloat16 [V, 2048] for
    MOE_FMT_BF16. Replaces prototype/lm_head/lm_head_kernels.h:474-512 (lmh_dot_batch)."""
    _need(h, "h")
    B, H = h.shape
    dev = h.device
    if fmt == L.MOE_FMT_BF16:
        _need(table, "table", torch.bfloat16, device=dev)
    else:
        _need(table, "table", torch.uint8, device=dev)
    V = table.shape[0]
    if row_ids is not None:
        _need(row_ids, "row_ids", torch.int32, device=dev)
        n = row_ids.numel()
    else:
        n = V
    out = torch.empty(B, n, dtype=torch.float32, device=dev)
    _check(L.lib.moe_lm_head(_p(h), _xdt(h), B, H, _p(table), fmt, V, _p(row_ids), n, _p(out),
                             _stream(h)), "lm_head")
    return out
