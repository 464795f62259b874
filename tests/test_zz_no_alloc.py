"""moe_block_forward_w_noalloc: the allocation-free variant of moe_block_forward_w (static device
scratch inside the library). Called through the C-ABI and checked bit for bit against
moe_block_forward_w with a caller workspace, on consecutive calls that shrink."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "moe_gfx950.h"


def test_scratch_bound_matches_the_header(pkg):
    L = pkg._lib
    text = HEADER.read_text()
    assert int(re.search(r"MOE_NOALLOC_MAX_T (\d+)", text).group(1)) == L.NOALLOC_MAX_T
    assert "MOE_NOALLOC_SCRATCH_BYTES (16u << 20)" in text and L.NOALLOC_SCRATCH_BYTES == 16 << 20
    ws = lambda T: L.lib.moe_workspace_bytes(T, 2048, 512, 256, 8, 512)
    assert ws(L.NOALLOC_MAX_T) <= L.NOALLOC_SCRATCH_BYTES < ws(L.NOALLOC_MAX_T + 1)


def test_too_many_tokens_refused_before_any_device_work(pkg):
    """One token over the limit: MOE_E_WORKSPACE, decided on the host (no GPU needed)."""
    L = pkg._lib
    W = L.LayerWeightsC()
    rc = L.lib.moe_block_forward_w_noalloc(
        None, L.MOE_DT_F32, L.NOALLOC_MAX_T + 1, 2048, 512, 256, 8, 512, ctypes.byref(W), 1e-6, 0,
        None, None, None, None, None, None, None, None, None, None, None, None)
    assert rc == L.MOE_E_WORKSPACE
    assert b"static scratch" in L.lib.moe_last_error()


def _call(pkg, fn, x, lw, norm_w, residual, ws=None):
    """One block through moe_block_forward_w (ws given) or _noalloc, every stage requested."""
    L, abi = pkg._lib, pkg.abi
    T, H = x.shape
    E, K, I, Is = lw.n_experts, lw.top_k, lw.i_e, lw.i_s
    dev = x.device
    out = torch.full((T, H), float("nan"), device=dev)
    st = {"logits": torch.empty(T, E, dtype=torch.bfloat16, device=dev),
          "ids": torch.empty(T, K, dtype=torch.int32, device=dev),
          "wb": torch.empty(T, K, dtype=torch.bfloat16, device=dev),
          "wf": torch.empty(T, K, dtype=torch.float32, device=dev),
          "routed": torch.empty(T, H, device=dev), "shared": torch.empty(T, H, device=dev),
          "gp": torch.empty(T, device=dev), "raw": torch.empty(T, K, H, device=dev)}
    W = lw.c_struct(norm_w)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    args = [p(x), L.MOE_DT_F32, T, H, I, E, K, Is, ctypes.byref(W), 1e-6, L.MOE_PATH_AUTO, p(residual),
            p(out), p(st["logits"]), p(st["ids"]), p(st["wb"]), p(st["wf"]), p(st["routed"]),
            p(st["shared"]), p(st["gp"]), p(st["raw"])]
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if fn == "w":
        rc = L.lib.moe_block_forward_w(*args, p(ws), ws.numel(), stream, None)
    else:
        rc = L.lib.moe_block_forward_w_noalloc(*args, stream, None)
    assert rc == L.MOE_OK, L.lib.moe_last_error()
    st["out"] = out
    return st


def _same_bits(a, b, what):
    a, b = a.cpu().contiguous(), b.cpu().contiguous()
    n = a.element_size()
    view = {4: torch.int32, 2: torch.int16}[n]
    assert torch.equal(a.view(view), b.view(view)), what


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_on_shrinking_calls(pkg, dev):
    """Calls in a row on one device, each against moe_block_forward_w:
    - T = 120 and then 64 with Q6_K down (config 4's weights) and T = 64 with the artifact's widths
      (Q5_K down, Q8_0 shared expert, f32 router and scalar gate, split gate/up, the norm in
      front): here the workspace entry forks the shared expert onto its second stream and the
      no-alloc entry runs it on the caller's stream, so these compare the forked and the one-stream
      orders;
    - T = 64 with Q4_K routed and bf16 shared weights (Zipf routing): both entries fold the shared
      expert into the router and routed launches (one stream);
    - T = 4 (GEMV path) and T = 1 (the single-launch decode layer, norm and residual fused)."""
    synth, abi, Q = pkg.synth, pkg.abi, pkg.quant
    lz = synth.make_layer(seed=1, device=dev, zipf=True)
    l0 = synth.make_layer(seed=0, device=dev)
    l6 = synth.make_layer(seed=3, device=dev, down_fmt=Q.FMT_Q6_K, zipf=True)
    la = synth.make_layer(seed=7, device=dev, down_fmt=Q.FMT_Q5_K, zipf=True,
                          router_dtype=torch.float32, scalar_gate_dtype=torch.float32,
                          split_gate_up=True, shared_fmt=Q.FMT_Q8_0)
    nw = synth.make_norm_weight(seed=5000, device=dev)
    ws = abi.workspace(dev, abi.workspace_bytes(120, 2048, 512, 256, 8, 512))
    for T, lw, norm in ((120, l6, None), (64, l6, None), (64, la, nw), (64, lz, None), (4, l0, nw),
                        (1, l0, nw), (1, lz, nw)):
        x = synth.make_input(T, seed=100 + T, device=dev)
        res = synth.make_input(T, seed=200 + T, device=dev) if norm is not None else None
        print(f"noalloc T={T} norm={norm is not None}", flush=True)
        a = _call(pkg, "noalloc", x, lw, norm, res)
        b = _call(pkg, "w", x, lw, norm, res, ws=ws)
        torch.cuda.synchronize()
        assert torch.isfinite(a["out"]).all()
        for k in a:
            _same_bits(a[k], b[k], f"T={T} {k}")
    assert abi.device_error_bits(dev) == 0
