"""Whole-block parity on BASELINE.json's configs (c0-c4) and the reference call surfaces."""
import pytest
import torch

from oracle import moe_oracle as O
from tolerances import assert_close

pytestmark = pytest.mark.gpu


def _compare(st, ref, rows=None, tag=""):
    ids = st["topk_ids"].cpu().long()
    lg = st["router_logits"].cpu()
    if rows is not None:
        ids, lg = ids[rows], lg[rows]
    assert torch.equal(lg.view(torch.int16), ref["router_logits"].view(torch.int16)), f"{tag} logits"
    assert torch.equal(ids, ref["topk_ids"]), f"{tag} ids"
    out = st["combined_out"].cpu()
    out = out[rows] if rows is not None else out
    assert_close(out, ref["combined_out"], f"{tag} combined_out")


def test_c0_decode_block(pkg, layer_c0, dev):
    lw, ow = layer_c0
    x = pkg.synth.make_input(1, seed=0, device=dev)
    st = pkg.block.moe_block(x, lw, pkg.load_geometry())
    ref = O.moe_block(x.cpu(), ow)
    _compare(st, ref, tag="c0")
    assert_close(st["routed_sum"], ref["routed_sum"], "c0 routed_sum")
    assert_close(st["shared_out"], ref["shared_out"], "c0 shared_out")
    assert_close(st["expert_raw"], ref["expert_raw"], "c0 expert_raw")


def test_c2_batched_decode_zipf(pkg, layer_zipf, dev):
    lw, ow = layer_zipf
    x = pkg.synth.make_input(64, seed=1, device=dev)
    for path in (1, 2):
        st = pkg.block.moe_block(x, lw, pkg.load_geometry(), path=path)
        ref = O.moe_block(x.cpu(), ow)
        _compare(st, ref, tag=f"c2 path={path}")


def test_c3_prefill_sampled_rows(pkg, layer_c0, dev):
    """T = 4096 bf16 activations on the MFMA path; the block is row-independent, so the oracle
    checks a seeded sample of 192 rows of the full-size run."""
    lw, ow = layer_c0
    x = pkg.synth.make_input(4096, seed=2, device=dev, dtype=torch.bfloat16)
    st = pkg.block.moe_block(x, lw, pkg.load_geometry())
    rows = torch.randperm(4096, generator=torch.Generator().manual_seed(2))[:192]
    ref = O.moe_block(x.cpu()[rows], ow)
    _compare(st, ref, rows=rows, tag="c3")


def test_c4_prefill_q6k_sampled_rows(pkg, layer_q6k, dev):
    lw, ow = layer_q6k
    x = pkg.synth.make_input(16384, seed=3, device=dev, dtype=torch.bfloat16)
    st = pkg.block.moe_block(x, lw, pkg.load_geometry())
    rows = torch.randperm(16384, generator=torch.Generator().manual_seed(3))[:128]
    ref = O.moe_block(x.cpu()[rows], ow)
    _compare(st, ref, rows=rows, tag="c4")


def test_reference_surfaces_agree(pkg, layer_c0, dev):
    """moe_router + moe_shared + moe_routed (engine/block_forward.py:614-667) compose to the same
    block as moe_block, and moe_block_m3 matches too."""
    lw, _ = layer_c0
    cfg = pkg.load_geometry()
    x = pkg.synth.make_input(3, seed=9, device=dev)
    r = pkg.block.moe_router(x, lw, cfg)
    s = pkg.block.moe_shared(x, lw, cfg)
    ro = pkg.block.moe_routed(x, lw, cfg, r)
    whole = pkg.block.moe_block(x, lw, cfg)
    torch.cuda.synchronize()
    assert torch.equal(r["topk_ids"], whole["topk_ids"])
    comb = ro["routed_sum"] + s["shared_out"]
    assert torch.allclose(comb, whole["combined_out"], rtol=0, atol=1e-6)
    out, info = pkg.block.moe_block_m3(x.view(1, 3, -1), pkg.block.DeviceLayers([lw]), 0)
    assert torch.equal(out.view(3, -1), whole["combined_out"])
    assert torch.equal(info["ids"].view(3, -1), whole["topk_ids"])
    assert int(info["used"]) == len(torch.unique(whole["topk_ids"]))


def test_deterministic_repeat(pkg, layer_c0, dev):
    lw, _ = layer_c0
    x = pkg.synth.make_input(64, seed=4, device=dev)
    a = pkg.abi.block_forward(x, lw)["combined_out"].clone()
    b = pkg.abi.block_forward(x, lw)["combined_out"]
    assert torch.equal(a, b)
