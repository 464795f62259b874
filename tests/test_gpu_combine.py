"""The combine's arithmetic bit for bit: every product and sum rounded to f32 on its own, addends
in ascending expert id with the weight reached by rank, and x1 + (routed + gate * shared_raw)
(speccheck/moe_ref.py:452-476, :514-517; engine/m3_forward.py:464, :737)."""
import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu


def _bits_equal(a, b, what):
    a, b = a.detach().cpu().contiguous(), b.detach().cpu().contiguous()
    nd = int((a.view(torch.int32) != b.view(torch.int32)).sum())
    assert nd == 0, f"{what}: {nd} of {a.numel()} values differ in their bits"


def test_moe_combine_bit_exact_vs_oracle(pkg, dev):
    """moe_combine on fixed y (sorted-pair order), ids, bf16 weights, shared_raw and gate_prob."""
    g = torch.Generator().manual_seed(21)
    T, K, E, H = 37, 8, 256, 2048
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    w = torch.rand(T, K, generator=g).to(torch.bfloat16)
    grp = pkg.abi.sort_permute(ids.to(dev), E)
    y = torch.randn(T * K, H, generator=g)
    sraw = torch.randn(T, H, generator=g)
    gp = torch.rand(T, generator=g)
    r = pkg.abi.combine(y.to(dev), grp, ids.to(dev), w.to(dev), sraw.to(dev), gp.to(dev), stages=True)
    torch.cuda.synchronize()
    pos = grp["pair_pos"].cpu().long().reshape(T, K)
    raw = y[pos]                                               # [T, K, H] in slot order
    routed = O.routed_combine(raw, ids.long(), w)
    _bits_equal(r["expert_raw"], raw, "expert_raw")
    _bits_equal(r["routed_sum"], routed, "routed_sum")
    _bits_equal(r["shared_out"], gp[:, None] * sraw, "shared_out")
    _bits_equal(r["combined_out"], O.final_add(routed, gp, sraw), "combined_out")


@pytest.mark.parametrize("T,path", [(1, 0), (1, 4), (4, 0), (64, 0)])
def test_block_combine_bits_with_residual(pkg, layer_c0, dev, T, path):
    """Each path's own combine (the single-launch decode layer at T = 1, the three-launch decode
    path, the GEMV path's and the MFMA path's combine kernel) against the oracle's combine
    arithmetic on the path's own stage outputs: routed_sum from expert_raw and the bf16 weights,
    out = residual + (routed_sum + shared_out)."""
    lw, _ = layer_c0
    x = pkg.synth.make_input(T, seed=30 + T, device=dev)
    res = pkg.synth.make_input(T, seed=40 + T, device=dev)
    st = pkg.abi.block_forward(x, lw, path=path, stages=True, residual=res)
    torch.cuda.synchronize()
    routed = O.routed_combine(st["expert_raw"].cpu(), st["topk_ids"].cpu().long(),
                              st["topk_weights"].cpu())
    _bits_equal(st["routed_sum"], routed, f"T={T} routed_sum")
    want = res.cpu() + (st["routed_sum"].cpu() + st["shared_out"].cpu())
    _bits_equal(st["combined_out"], want, f"T={T} out")


@pytest.mark.parametrize("T", [1, 4])
def test_bf16_down_auto_path(pkg, dev, T):
    """Q4_K gate_up with plain bf16 down: MOE_PATH_AUTO must take a path that reads bf16 down
    (the MFMA path) at decode sizes, and the block must match the oracle."""
    from tolerances import assert_close
    lw = pkg.synth.make_layer(seed=11, device=dev, down_fmt=pkg.quant.FMT_BF16)
    ow = O.from_device(lw)
    x = pkg.synth.make_input(T, seed=11, device=dev)
    st = pkg.abi.block_forward(x, lw, stages={"topk_ids", "router_logits"})
    torch.cuda.synchronize()
    ref = O.moe_block(x.cpu(), ow)
    assert torch.equal(st["topk_ids"].cpu().long(), ref["topk_ids"])
    assert_close(st["combined_out"], ref["combined_out"], f"bf16 down T={T}")
