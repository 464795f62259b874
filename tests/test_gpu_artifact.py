"""The shipped artifact's weight widths (engine/block_forward.py:221-231, policy A): F32 router,
F32 scalar shared gate, separate gate and up expert records, Q5_K down. Routing bit-exact against
the correctly rounded oracle, block outputs within the block tolerance, and the split records
giving the same bits as the fused record they were cut from."""
import pytest
import torch

from oracle import moe_oracle as O
from tolerances import assert_close

pytestmark = pytest.mark.gpu


def _norm_weight(seed, H, dev):
    g = torch.Generator().manual_seed(seed)
    return (1.0 + 0.1 * torch.randn(H, generator=g)).to(dev)


@pytest.mark.parametrize("T,dtype", [(1, torch.float32), (9, torch.float32), (64, torch.float32),
                                     (300, torch.bfloat16), (4096, torch.bfloat16)])
def test_f32_router_bit_exact(pkg, layer_artifact, dev, T, dtype):
    """R1 over f32 router rows (f32 x f32 products are exact in f64, so the certified dot needs
    no change) on every router kernel: the small-T GEMV, the MFMA tile kernel and the large-T
    GEMM; logits and ids bit-exact, weights as the R4/R5 functions of them."""
    lw, _ = layer_artifact
    assert lw.router.dtype == torch.float32
    x = pkg.synth.make_input(T, seed=700 + T, device=dev, dtype=dtype)
    r = pkg.abi.router_topk(x, lw.router, 8, lw.router_bias)
    torch.cuda.synchronize()
    ref = O.route(x.cpu(), lw.router.cpu(), 8, lw.router_bias.cpu())
    got = r["router_logits"].cpu()
    assert torch.equal(got.view(torch.int16), ref["router_logits"].view(torch.int16)), \
        f"{(got != ref['router_logits']).sum().item()} logits differ"
    assert torch.equal(r["topk_ids"].cpu().long(), ref["topk_ids"])
    assert torch.allclose(r["topk_weights_f32"].cpu(), ref["topk_weights_f32"], rtol=4e-6, atol=0)


def test_f32_router_differs_from_its_bf16_rounding(pkg, layer_artifact, dev):
    """The f32 rows are used as f32: rounding them to bf16 first changes some logits (a kernel that
    read the f32 tensor as bf16 pairs, or rounded it, would fail the bit-exact test above)."""
    lw, _ = layer_artifact
    x = pkg.synth.make_input(64, seed=777, device=dev)
    a = pkg.abi.router_topk(x, lw.router, 8, lw.router_bias)["router_logits"]
    b = pkg.abi.router_topk(x, lw.router.to(torch.bfloat16), 8, lw.router_bias)["router_logits"]
    torch.cuda.synchronize()
    assert (a != b).sum().item() > 0


@pytest.mark.parametrize("T,path,dtype", [(1, 1, torch.float32), (16, 1, torch.float32),
                                          (64, 2, torch.float32), (257, 2, torch.bfloat16),
                                          (64, 3, torch.float32)])
def test_q8_0_shared_expert_and_f32_scalar_gate(pkg, layer_artifact, dev, T, path, dtype):
    """The shared expert on Q8_0 rows (GEMV at small T; the 160-row f16 MFMA kernels otherwise,
    also under MOE_PATH_MFMA_BF16) and the f32 scalar gate, against the oracle's exact d * q."""
    lw, ow = layer_artifact
    assert lw.shared_scalar_gate.dtype == torch.float32 and lw.shared_gate.dtype == torch.uint8
    x = pkg.synth.make_input(T, seed=720 + T, device=dev, dtype=dtype)
    raw, prob = pkg.abi.shared_expert(x, lw.shared_gate, lw.shared_up, lw.shared_down,
                                      lw.shared_scalar_gate, path)
    torch.cuda.synchronize()
    s = O.shared_expert(x.cpu(), ow)
    assert_close(raw, s["shared_raw"], f"shared_raw T={T} path={path}")
    assert torch.allclose(prob.cpu(), s["shared_gate_prob"].view(-1), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("T,path", [(1, 1), (9, 1), (160, 2), (64, 3)])
def test_split_gate_up_same_bits_as_fused(pkg, layer_c0, dev, T, path):
    """Separate gate and up tensors (the same bytes, cut apart) give the fused record's bits on
    every expert path: GEMV, the 160-row MFMA kernels and the bf16-operand MFMA kernel."""
    lw, _ = layer_c0
    sp = lw.split_gate_up()
    assert sp.up_q is not None and sp.gate_up_q.data_ptr() != lw.gate_up_q.data_ptr()
    x = pkg.synth.make_input(T, seed=740 + T, device=dev)
    r = pkg.abi.router_topk(x, lw.router, 8, lw.router_bias)
    gr = pkg.abi.sort_permute(r["topk_ids"], lw.n_experts)
    a = pkg.abi.experts(x, lw.gate_up_q, lw.gate_up_fmt, lw.down_q, lw.down_fmt, gr, 8, path)
    b = pkg.abi.experts(x, sp.gate_up_q, sp.gate_up_fmt, sp.down_q, sp.down_fmt, gr, 8, path,
                        up_q=sp.up_q)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_split_gate_up_decode_paths_same_bits(pkg, layer_c0, dev):
    """Single tokens through the single-launch layer and the three-launch form: the split record
    reproduces the fused record's block output and routing bit for bit."""
    lw, _ = layer_c0
    sp = lw.split_gate_up()
    for path in (pkg._lib.MOE_PATH_GEMV, pkg._lib.MOE_PATH_GEMV_MULTI):
        for seed in range(4):
            x = pkg.synth.make_input(1, seed=760 + seed, device=dev)
            a = pkg.abi.block_forward(x, lw, path=path, stages={"topk_ids"})
            b = pkg.abi.block_forward(x, sp, path=path, stages={"topk_ids"})
            torch.cuda.synchronize()
            assert torch.equal(a["topk_ids"], b["topk_ids"]), (path, seed)
            assert torch.equal(a["combined_out"], b["combined_out"]), (path, seed)
    assert pkg.abi.device_error_bits(dev) == 0


def _compare(st, ref, tag, rows=None):
    ids, lg, out = st["topk_ids"].cpu().long(), st["router_logits"].cpu(), st["combined_out"].cpu()
    if rows is not None:
        ids, lg, out = ids[rows], lg[rows], out[rows]
    assert torch.equal(lg.view(torch.int16), ref["router_logits"].view(torch.int16)), tag
    assert torch.equal(ids, ref["topk_ids"]), tag
    assert_close(out, ref["combined_out"], f"{tag} combined_out")


def test_artifact_block_decode(pkg, layer_artifact, dev):
    """moe_block_forward_w at T = 1 with every artifact width, through the reference surface."""
    lw, ow = layer_artifact
    assert not lw.default_widths
    for seed in range(4):
        x = pkg.synth.make_input(1, seed=780 + seed, device=dev)
        st = pkg.block.moe_block(x, lw, pkg.load_geometry())
        ref = O.moe_block(x.cpu(), ow)
        _compare(st, ref, f"artifact decode seed={seed}")
        assert_close(st["shared_out"], ref["shared_out"], "artifact shared_out")
        assert_close(st["expert_raw"], ref["expert_raw"], "artifact expert_raw")


def test_artifact_residual_step_with_norm(pkg, layer_artifact, dev):
    """engine/m3_forward.py:732-737 on the artifact widths: x1 + MoE(rmsnorm_a(x1, w)) in place."""
    lw, ow = layer_artifact
    w = _norm_weight(79, 2048, dev)
    x1 = pkg.synth.make_input(3, seed=79, device=dev) * 5.0
    ref = O.residual_step(x1.cpu(), ow, w.cpu(), 1e-6)
    for i in range(3):
        h = x1[i:i + 1].clone()
        st = pkg.abi.block_forward(h, lw, stages={"topk_ids"}, out=h, residual=h, norm_w=w)
        torch.cuda.synchronize()
        assert torch.equal(st["topk_ids"].cpu().long(), ref["topk_ids"][i:i + 1]), i
        assert_close(h.cpu() - x1[i:i + 1].cpu(), ref["combined_out"][i:i + 1], f"token {i}")


@pytest.mark.parametrize("path", [1, 2])
def test_artifact_block_batched(pkg, layer_artifact, dev, path):
    lw, ow = layer_artifact
    x = pkg.synth.make_input(64, seed=790 + path, device=dev)
    st = pkg.block.moe_block(x, lw, pkg.load_geometry(), path=path)
    _compare(st, O.moe_block(x.cpu(), ow), f"artifact T=64 path={path}")


def test_artifact_block_prefill_sampled_rows(pkg, layer_artifact, dev):
    lw, ow = layer_artifact
    x = pkg.synth.make_input(2048, seed=795, device=dev, dtype=torch.bfloat16)
    st = pkg.block.moe_block(x, lw, pkg.load_geometry())
    rows = torch.randperm(2048, generator=torch.Generator().manual_seed(795))[:96]
    _compare(st, O.moe_block(x.cpu()[rows], ow), "artifact prefill", rows=rows)


def test_next_hint_over_artifact_layers_same_bits(pkg, layer_c0, layer_artifact, dev):
    """A layer chain that alternates a bf16-router layer and an artifact-width layer: the next-layer
    descriptor (moe_block_forward_w's `next`, moe_block_forward_prefetch's hint) never changes a
    bit, including when the next layer's router is f32 (that hint is skipped)."""
    lw0, _ = layer_c0
    lw1, _ = layer_artifact
    layers = [(lw0, _norm_weight(81, 2048, dev)), (lw1, _norm_weight(82, 2048, dev))]
    x = pkg.synth.make_input(1, seed=81, device=dev)
    a, b = x.clone(), x.clone()
    for step in range(3):
        for l, (lw, w) in enumerate(layers):
            nxt, nxt_w = layers[(l + 1) % 2]
            pkg.abi.block_forward(a, lw, out=a, residual=a, norm_w=w)
            pkg.abi.block_forward(b, lw, out=b, residual=b, norm_w=w, next_layer=nxt,
                                  next_norm_w=nxt_w)
        torch.cuda.synchronize()
        assert torch.equal(a, b), step
        assert torch.isfinite(a).all()
    assert pkg.abi.device_error_bits(dev) == 0


@pytest.mark.parametrize("fixture", ["layer_artifact", "layer_q5k"])
def test_artifact_decode_single_and_three_launch_agree(pkg, dev, request, fixture):
    """The single-launch layer with f32 router rows, an f32 scalar gate, split gate/up and Q5_K
    down, and the three-launch form of the same arithmetic: both match the oracle's routing bit for
    bit and its outputs within the block tolerance, token by token, and no bounded spin timed out."""
    lw, ow = request.getfixturevalue(fixture)
    xs = pkg.synth.make_input(6, seed=810, device=dev)
    ref = O.moe_block(xs.cpu(), ow)
    for path in (pkg._lib.MOE_PATH_GEMV, pkg._lib.MOE_PATH_GEMV_MULTI):
        outs, ids = [], []
        for i in range(6):
            st = pkg.abi.block_forward(xs[i:i + 1].contiguous(), lw, path=path, stages={"topk_ids"})
            outs.append(st["combined_out"])
            ids.append(st["topk_ids"])
        torch.cuda.synchronize()
        assert torch.equal(torch.cat(ids).cpu().long(), ref["topk_ids"]), (fixture, path)
        assert_close(torch.cat(outs), ref["combined_out"], f"{fixture} decode path {path}")
    assert pkg.abi.device_error_bits(dev) == 0
