"""Routed experts (GEMV and MFMA paths) and the shared expert vs the f32 oracle."""
import pytest
import torch

from oracle import moe_oracle as O
from tolerances import assert_close

pytestmark = pytest.mark.gpu


def _route_and_group(pkg, lw, x):
    r = pkg.abi.router_topk(x, lw.router, 8, lw.router_bias)
    gr = pkg.abi.sort_permute(r["topk_ids"], lw.n_experts)
    return r, gr


def _oracle_raw(ow, x_cpu, ids_cpu):
    e = O.experts_and_combine(x_cpu, ids_cpu.long(), torch.ones(ids_cpu.shape, dtype=torch.bfloat16), ow)
    return e["expert_raw"]


# MOE_PATH_MFMA_BF16 (3) rounds weights and s to 8 significant bits: its documented bound is 8e-3
BOUND = {1: 2e-3, 2: 2e-3, 3: 8e-3}


@pytest.mark.parametrize("T,path", [(1, 1), (4, 1), (16, 1), (1, 2), (64, 2), (200, 2), (64, 3)])
def test_routed_experts_vs_oracle(pkg, layer_c0, dev, T, path):
    lw, ow = layer_c0
    x = pkg.synth.make_input(T, seed=100 + T, device=dev)
    r, gr = _route_and_group(pkg, lw, x)
    y = pkg.abi.experts(x, lw.gate_up_q, lw.gate_up_fmt, lw.down_q, lw.down_fmt, gr, 8, path)
    torch.cuda.synchronize()
    pos = gr["pair_pos"].cpu().long()
    raw = y.cpu()[pos].view(T, 8, -1)
    want = _oracle_raw(ow, x.cpu(), r["topk_ids"].cpu())
    assert_close(raw, want, f"expert_raw T={T} path={path}", max_abs=BOUND[path])


def test_small_and_large_tile_kernels_same_bits(pkg, layer_zipf, dev):
    """Q4_K experts at up to 256 tokens run on 32-row tiles (one block per tile and slab), above
    on the 160-row persistent kernels. Both take the same K steps in the same order, so a
    (token, slot) row comes out with the same bits whichever tile it sits in: the rows of a
    256-token call equal those of the same tokens inside a 257-token call (Zipf routing: a few
    experts with many rows, many with one)."""
    lw, _ = layer_zipf
    x = pkg.synth.make_input(257, seed=257, device=dev)
    rows = []
    for T in (256, 257):
        r, gr = _route_and_group(pkg, lw, x[:T].contiguous())
        y = pkg.abi.experts(x[:T].contiguous(), lw.gate_up_q, lw.gate_up_fmt, lw.down_q, lw.down_fmt, gr, 8, 2)
        torch.cuda.synchronize()
        rows.append(y.cpu()[gr["pair_pos"].cpu().long()][: 256 * 8])
    assert torch.isfinite(rows[0]).all()
    assert torch.equal(rows[0], rows[1])


def test_routed_experts_q6k_down(pkg, layer_q6k, dev):
    """GEMV (path 1) and the 160-row MFMA kernels (path 2: Q6_K down decoded in the MFMA waves
    from raw super-block bytes in LDS); at 600 Zipf-routed tokens the hot experts span several
    tiles and end on a partial one."""
    lw, ow = layer_q6k
    for T, path in ((2, 1), (96, 2), (600, 2)):
        x = pkg.synth.make_input(T, seed=7 + T, device=dev)
        r, gr = _route_and_group(pkg, lw, x)
        y = pkg.abi.experts(x, lw.gate_up_q, lw.gate_up_fmt, lw.down_q, lw.down_fmt, gr, 8, path)
        torch.cuda.synchronize()
        raw = y.cpu()[gr["pair_pos"].cpu().long()].view(T, 8, -1)
        want = _oracle_raw(ow, x.cpu(), r["topk_ids"].cpu())
        assert_close(raw, want, f"expert_raw q6k T={T} path={path}", max_abs=BOUND[path])


def test_routed_experts_q5k_down(pkg, layer_q5k, dev):
    lw, ow = layer_q5k
    for T, path in ((1, 1), (9, 1), (160, 2)):
        x = pkg.synth.make_input(T, seed=30 + T, device=dev)
        r, gr = _route_and_group(pkg, lw, x)
        y = pkg.abi.experts(x, lw.gate_up_q, lw.gate_up_fmt, lw.down_q, lw.down_fmt, gr, 8, path)
        torch.cuda.synchronize()
        raw = y.cpu()[gr["pair_pos"].cpu().long()].view(T, 8, -1)
        want = _oracle_raw(ow, x.cpu(), r["topk_ids"].cpu())
        assert_close(raw, want, f"expert_raw q5k T={T} path={path}", max_abs=BOUND[path])


# path 2 up to 256 tokens runs the narrow-slab kernels (one or two 32-row groups in the last
# 64-row tile: 7, 33, 100), above it the 128 x 256 items (257)
@pytest.mark.parametrize("T,path,dtype", [(1, 1, torch.float32), (16, 1, torch.float32),
                                          (7, 2, torch.float32), (33, 2, torch.bfloat16),
                                          (64, 2, torch.float32), (100, 2, torch.float32),
                                          (256, 2, torch.bfloat16), (257, 2, torch.bfloat16),
                                          (64, 3, torch.bfloat16)])
def test_shared_expert_vs_oracle(pkg, layer_c0, dev, T, path, dtype):
    lw, ow = layer_c0
    x = pkg.synth.make_input(T, seed=200 + T, device=dev, dtype=dtype)
    raw, prob = pkg.abi.shared_expert(x, lw.shared_gate, lw.shared_up, lw.shared_down,
                                      lw.shared_scalar_gate, path)
    torch.cuda.synchronize()
    s = O.shared_expert(x.cpu(), ow)
    assert_close(raw, s["shared_raw"], f"shared_raw T={T} path={path}", max_abs=BOUND[path])
    assert torch.allclose(prob.cpu(), s["shared_gate_prob"].view(-1), rtol=1e-5, atol=1e-6)
