"""Closed-form pins of the oracle's MoE block (CPU only, small synthetic geometry)."""
import importlib.util
from pathlib import Path

import numpy as np
import torch

from oracle import ggml_quant as GQ
from oracle import moe_oracle as O

ROOT = Path(__file__).resolve().parents[1]
_spec = importlib.util.spec_from_file_location("q_", ROOT / "qwen3.6-35b-a3b_amd" / "quant.py")
Q = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(Q)

E, H, I, K = 16, 256, 256, 8


def _layer(seed, gu=None, dn=None, zero_scalar_gate=False):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g) * 0.05
    gu = r(E, 2 * I, H) if gu is None else gu
    dn = r(E, H, I) if dn is None else dn
    return O.LayerWeights(
        router=r(E, H).to(torch.bfloat16),
        gate_up_q=Q.quantize(gu.reshape(-1, H), Q.FMT_Q4_K).numpy().reshape(E, 2 * I, -1),
        gate_up_fmt=Q.FMT_Q4_K,
        down_q=Q.quantize(dn.reshape(-1, I), Q.FMT_Q6_K).numpy().reshape(E, H, -1),
        down_fmt=Q.FMT_Q6_K,
        shared_gate=r(I, H).to(torch.bfloat16), shared_up=r(I, H).to(torch.bfloat16),
        shared_down=r(H, I).to(torch.bfloat16),
        shared_scalar_gate=torch.zeros(1, H, dtype=torch.bfloat16) if zero_scalar_gate
        else r(1, H).to(torch.bfloat16))


def test_identical_experts_make_routing_irrelevant():
    """With every expert equal, routed = expert(x) whatever the routing (weights sum to 1 up to
    the bf16 cast of each weight)."""
    g = torch.Generator().manual_seed(1)
    gu1 = torch.randn(1, 2 * I, H, generator=g) * 0.05
    dn1 = torch.randn(1, H, I, generator=g) * 0.05
    lw = _layer(2, gu=gu1.expand(E, -1, -1).contiguous(), dn=dn1.expand(E, -1, -1).contiguous())
    x = torch.randn(5, H, generator=g)
    out = O.moe_block(x, lw, K)
    gu, dn = lw.expert_f32(0)
    single = O.expert_apply(x, gu, dn)
    wsum = out["topk_weights"].float().sum(-1, keepdim=True)
    assert torch.allclose(out["routed_sum"], single * wsum, rtol=1e-4, atol=1e-6)


def test_zero_experts_and_zero_shared_give_zero():
    lw = _layer(3, gu=torch.zeros(E, 2 * I, H), dn=torch.zeros(E, H, I))
    lw.shared_down = torch.zeros(H, I, dtype=torch.bfloat16)
    x = torch.randn(4, H)
    out = O.moe_block(x, lw, K)
    assert torch.count_nonzero(out["combined_out"]) == 0


def test_scalar_gate_zero_is_one_half():
    lw = _layer(4, zero_scalar_gate=True)
    x = torch.randn(3, H)
    s = O.shared_expert(x, lw)
    assert torch.all(s["shared_gate_prob"] == 0.5)
    assert torch.equal(s["shared_out"], 0.5 * s["shared_raw"])


def test_gate_first_split_is_observable():
    """Swapping the gate and up halves changes the expert output (spec §11.4): the oracle's
    chunk(2) order is a tested fact, not a convention that could silently flip."""
    lw = _layer(5)
    x = torch.randn(2, H)
    gu, dn = lw.expert_f32(3)
    good = O.expert_apply(x, gu, dn)
    swapped = O.expert_apply(x, torch.cat([gu[I:], gu[:I]]), dn)
    assert (good - swapped).abs().max() > 1e-3


def test_expert_apply_matches_one_hot_closed_form():
    """x = e_j: gate = W_gate[:, j], up = W_up[:, j], so y = W_down @ (silu(W_g[:,j]) * W_u[:,j])."""
    lw = _layer(6)
    gu, dn = lw.expert_f32(2)
    j = 37
    x = torch.zeros(1, H)
    x[0, j] = 1.0
    y = O.expert_apply(x, gu, dn)[0]
    want = dn.double() @ (torch.nn.functional.silu(gu[:I, j].double()) * gu[I:, j].double())
    assert torch.allclose(y.double(), want, rtol=1e-5, atol=1e-7)


def test_all_experts_selected_when_k_equals_e():
    """E = K: every expert is selected and the weights are the full softmax, renormalised."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(4, H, generator=g)
    w = (torch.randn(8, H, generator=g) * 0.05).to(torch.bfloat16)
    r = O.route(x, w, 8)
    assert torch.equal(torch.sort(r["topk_ids"], -1).values, torch.arange(8).expand(4, 8))
    assert torch.allclose(r["topk_weights_f32"].sum(-1), torch.ones(4), atol=1e-6)


def test_combine_is_ascending_expert_order_with_rank_weights():
    """routed[t] = sum over ascending expert id of w[t, rank] * raw[t, rank]; a combine that used
    the expert id to index w would differ (weights are distinct by construction)."""
    lw = _layer(8)
    x = torch.randn(6, H)
    r = O.route(x, lw.router, K)
    e = O.experts_and_combine(x, r["topk_ids"], r["topk_weights"], lw)
    raw, w = e["expert_raw"], r["topk_weights"].float()
    want = (raw * w[..., None]).double().sum(1)
    assert torch.allclose(e["routed_sum"].double(), want, rtol=1e-5, atol=1e-7)
    w_by_id = torch.gather(w, 1, (r["topk_ids"] % K))
    wrong = (raw * w_by_id[..., None]).double().sum(1)
    assert (wrong - want).abs().max() > 1e-4


def _silu64(z: torch.Tensor) -> torch.Tensor:
    """silu(z) = z / (1 + e^-z) (moe_gather_kernels.h:514), evaluated in f64 from its definition."""
    return z / (1.0 + torch.exp(-z))


def test_shared_expert_matches_one_hot_closed_form():
    """x = e_j (speccheck/moe_ref.py:480-495): gate x = W_sg[:, j], up x = W_su[:, j], so
    shared_raw = W_sd @ (silu(W_sg[:, j]) * W_su[:, j]) and gate_prob = sigmoid(w_sg_scalar[j])."""
    lw = _layer(9)
    for j in (0, 37, H - 1):
        x = torch.zeros(1, H)
        x[0, j] = 1.0
        s = O.shared_expert(x, lw)
        g = lw.shared_gate.double()[:, j]
        u = lw.shared_up.double()[:, j]
        want = lw.shared_down.double() @ (_silu64(g) * u)
        assert torch.allclose(s["shared_raw"][0].double(), want, rtol=1e-5, atol=1e-7)
        p = 1.0 / (1.0 + torch.exp(-lw.shared_scalar_gate.double()[0, j]))
        assert abs(s["shared_gate_prob"].item() - p.item()) <= 2e-7
        # negative controls: silu on the up projection, or the gate and up rows exchanged
        wrong = lw.shared_down.double() @ (g * _silu64(u))
        assert (wrong - want).abs().max() > 1e-4
        assert (s["shared_raw"][0].double() - wrong).abs().max() > 1e-4


def test_shared_expert_two_hot_is_not_linear_in_x():
    """silu makes the expert nonlinear: x = e_i + e_j is not the sum of the one-hot outputs, and the
    closed form silu(g_i + g_j) * (u_i + u_j) is what the oracle computes."""
    lw = _layer(10)
    i, j = 5, 200
    x = torch.zeros(1, H)
    x[0, i] = 1.0
    x[0, j] = 1.0
    s = O.shared_expert(x, lw)["shared_raw"][0].double()
    g = lw.shared_gate.double()[:, i] + lw.shared_gate.double()[:, j]
    u = lw.shared_up.double()[:, i] + lw.shared_up.double()[:, j]
    want = lw.shared_down.double() @ (_silu64(g) * u)
    assert torch.allclose(s, want, rtol=1e-5, atol=1e-7)


def test_metrics_fields_and_refusals():
    """The comparator (speccheck/moe_ref.py:578-630): n_gt_1ulp counts against one bf16 step at
    the reference's max |value|, and mismatched dtypes, non-finite values and an all-zero
    reference are refused."""
    import pytest

    assert O.ulp_of(1.0) == 2.0 ** -7
    assert O.ulp_of(3.0) == 2.0 ** -6
    assert O.ulp_of(0.75) == 2.0 ** -8
    assert O.ulp_of(-2.0) == 2.0 ** -6
    assert O.ulp_of(0.0) == 0.0 and O.ulp_of(float("inf")) == 0.0
    ref = torch.tensor([1.0, -0.5, 0.25, 1.5])        # max |ref| = 1.5: one step = 2^-7
    got = ref + torch.tensor([0.0, 2.0 ** -8, 2.0 ** -6, 0.5])
    m = O.metrics(got, ref, name="t")
    assert m["ulp_of_refmax"] == 2.0 ** -7
    assert m["ndiff"] == 3 and m["n_gt_1ulp"] == 2 and m["n_gt_100ulp"] == 0
    assert m["max_abs"] == 0.5 and m["max_abs_over_scale"] == 0.5 / 1.5
    with pytest.raises(AssertionError, match="dtype"):
        O.metrics(got.double(), ref)
    with pytest.raises(AssertionError, match="shape"):
        O.metrics(got[:3], ref)
    with pytest.raises(AssertionError, match="non-finite"):
        O.metrics(torch.tensor([float("nan"), 0.0, 0.0, 1.0]), ref)
    with pytest.raises(AssertionError, match="all zero"):
        O.metrics(got, torch.zeros(4))


# ------------------------------------------------------------------------------------------------
# Pins for the reference's own must-catch injections (speccheck/selftest_moe.py:65-73, cases
# :93-107) and the combine's addend order (speccheck/moe_ref.py:464-475). Each test fixes a fact a
# plausible one-line slip in the oracle would break; the closed forms are evaluated from the
# definitions (one-hot columns, hand-built addends, an own bf16 RNE on bit patterns), not by
# calling the oracle's formula a second time.

def _bf16_rne_f32(v: torch.Tensor) -> torch.Tensor:
    """f32 -> bf16 round-to-nearest-even on the bit pattern (moe_router_kernels.h:189-205),
    returned as f32 values: (b + 0x7FFF + ((b >> 16) & 1)) >> 16, then << 16."""
    b = v.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    r = torch.where(r >= 2 ** 31, r - 2 ** 32, r)
    return r.to(torch.int32).view(torch.float32)


def test_gather_applies_each_slots_own_expert():
    """expert_raw[t, k] is expert ids[t, k] applied to x[t] (`wrong_expert_index`,
    speccheck/selftest_moe.py:66). With x[t] = e_j the closed form is
    W_down[e] @ (silu(W_gu[e][j-th column of the gate rows]) * (j-th column of the up rows)), which
    a gather that used a neighbouring expert's weights cannot meet (experts are distinct draws)."""
    lw = _layer(11)
    cols = [3, 77, 130, 255, 1, 200]
    x = torch.zeros(len(cols), H)
    for t, j in enumerate(cols):
        x[t, j] = 1.0
    out = O.moe_block(x, lw, K)
    ids = out["topk_ids"]
    assert ids.shape == (len(cols), K)
    closed = {}

    def closed_form(e, j):
        if (e, j) not in closed:
            gu, dn = lw.expert_f32(e)
            closed[e, j] = dn.double() @ (_silu64(gu[:I, j].double()) * gu[I:, j].double())
        return closed[e, j]

    for t, j in enumerate(cols):
        for k in range(K):
            e = int(ids[t, k])
            want = closed_form(e, j)
            got = out["expert_raw"][t, k].double()
            assert torch.allclose(got, want, rtol=1e-5, atol=1e-7), (t, k, e)
            # negative control: the neighbouring expert's closed form is far away
            assert (closed_form((e + 1) % E, j) - want).abs().max() > 1e-4


def test_r5_weights_are_cast_to_bf16_before_the_multiply():
    """R5 (`cast_after_multiply`, speccheck/selftest_moe.py:70; moe_ref.py:345-355): the routing
    weights handed to the combine are bf16_rne(vals / sum vals). With unit expert rows (slot k writes
    column k only) routed_sum[t, k] is exactly f32(w_bf16[t, k]); a combine fed the f32 weights
    would carry bits below bf16 precision."""
    lw = _layer(12)
    g = torch.Generator().manual_seed(12)
    T = 24
    x = torch.randn(T, H, generator=g)
    r = O.route(x, lw.router, K)
    assert r["topk_weights"].dtype == torch.bfloat16
    wpre = r["topk_weights_f32"]
    assert wpre.dtype == torch.float32
    # the pre-cast weights are not bf16 values, so the cast is observable
    assert ((wpre.view(torch.int32) & 0xFFFF) != 0).float().mean() > 0.9
    want = _bf16_rne_f32(wpre)
    assert torch.equal(r["topk_weights"].float(), want)
    raw = torch.zeros(T, K, H)
    for k in range(K):
        raw[:, k, k] = 1.0
    e = O.routed_combine(raw, r["topk_ids"], r["topk_weights"])
    assert torch.equal(e[:, :K], want)
    assert torch.count_nonzero(e[:, K:]) == 0
    # and through the block's own gather/combine
    blk = O.experts_and_combine(x[:2], r["topk_ids"][:2], r["topk_weights"][:2], lw)
    assert blk["routed_sum"].dtype == torch.float32


def test_combine_adds_in_ascending_expert_id():
    """The combine's addends go in ascending expert id with the weight reached by rank
    (speccheck/moe_ref.py:464-475). Addends 2^24, 1, -2^24 make the order visible in f32:
    ascending id gives (2^24 + 1) - 2^24 = 2^24 - 2^24 = 0 (2^24 + 1 rounds to even), rank order
    gives (-2^24 + 2^24) + 1 = 1."""
    ids = torch.tensor([[7, 1, 3, 0, 2, 4, 5, 6],      # rank 0 holds expert 7, rank 1 expert 1 ...
                        [2, 6, 0, 1, 3, 4, 5, 7]])
    w = torch.ones(2, K, dtype=torch.bfloat16)
    raw = torch.zeros(2, K, 4)
    big = float(2 ** 24)
    # token 0, column 0: rank 0 (expert 7) -big, rank 1 (expert 1) +big, rank 2 (expert 3) +1
    raw[0, 0, 0], raw[0, 1, 0], raw[0, 2, 0] = -big, big, 1.0
    # token 1, column 1: expert 0 (rank 2) +big, expert 2 (rank 0) +1, expert 6 (rank 1) -big
    raw[1, 2, 1], raw[1, 0, 1], raw[1, 1, 1] = big, 1.0, -big
    # column 2: weights by rank, not by id: distinct power-of-two weights, one unit addend each
    wd = torch.tensor([[2.0 ** -k for k in range(K)]] * 2).to(torch.bfloat16)
    raw[:, :, 2] = 1.0
    out = O.routed_combine(raw, ids, w)
    assert out[0, 0].item() == 0.0
    assert out[1, 1].item() == 0.0           # ids 0 (+big), 2 (+1 -> rounds away), 6 (-big)
    rank_order = (torch.tensor(-big) + torch.tensor(big)) + torch.tensor(1.0)
    assert rank_order.item() == 1.0          # the order the test excludes
    outw = O.routed_combine(raw, ids, wd)
    assert torch.equal(outw[:, 2], wd.float().sum(-1))
    # token 0 with column 3 = rank index: the sum is the same in every order, so weights by rank
    raw[:, :, 3] = torch.arange(K, dtype=torch.float32)
    outw = O.routed_combine(raw, ids, wd)
    want = sum(float(wd[0, k]) * k for k in range(K))
    assert outw[0, 3].item() == want


def test_from_device_stacks_gate_before_up_for_split_records():
    """Separate `ffn_gate_exps` / `ffn_up_exps` records become the fused record's row order: gate
    rows 0..I-1, up rows I..2I-1 (spec §11.4: chunk(2) on the output axis, gate first)."""
    from types import SimpleNamespace
    e_, h_, i_ = 2, 256, 3
    rb = Q.row_bytes(Q.FMT_Q4_K, h_)
    gate = torch.full((e_, i_, rb), 11, dtype=torch.uint8)
    up = torch.full((e_, i_, rb), 22, dtype=torch.uint8)
    bf = lambda *s: torch.zeros(*s, dtype=torch.bfloat16)
    dev = SimpleNamespace(router=bf(e_, h_), gate_up_q=gate, up_q=up, gate_up_fmt=Q.FMT_Q4_K,
                          down_q=torch.zeros(e_, h_, Q.row_bytes(Q.FMT_Q4_K, 256), dtype=torch.uint8),
                          down_fmt=Q.FMT_Q4_K, shared_gate=bf(4, h_), shared_up=bf(4, h_),
                          shared_down=bf(h_, 4), shared_scalar_gate=bf(1, h_), router_bias=None)
    lw = O.from_device(dev)
    assert lw.gate_up_q.shape == (e_, 2 * i_, rb)
    assert (lw.gate_up_q[:, :i_] == 11).all() and (lw.gate_up_q[:, i_:] == 22).all()
