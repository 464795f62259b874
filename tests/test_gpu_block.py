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


def test_c3_prefill_sampled_rows(pkg, layer_c3, dev):
    """T = 4096 bf16 activations on the MFMA path (config 3: seed 2 weights and input); the block
    is row-independent, so the oracle checks a seeded sample of 192 rows of the full-size run."""
    lw, ow = layer_c3
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


@pytest.mark.parametrize("T,bf16", [(7, False), (64, False), (200, True), (256, True)])
def test_small_t_folded_block_vs_stage_calls(pkg, layer_c3, dev, T, bf16):
    """Up to 256 tokens the block runs the shared expert inside the router and routed down
    launches, on the caller's stream alone. The separate stage calls (engine/block_forward.py:614-667: their
    own router, shared-expert and routed-expert launches) give the same routing, and shared and
    block outputs within the oracle tolerance; the oracle checks sampled rows of the block."""
    lw, ow = layer_c3
    cfg = pkg.load_geometry()
    x = pkg.synth.make_input(T, seed=33, device=dev, dtype=torch.bfloat16 if bf16 else torch.float32)
    r = pkg.block.moe_router(x, lw, cfg)
    s = pkg.block.moe_shared(x, lw, cfg)
    ro = pkg.block.moe_routed(x, lw, cfg, r)
    whole = pkg.block.moe_block(x, lw, cfg)
    torch.cuda.synchronize()
    assert torch.equal(r["topk_ids"], whole["topk_ids"])
    assert_close(whole["shared_out"].cpu(), s["shared_out"].cpu(), f"T={T} shared_out vs stage call")
    assert_close(whole["combined_out"].cpu(), (ro["routed_sum"] + s["shared_out"]).cpu(),
                 f"T={T} combined_out vs stage calls")
    rows = torch.randperm(T, generator=torch.Generator().manual_seed(T))[:min(T, 24)]
    ref = O.moe_block(x.cpu()[rows], ow)
    _compare(whole, ref, rows=rows, tag=f"folded T={T}")


@pytest.mark.parametrize("T", [24, 64, 136, 256])
def test_small_t_sort_in_router_launch(pkg, layer_zipf, dev, T):
    """From 17 to 256 tokens (Q4_K experts, bf16 shared expert; at 16 tokens and below the shared
    expert takes its GEMV form and the block its separate launches) the block sorts its (token, slot)
    pairs inside the router launch: the last 16-token group to finish routing counts its arrival
    in a sync word, resets it, and sorts. Two calls in a row give the same bits and report nothing
    in the status word. A count no launch produces, planted in that word from the host, makes the
    arrivals report MOE_STATUS_SYNC_STATE (the last arrival is taken modulo the number of groups,
    so the sort still runs once and the grouped GEMMs read a consistent tile list); after
    moe_workspace_init the call gives the first bits again. The word sits after the router's 256
    tile counters and 16 group counters."""
    import ctypes
    L, abi, synth = pkg._lib, pkg.abi, pkg.synth
    lw, _ = layer_zipf
    x = synth.make_input(T, seed=T, device=dev)
    outs = []
    for _ in range(2):
        o = torch.empty(T, 2048, dtype=torch.float32, device=dev)
        abi.block_forward(x, lw, out=o)
        torch.cuda.synchronize()
        assert abi.workspace_status(dev) == 0
        outs.append(o.cpu())
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    buf = abi.workspace(dev, 0)
    buf[:L.SYNC_BYTES].view(torch.int32)[L.ROUTER_CNT_WORD + 256 + 16] = 1000
    o = torch.empty(T, 2048, dtype=torch.float32, device=dev)
    abi.block_forward(x, lw, out=o)
    torch.cuda.synchronize()
    assert abi.workspace_status(dev) & L.STATUS_SYNC_STATE
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    assert L.lib.moe_workspace_init(ctypes.c_void_p(buf.data_ptr()), buf.numel(), stream) == L.MOE_OK
    abi.block_forward(x, lw, out=o)
    torch.cuda.synchronize()
    assert abi.workspace_status(dev) == 0
    assert torch.equal(o.cpu().view(torch.int32), outs[0].view(torch.int32))


def test_deterministic_repeat(pkg, layer_c0, dev):
    lw, _ = layer_c0
    x = pkg.synth.make_input(64, seed=4, device=dev)
    a = pkg.abi.block_forward(x, lw)["combined_out"].clone()
    b = pkg.abi.block_forward(x, lw)["combined_out"]
    assert torch.equal(a, b)


def test_decode_fused_residual_in_place(pkg, layer_c0, dev):
    """The fused single-token path with the residual add done in place (out aliases residual):
    out = x + MoE(x)."""
    lw, ow = layer_c0
    x = pkg.synth.make_input(1, seed=21, device=dev)
    ref = O.moe_block(x.cpu(), ow)
    buf = x.clone()
    pkg.abi.block_forward(buf, lw, out=buf, residual=buf)
    torch.cuda.synchronize()
    assert_close(buf.cpu() - x.cpu(), ref["combined_out"], "fused residual")


def test_decode_fused_q6k_down(pkg, layer_q6k, dev):
    lw, ow = layer_q6k
    for seed in (1, 2, 3):
        x = pkg.synth.make_input(1, seed=40 + seed, device=dev)
        st = pkg.block.moe_block(x, lw, pkg.load_geometry())
        _compare(st, O.moe_block(x.cpu(), ow), tag=f"fused q6k seed={seed}")


def test_decode_fused_many_tokens_sequential(pkg, layer_zipf, dev):
    """64 sequential single-token calls (Zipf-skewed routing) through the fused path: every one
    matches the oracle bit for bit on routing; exercises the device ticket reset between calls."""
    lw, ow = layer_zipf
    xs = pkg.synth.make_input(64, seed=77, device=dev)
    outs = [pkg.block.moe_block(xs[i:i + 1], lw, pkg.load_geometry()) for i in range(64)]
    ref = O.moe_block(xs.cpu(), ow)
    ids = torch.cat([o["topk_ids"] for o in outs]).cpu()
    assert torch.equal(ids, ref["topk_ids"])
    out = torch.cat([o["combined_out"] for o in outs]).cpu()
    assert_close(out, ref["combined_out"], "fused x64")


def test_decode_single_launch_and_three_launch_paths_agree(pkg, layer_c0, dev):
    """The persistent single-launch layer and the three-launch form of the same arithmetic both
    match the oracle on 32 tokens, and no bounded spin timed out."""
    lw, ow = layer_c0
    xs = pkg.synth.make_input(32, seed=5, device=dev)
    ref = O.moe_block(xs.cpu(), ow)
    for path in (pkg._lib.MOE_PATH_GEMV, pkg._lib.MOE_PATH_GEMV_MULTI):
        outs, ids = [], []
        for i in range(32):
            st = pkg.abi.block_forward(xs[i:i + 1].contiguous(), lw, path=path, stages={"topk_ids"})
            outs.append(st["combined_out"])
            ids.append(st["topk_ids"])
        torch.cuda.synchronize()
        assert torch.equal(torch.cat(ids).cpu().long(), ref["topk_ids"]), path
        assert_close(torch.cat(outs), ref["combined_out"], f"decode path {path}")
    assert pkg.abi.device_error_bits(dev) == 0


def test_decode_graph_replay_matches_eager(pkg, layer_c0, dev):
    """The single-launch layer inside a captured HIP graph, replayed several times with eager work
    between replays: every replay equals the eager result bit for bit (the epoch-tagged exchange
    words must advance correctly across replays)."""
    lw, _ = layer_c0
    x0 = pkg.synth.make_input(1, seed=99, device=dev)
    xin = x0.clone()
    out = torch.empty_like(x0)
    pkg.abi.block_forward(xin, lw, out=out)        # eager, also allocates the workspace
    torch.cuda.synchronize()
    want = out.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            pkg.abi.block_forward(xin, lw, out=out)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(5):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
        pkg.abi.block_forward(xin, lw, out=out)    # eager call between replays
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
    assert pkg.abi.device_error_bits(dev) == 0


def _tied_router(lw, ow, groups, dev):
    """Copies of the layer whose router gives tied logits: every expert of a group gets the first
    member's router row and the group's bias, so their logits (and probabilities) are equal."""
    import dataclasses
    router = lw.router.clone()
    bias = torch.zeros(lw.n_experts, dtype=torch.float32, device=dev)
    for members, b in groups:
        for e in members:
            router[e] = router[members[0]]
            bias[e] = b
    lw2 = dataclasses.replace(lw, router=router, router_bias=bias)
    ow2 = dataclasses.replace(ow, router=router.cpu(), router_bias=bias.cpu())
    return lw2, ow2


@pytest.mark.parametrize("case", ["inner", "boundary"])
def test_decode_single_launch_ties(pkg, layer_c0, dev, case):
    """Tied probabilities through the single-launch layer. 'inner': two equal experts inside the
    top 8 (the fast selection is exact up to slot order); 'boundary': the 8th and 9th are equal
    (which one torch keeps depends on its partition order, so the exact replay must run). With
    routing outputs requested the ids match torch's order exactly; without them the block output
    is the same bits (the combine runs in ascending expert id, independent of slot order)."""
    lw, ow = layer_c0
    if case == "inner":
        groups = [([10, 11], 8.0), ([20], 8.0), ([21], 8.0), ([22], 8.0), ([23], 8.0),
                  ([24], 8.0), ([25], 8.0)]
    else:
        groups = [([30], 12.0), ([31], 12.0), ([32], 12.0), ([33], 12.0), ([34], 12.0),
                  ([35], 12.0), ([36], 12.0), ([40, 41], 6.0)]
    lw2, ow2 = _tied_router(lw, ow, groups, dev)
    xs = pkg.synth.make_input(6, seed=17, device=dev)
    ref = O.moe_block(xs.cpu(), ow2)
    for i in range(xs.shape[0]):
        x = xs[i:i + 1].contiguous()
        st = pkg.abi.block_forward(x, lw2, stages={"topk_ids", "topk_weights"})
        plain = pkg.abi.block_forward(x, lw2)
        torch.cuda.synchronize()
        assert torch.equal(st["topk_ids"].cpu().long(), ref["topk_ids"][i:i + 1]), (case, i)
        assert_close(st["combined_out"].cpu(), ref["combined_out"][i:i + 1], f"{case} token {i}")
        assert torch.equal(plain["combined_out"], st["combined_out"]), (case, i)
    assert pkg.abi.device_error_bits(dev) == 0


def _norm_weight(seed, H, dev):
    g = torch.Generator().manual_seed(seed)
    return (1.0 + 0.1 * torch.randn(H, generator=g)).to(dev)


@pytest.mark.parametrize("path", ["single_launch", "three_launch"])
def test_decode_with_post_attention_norm(pkg, layer_c0, dev, path):
    """engine/m3_forward.py:732-737 in one call: x = x1 + MoE(rmsnorm_a(x1, w)) with the norm fused
    into the single-launch layer (or a norm kernel in front of the three-launch form). Routing
    bit-exact against the oracle, x_out within the block tolerance, residual updated in place."""
    lw, ow = layer_c0
    w = _norm_weight(31, 2048, dev)
    scales = torch.tensor([0.25, 1.0, 3.0, 17.0, 0.5, 8.0], device=dev).view(-1, 1)
    x1 = pkg.synth.make_input(6, seed=31, device=dev) * scales
    ref = O.residual_step(x1.cpu(), ow, w.cpu(), 1e-6)
    p = pkg._lib.MOE_PATH_GEMV if path == "single_launch" else pkg._lib.MOE_PATH_GEMV_MULTI
    for i in range(x1.shape[0]):
        h = x1[i:i + 1].clone()
        st = pkg.abi.block_forward(h, lw, path=p, stages={"topk_ids"}, out=h, residual=h, norm_w=w)
        torch.cuda.synchronize()
        assert torch.equal(st["topk_ids"].cpu().long(), ref["topk_ids"][i:i + 1]), (path, i)
        assert_close(h.cpu() - x1[i:i + 1].cpu(), ref["combined_out"][i:i + 1], f"{path} token {i}")
    assert pkg.abi.device_error_bits(dev) == 0


@pytest.mark.parametrize("path", [1, 2])
def test_batched_with_post_attention_norm(pkg, layer_zipf, dev, path):
    """The norm kernel in front of the multi-token paths (GEMV and MFMA), c2 shapes."""
    lw, ow = layer_zipf
    w = _norm_weight(32, 2048, dev)
    x1 = pkg.synth.make_input(64, seed=32, device=dev) * 4.0
    ref = O.residual_step(x1.cpu(), ow, w.cpu(), 1e-6)
    st = pkg.abi.block_forward(x1, lw, path=path, stages={"topk_ids"}, residual=x1, norm_w=w)
    assert torch.equal(st["topk_ids"].cpu().long(), ref["topk_ids"]), path
    assert_close(st["combined_out"].cpu() - x1.cpu(), ref["combined_out"], f"norm path {path}")


def test_decode_next_layer_hint_same_bits(pkg, layer_c0, layer_zipf, dev):
    """moe_block_forward_prefetch (the next layer's router rows and norm weight warmed into the
    L2 of the XCD that reads them first) gives the same bits as moe_block_forward, through a
    two-layer chain h <- h + MoE(rmsnorm(h)) run for several tokens."""
    lw0, _ = layer_c0
    lw1, _ = layer_zipf
    layers = [(lw0, _norm_weight(51, 2048, dev)), (lw1, _norm_weight(52, 2048, dev))]
    x = pkg.synth.make_input(1, seed=51, device=dev)
    a, b = x.clone(), x.clone()
    for step in range(6):
        for l, (lw, w) in enumerate(layers):
            nxt, nxt_w = layers[(l + 1) % 2]
            pkg.abi.block_forward(a, lw, out=a, residual=a, norm_w=w)
            pkg.abi.block_forward(b, lw, out=b, residual=b, norm_w=w, next_layer=nxt,
                                  next_norm_w=nxt_w if step % 2 else None)
        torch.cuda.synchronize()
        assert torch.equal(a, b), step
        assert torch.isfinite(a).all()
    assert pkg.abi.device_error_bits(dev) == 0


def test_decode_q5k_down(pkg, layer_q5k, dev):
    """Single tokens with Q5_K down (the three-launch decode path) match the oracle."""
    lw, ow = layer_q5k
    for seed in (1, 2, 3):
        x = pkg.synth.make_input(1, seed=60 + seed, device=dev)
        st = pkg.block.moe_block(x, lw, pkg.load_geometry())
        _compare(st, O.moe_block(x.cpu(), ow), tag=f"q5k decode seed={seed}")


def test_prefill_q5k_down_sampled_rows(pkg, layer_q5k, dev):
    """T = 2048 bf16 activations with Q5_K down on the MFMA path (160-row kernels)."""
    lw, ow = layer_q5k
    x = pkg.synth.make_input(2048, seed=5, device=dev, dtype=torch.bfloat16)
    st = pkg.block.moe_block(x, lw, pkg.load_geometry())
    rows = torch.randperm(2048, generator=torch.Generator().manual_seed(5))[:96]
    ref = O.moe_block(x.cpu()[rows], ow)
    _compare(st, ref, rows=rows, tag="q5k prefill")


def test_prefill_shared_stream_fork_same_bits_and_graph(pkg, layer_c0, dev):
    """From 7 tokens the shared expert runs on the library's second stream (forked from and joined
    back into the caller's stream by events). On the same (MFMA) kernels, the rows of a 7-token
    call equal those of a 6-token call, which runs every kernel on one stream, bit for bit; and the
    fork/join captured in a graph replays to the eager bits (7 and 256 tokens), with eager calls
    between the replays."""
    lw, _ = layer_c0
    mfma = pkg._lib.MOE_PATH_MFMA
    x7 = pkg.synth.make_input(7, seed=70, device=dev)
    a = pkg.abi.block_forward(x7, lw, path=mfma, stages={"topk_ids"})
    b = pkg.abi.block_forward(x7[:6].contiguous(), lw, path=mfma, stages={"topk_ids"})
    torch.cuda.synchronize()
    assert torch.equal(a["topk_ids"][:6], b["topk_ids"])
    assert torch.equal(a["combined_out"][:6], b["combined_out"])
    for T in (7, 256):
        _graph_replays_match(pkg, lw, pkg.synth.make_input(T, seed=71, device=dev, dtype=torch.bfloat16))


def _graph_replays_match(pkg, lw, x):
    want = pkg.abi.block_forward(x, lw)["combined_out"].clone()
    torch.cuda.synchronize()
    out = torch.empty_like(want)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            pkg.abi.block_forward(x, lw, out=out)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), rep
        other = pkg.abi.block_forward(x, lw)["combined_out"]
        torch.cuda.synchronize()
        assert torch.equal(other, want), rep


@pytest.mark.parametrize("T", [7, 300])
def test_block_output_independent_of_tie_slot_order(pkg, layer_c0, dev, T):
    """Router rows in equal pairs, so most tokens have equal probabilities inside their top 8.
    Without routing outputs the block forward keeps the fast top-k's slot order among them; asked
    for ids and per-slot expert rows it replays torch's order. The combine sums in ascending expert
    id with the same weights, so the block output is the same bits; the replayed ids are torch's."""
    import dataclasses
    from oracle import moe_oracle as O
    lw, _ = layer_c0
    g = torch.Generator().manual_seed(97 + T)
    half = (torch.randn(128, 2048, generator=g) * 0.02).to(torch.bfloat16)
    router = torch.cat([half, half])[torch.randperm(256, generator=g)].contiguous().to(dev)
    lt = dataclasses.replace(lw, router=router)
    x = pkg.synth.make_input(T, seed=97 + T, device=dev, dtype=torch.bfloat16)
    a = pkg.abi.block_forward(x, lt)
    b = pkg.abi.block_forward(x, lt, stages={"topk_ids", "expert_raw"})
    torch.cuda.synchronize()
    assert torch.equal(a["combined_out"], b["combined_out"])
    ref = O.route(x.cpu(), router.cpu(), 8, None)
    assert torch.equal(b["topk_ids"].cpu().long(), ref["topk_ids"])


@pytest.mark.parametrize("fmt", ["q5k", "q6k"])
def test_decode_single_launch_q5k_q6k_down(pkg, layer_q5k, layer_q6k, dev, fmt):
    """Q5_K and Q6_K down (the artifact's widths) in the single-launch decode layer, with the
    post-attention norm and residual fused: routing bit-exact vs the oracle on 16 tokens and the
    same results as the three-launch path within the block bars."""
    lw, ow = layer_q5k if fmt == "q5k" else layer_q6k
    L = pkg._lib
    w = pkg.synth.make_norm_weight(seed=61, device=dev)
    xs = pkg.synth.make_input(16, seed=60, device=dev)
    ref = O.residual_step(xs.cpu(), ow, w.cpu(), 1e-6)
    outs = {}
    for path in (L.MOE_PATH_GEMV, L.MOE_PATH_GEMV_MULTI):
        got, ids = [], []
        for i in range(16):
            x1 = xs[i:i + 1].contiguous()
            st = pkg.abi.block_forward(x1, lw, path=path, stages={"topk_ids"}, residual=x1, norm_w=w)
            got.append(st["combined_out"])
            ids.append(st["topk_ids"])
        torch.cuda.synchronize()
        assert torch.equal(torch.cat(ids).cpu().long(), ref["topk_ids"]), (fmt, path)
        outs[path] = torch.cat(got)
        assert_close(outs[path], ref["x_out"], f"{fmt} decode path {path}")
    assert pkg.abi.device_error_bits(dev) == 0
