"""Config 1 on the GPU: 40 resident layer instances (built as the benchmark builds them) and the
decoder's MoE half per layer, h <- h + MoE(rmsnorm(h)) with the norm and residual fused into the
single-launch decode layer and the next layer's weights named as the L2 warm-up hint
(engine/m3_forward.py:714-758). Teacher-forced: every layer is checked against the oracle's
residual_step on the device's own input to that layer. Then the chain is captured in a HIP graph,
replayed, and must give the eager chain's bits."""
import pytest
import torch

from oracle import moe_oracle as O
from tolerances import assert_close

pytestmark = pytest.mark.gpu

N_LAYERS = 40
EPS = 1e-6


class _DeviceExperts:
    """Expert records left on the device; the oracle copies only the experts it decodes."""

    def __init__(self, t: torch.Tensor):
        self.t = t
        self.shape = tuple(t.shape)

    def __getitem__(self, e):
        return self.t[e].cpu().numpy()


def _oracle_layer(lw) -> O.LayerWeights:
    return O.LayerWeights(
        router=lw.router.cpu(), gate_up_q=_DeviceExperts(lw.gate_up_q), gate_up_fmt=lw.gate_up_fmt,
        down_q=_DeviceExperts(lw.down_q), down_fmt=lw.down_fmt, shared_gate=lw.shared_gate.cpu(),
        shared_up=lw.shared_up.cpu(), shared_down=lw.shared_down.cpu(),
        shared_scalar_gate=lw.shared_scalar_gate.cpu(),
        router_bias=None if lw.router_bias is None else lw.router_bias.cpu())


@pytest.fixture(scope="module")
def chain(pkg, dev):
    synth = pkg.synth
    layers = [synth.make_layer(seed=1000 + l, device=dev) for l in range(N_LAYERS)]
    norms = [synth.make_norm_weight(seed=5000 + l, device=dev) for l in range(N_LAYERS)]
    torch.cuda.synchronize()
    yield layers, norms
    del layers
    torch.cuda.empty_cache()


def _layer_call(abi, x, layers, norms, l, stages=False):
    L = len(layers)
    out = torch.empty_like(x)
    st = abi.block_forward(x, layers[l], out=out, residual=x, norm_w=norms[l], norm_eps=EPS,
                           next_layer=layers[(l + 1) % L], next_norm_w=norms[(l + 1) % L],
                           stages=stages)
    return out, st


def test_c1_forty_layers_teacher_forced(pkg, dev, chain):
    """Three token streams through the 40 layers: routing bit-exact and x_out within the block
    bars at every layer; the unstaged call (as the benchmark makes it) gives the same bits."""
    layers, norms = chain
    abi = pkg.abi
    xs = [pkg.synth.make_input(1, seed=s, device=dev) for s in (0, 1, 2)]
    for l in range(N_LAYERS):
        ow = _oracle_layer(layers[l])
        nw = norms[l].cpu()
        for i in range(len(xs)):
            x_in = xs[i]
            out, st = _layer_call(abi, x_in, layers, norms, l, stages={"topk_ids", "router_logits"})
            plain, _ = _layer_call(abi, x_in, layers, norms, l)
            torch.cuda.synchronize()
            ref = O.residual_step(x_in.cpu(), ow, nw, EPS)
            tag = f"layer {l} stream {i}"
            assert torch.equal(st["router_logits"].cpu().view(torch.int16),
                               ref["router_logits"].view(torch.int16)), tag + " logits"
            assert torch.equal(st["topk_ids"].cpu().long(), ref["topk_ids"]), tag + " ids"
            assert_close(out, ref["x_out"], tag + " x_out")
            assert torch.equal(plain.cpu().view(torch.int32), out.cpu().view(torch.int32)), tag
            xs[i] = out
    assert abi.device_error_bits(dev) == 0


def test_c1_chain_graph_replay_matches_eager(pkg, dev, chain):
    """One token through the 40 layers, eager and as a replayed HIP graph (twice, with eager work
    in between): the same bits, and no spin timeout recorded."""
    layers, norms = chain
    abi = pkg.abi
    x0 = pkg.synth.make_input(1, seed=3, device=dev)
    x = x0.clone()
    for l in range(N_LAYERS):
        x, _ = _layer_call(abi, x, layers, norms, l)
    torch.cuda.synchronize()
    eager = x.cpu()
    buf = x0.clone()

    def chain_fn():
        for l in range(N_LAYERS):
            abi.block_forward(buf, layers[l], out=buf, residual=buf, norm_w=norms[l], norm_eps=EPS,
                              next_layer=layers[(l + 1) % N_LAYERS],
                              next_norm_w=norms[(l + 1) % N_LAYERS])

    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            chain_fn()
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    for rep in range(2):
        buf.copy_(x0)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(buf.cpu().view(torch.int32), eager.view(torch.int32)), f"replay {rep}"
        _ = _layer_call(abi, x0, layers, norms, 0)          # eager work between replays
        torch.cuda.synchronize()
    assert abi.device_error_bits(dev) == 0


def test_decode_layer_reports_a_forced_timeout(pkg, layer_c0, dev):
    """The status path without a real timeout: with the workspace's test hook set, every wait of
    the single-launch decode layer completes and then reports a timeout. moe_workspace_status
    must return the bit (stream-ordered) and clear it, and every output row must be NaN; with the
    hook cleared the same call gives the normal, finite result again."""
    lw, _ = layer_c0
    abi, L = pkg.abi, pkg._lib
    x = pkg.synth.make_input(1, seed=9, device=dev)
    good = abi.block_forward(x, lw)["combined_out"].clone()
    torch.cuda.synchronize()
    assert abi.workspace_status(dev) == 0
    abi.set_test_hook(dev, True)
    try:
        bad = abi.block_forward(x, lw, stages={"routed_sum", "shared_out"})
        torch.cuda.synchronize()
        assert torch.isnan(bad["combined_out"]).all()
        assert torch.isnan(bad["routed_sum"]).all() and torch.isnan(bad["shared_out"]).all()
        assert abi.workspace_status(dev) == L.STATUS_SPIN_TIMEOUT
        assert abi.workspace_status(dev) == 0                     # read clears it
    finally:
        abi.set_test_hook(dev, False)
    again = abi.block_forward(x, lw)["combined_out"]
    torch.cuda.synchronize()
    assert torch.equal(again.cpu().view(torch.int32), good.cpu().view(torch.int32))
    assert abi.workspace_status(dev) == 0
