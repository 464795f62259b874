"""R1 logits bit-exact vs the correctly rounded oracle; R3 ids bit-exact vs torch's CPU topk,
including tie-laden rows and the heap-select branch; R4/R5 weights within f32 rounding."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from oracle import topk_model as TM

pytestmark = pytest.mark.gpu


def _check_route(pkg, x, w_router, bias, K=8):
    r = pkg.abi.router_topk(x, w_router, K, bias, want_probs=True)
    torch.cuda.synchronize()
    ref_logits, _ = O.r1_logits(x.cpu(), w_router.cpu(), None if bias is None else bias.cpu())
    got_logits = r["router_logits"].cpu()
    assert torch.equal(got_logits.view(torch.int16), ref_logits.view(torch.int16)), \
        f"{(got_logits != ref_logits).sum().item()} logits differ"
    # R2/R3 on the (identical) logits: torch CPU softmax + topk are the reference
    probs = torch.softmax(ref_logits.float(), dim=-1)
    vals, ids = torch.topk(probs, K, dim=-1)
    got_ids = r["topk_ids"].cpu().long()
    bad = (got_ids != ids).any(dim=-1)
    assert not bad.any(), f"ids differ on {bad.sum().item()} of {len(bad)} rows; first {bad.nonzero()[:5].flatten().tolist()}"
    # probabilities: same function, different exp implementation -> a few f32 ulps
    assert torch.allclose(r["router_probs"].cpu(), probs, rtol=2e-6, atol=1e-9)
    wpre = vals / vals.sum(-1, keepdim=True)
    assert torch.allclose(r["topk_weights_f32"].cpu(), wpre, rtol=4e-6, atol=0)
    # R5: bf16 of wpre; equal unless the f32 value sits within a few ulps of a rounding boundary
    wb = r["topk_weights"].cpu()
    diff = (wb.float() != wpre.to(torch.bfloat16).float())
    if diff.any():
        b = wpre[diff].view(torch.int32) & 0xFFFF
        assert ((b - 0x8000).abs() < 64).all(), "bf16 weight differs away from a rounding boundary"
    return r, got_ids


def test_router_decode_c0(pkg, layer_c0, dev):
    lw, _ = layer_c0
    x = pkg.synth.make_input(1, seed=0, device=dev)
    _check_route(pkg, x, lw.router, None)


# 8..256 tokens: R1-R5 in one launch (K split over blocks, last arrivals reduce and route)
@pytest.mark.parametrize("T,dtype", [(8, torch.float32), (9, torch.float32), (64, torch.float32),
                                     (200, torch.bfloat16), (256, torch.float32),
                                     (300, torch.bfloat16), (4096, torch.bfloat16)])
def test_router_batched(pkg, layer_c0, dev, T, dtype):
    lw, _ = layer_c0
    x = pkg.synth.make_input(T, seed=T, device=dev, dtype=dtype)
    _check_route(pkg, x, lw.router, None)


def test_router_zipf_bias(pkg, layer_zipf, dev):
    lw, _ = layer_zipf
    x = pkg.synth.make_input(64, seed=1, device=dev)
    _check_route(pkg, x, lw.router, lw.router_bias)


@pytest.mark.parametrize("T", [1, 64, 700])
def test_router_tie_laden_rows(pkg, dev, T):
    """Router rows drawn from 3 distinct rows: logits repeat exactly, so nearly every row has
    ties inside the top 8 and across the 8/9 boundary; ids must follow torch's tie order."""
    g = torch.Generator().manual_seed(11 + T)
    base = (torch.randn(3, 2048, generator=g) * 0.02).to(torch.bfloat16)
    assign = torch.randint(0, 3, (256,), generator=g)
    w = base[assign].contiguous().to(dev)
    x = torch.randn(T, 2048, generator=g).to(dev)
    _check_route(pkg, x, w, None)


@pytest.mark.parametrize("T", [2, 40])
def test_router_midpoint_logits_round_to_even(pkg, dev, T):
    """Logits that are exact bf16 midpoints (1 + 2^-8 -> 1.0, ties to even) and just above one
    (-> 1 + 2^-7): the certified path must fall back and decide exactly. T = 2 runs the
    small-T kernel, T = 40 the MFMA tile kernel (rows alternate the two patterns)."""
    H = 2048
    x = torch.zeros(T, H)
    x[0::2, 0], x[0::2, 1] = 1.0, 2.0 ** -8
    x[1::2, 0], x[1::2, 1], x[1::2, 2] = 1.0, 2.0 ** -8, 2.0 ** -40
    w = torch.zeros(256, H)
    w[:, 0:3] = 1.0
    r = pkg.abi.router_topk(x.to(dev), w.to(torch.bfloat16).to(dev), 8)
    lg = r["router_logits"].cpu().float()
    assert (lg[0::2] == 1.0).all()
    assert (lg[1::2] == 1.0 + 2.0 ** -7).all()


@pytest.mark.parametrize("T,E,dtype", [(45, 200, torch.float32), (33, 24, torch.bfloat16)])
def test_router_ragged_tiles(pkg, dev, T, E, dtype):
    """T and E that leave partial 32-token / 128-expert / 16-expert tiles, with a bias."""
    g = torch.Generator().manual_seed(T * 1000 + E)
    w = (torch.randn(E, 2048, generator=g) * 0.02).to(torch.bfloat16)
    bias = torch.randn(E, generator=g) * 0.1
    x = torch.randn(T, 2048, generator=g).to(dtype)
    _check_route(pkg, x.to(dev), w.to(dev), bias.to(dev))


def test_router_heap_select_branch(pkg, dev):
    """An adversarial row drives libstdc++'s introselect into heap-select; inject it as logits
    through the bias with a zero router matrix."""
    vals = TM.adversarial_row(256, 8, start=-40.0)
    ids_model, heap = TM.torch_cpu_topk(vals, 8)
    assert heap
    bias = torch.tensor(vals, dtype=torch.float32)
    x = torch.randn(1, 2048)
    w = torch.zeros(256, 2048, dtype=torch.bfloat16)
    r, got = _check_route(pkg, x.to(dev), w.to(dev), bias.to(dev))
    assert got[0].tolist() == ids_model


def _router_f64_path(pkg, x, w, bias, K=8):
    """moe_router_topk with the logits given and no workspace: R1 stays on the f64 matrix cores."""
    L = pkg._lib
    T, H = x.shape
    E = w.shape[0]
    dev = x.device
    lg = torch.empty(T, E, dtype=torch.bfloat16, device=dev)
    ids = torch.empty(T, K, dtype=torch.int32, device=dev)
    wf = torch.empty(T, K, dtype=torch.float32, device=dev)
    wb = torch.empty(T, K, dtype=torch.bfloat16, device=dev)
    xdt = L.MOE_DT_F32 if x.dtype == torch.float32 else L.MOE_DT_BF16
    wdt = L.MOE_DT_F32 if w.dtype == torch.float32 else L.MOE_DT_BF16
    p = lambda t: None if t is None else t.data_ptr()
    rc = L.lib.moe_router_topk(p(x), xdt, p(w), wdt, p(bias), T, H, E, K, p(lg), None, p(ids),
                               p(wf), p(wb), None, 0, torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0
    return lg, ids


@pytest.mark.parametrize("xdt,wdt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.bfloat16), (torch.float32, torch.float32)])
def test_router_int8_and_f64_matrix_cores_same_bits(pkg, dev, xdt, wdt):
    """R1 at T = 4096 on the int8 matrix cores (digit-split, certified) and on the f64 ones: the
    same logits and ids bit for bit, for every x / router width, with a bias."""
    g = torch.Generator().manual_seed(4242)
    x = torch.randn(4096, 2048, generator=g).to(xdt).to(dev)
    w = (torch.randn(256, 2048, generator=g) * 0.02).to(wdt).to(dev)
    bias = (torch.randn(256, generator=g) * 0.1).to(dev)
    r = pkg.abi.router_topk(x, w, 8, bias)
    lg, ids = _router_f64_path(pkg, x, w, bias)
    torch.cuda.synchronize()
    assert torch.equal(r["router_logits"].view(torch.int16), lg.view(torch.int16)), \
        f"{(r['router_logits'] != lg).sum().item()} logits differ"
    assert torch.equal(r["topk_ids"], ids)


@pytest.mark.parametrize("xdt,wdt", [(torch.bfloat16, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.bfloat16), (torch.float32, torch.float32)])
def test_router_single_launch_and_per_tile_kernels_same_bits(pkg, dev, xdt, wdt):
    """T = 100 (a partial 16-token group): R1-R5 in one launch (K split over four blocks per tile,
    the partials and the routing done by the last arrivals) against the one-block-per-tile R1 and
    the separate top-k launch: the same logits, ids and weights bit for bit, twice in a row (the
    arrival counters are back at zero after each launch)."""
    g = torch.Generator().manual_seed(100)
    x = torch.randn(100, 2048, generator=g).to(xdt).to(dev)
    w = (torch.randn(256, 2048, generator=g) * 0.02).to(wdt).to(dev)
    bias = (torch.randn(256, generator=g) * 0.1).to(dev)
    lg, ids = _router_f64_path(pkg, x, w, bias)
    for _ in range(2):
        r = pkg.abi.router_topk(x, w, 8, bias)
        torch.cuda.synchronize()
        assert torch.equal(r["router_logits"].view(torch.int16), lg.view(torch.int16))
        assert torch.equal(r["topk_ids"], ids)


@pytest.mark.parametrize("T,E,xdt,wdt", [(333, 200, torch.bfloat16, torch.float32),
                                         (257, 24, torch.float32, torch.bfloat16),
                                         (700, 256, torch.bfloat16, torch.bfloat16),
                                         (333, 200, torch.bfloat16, torch.bfloat16),
                                         (1100, 24, torch.bfloat16, torch.bfloat16)])
def test_router_int8_ragged_and_wide_range(pkg, dev, T, E, xdt, wdt):
    """The int8 R1 on partial 64-token / 64-expert tiles, with rows whose elements span 2^-40 ..
    2^3 (so some fall below the digit grid and the certificate, or the double-double recompute,
    must carry them), against the correctly rounded oracle."""
    g = torch.Generator().manual_seed(T + 7 * E)
    x = torch.randn(T, 2048, generator=g) * torch.exp2(-40 * torch.rand(T, 2048, generator=g))
    w = torch.randn(E, 2048, generator=g) * 0.02 * torch.exp2(-30 * torch.rand(E, 2048, generator=g))
    x[::5, ::3] *= 8.0
    bias = torch.randn(E, generator=g) * 0.1
    x, w = x.to(xdt), w.to(wdt)
    _check_route(pkg, x.to(dev), w.to(dev), bias.to(dev))


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_router_int8_midpoints_round_to_even(pkg, dev, xdt):
    """Exact bf16 midpoints and values 2^-40 above them at T = 300 (the int8 R1): the digit sums
    land on the midpoint, the certificate refuses, and the wave's double-double recompute decides
    (ties to even; the 2^-40 element, below the x digit grid, rounds up)."""
    T, H = 300, 2048
    x = torch.zeros(T, H)
    x[0::2, 0], x[0::2, 1] = 1.0, 2.0 ** -8
    x[1::2, 0], x[1::2, 1], x[1::2, 2] = 1.0, 2.0 ** -8, 2.0 ** -40
    w = torch.zeros(256, H)
    w[:, 0:3] = 1.0
    r = pkg.abi.router_topk(x.to(xdt).to(dev), w.to(torch.bfloat16).to(dev), 8)
    lg = r["router_logits"].cpu().float()
    assert (lg[0::2] == 1.0).all()
    assert (lg[1::2] == 1.0 + 2.0 ** -7).all()


@pytest.mark.parametrize("T", [1, 64, 256, 2048])
def test_router_r2_near_equal_probabilities(pkg, dev, T):
    """R2 fixture (tests/r2_fixture.py): rows whose distinct near-zero logits give probabilities
    within a few f32 ulps. x[t] = e_t and router column t = row t's logits, so R1 returns them
    exactly. The ids must equal the box host's torch.topk(torch.softmax) on every row outside the
    fragile class (distinct logits within 2 ulps in the top 9). Inside it they depend on the last
    bit of each exp and of the reciprocal of the sum: the device's exps are correctly rounded and
    torch's CPU softmax exps are within one ulp of that, so the ids may differ on a small share of
    these rows (measured: 1 of 2,360 fragile rows; hipcc's expf instead gave 546). The bound below
    is 2 % of the fragile rows; the count is printed."""
    import r2_fixture as F
    rows = F.logit_rows(T, seed=100 + T)
    H = 2048
    w = torch.zeros(256, H, dtype=torch.bfloat16)
    w[:, :T] = rows.t()
    x = torch.zeros(T, H)
    x[torch.arange(T), torch.arange(T)] = 1.0
    r = pkg.abi.router_topk(x.to(dev), w.to(dev), 8)
    torch.cuda.synchronize()
    assert torch.equal(r["router_logits"].cpu().view(torch.int16), rows.view(torch.int16))
    _, ids = torch.topk(torch.softmax(rows.float(), dim=-1), 8, dim=-1)
    differ = (r["topk_ids"].cpu().long() != ids).any(-1)
    frag = F.fragile_rows(rows)
    print(f"\nR2 fixture T={T}: fragile rows {int(frag.sum())}, ids differ on "
          f"{int((differ & frag).sum())} of them; robust rows {int((~frag).sum())}, "
          f"differ {int((differ & ~frag).sum())}", flush=True)
    assert not (differ & ~frag).any()
    assert int((differ & frag).sum()) <= max(1, int(0.02 * int(frag.sum())))


def test_router_chain_reports_a_count_it_cannot_produce(pkg, dev):
    """The single-launch router (8-256 tokens) counts block arrivals in the workspace's sync words
    and each last arriver resets its counter. A counter left at a value no launch produces (set
    here from the host, as after a workspace that skipped moe_workspace_init) makes the arrivals
    set MOE_STATUS_SYNC_STATE in the status word; the launch has no waits, so it still ends. After
    moe_workspace_init the same call gives the first call's bits again and reports nothing."""
    import ctypes
    L, abi, synth = pkg._lib, pkg.abi, pkg.synth
    lw = synth.make_layer(seed=1, device=dev, zipf=True)
    x = synth.make_input(64, seed=1, device=dev)
    good = abi.router_topk(x, lw.router, 8, lw.router_bias)
    torch.cuda.synchronize()
    assert abi.workspace_status(dev) == 0
    buf = abi.workspace(dev, 0)
    buf[:L.SYNC_BYTES].view(torch.int32)[L.ROUTER_CNT_WORD + 3] = 1000
    abi.router_topk(x, lw.router, 8, lw.router_bias)
    assert abi.workspace_status(dev) & L.STATUS_SYNC_STATE
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    assert L.lib.moe_workspace_init(ctypes.c_void_p(buf.data_ptr()), buf.numel(), stream) == L.MOE_OK
    again = abi.router_topk(x, lw.router, 8, lw.router_bias)
    torch.cuda.synchronize()
    assert abi.workspace_status(dev) == 0
    for k in ("router_logits", "topk_ids", "topk_weights", "topk_weights_f32"):
        assert torch.equal(again[k].cpu(), good[k].cpu()), k
