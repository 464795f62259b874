"""Benchmark of the gfx950 MoE block on BASELINE.json's configs (one MI355X).

Headline (`value`): Q4_K MoE-layer decode at bs=1, config 1 — 40 independent resident layer
instances (~18.1 GB of Q4_K experts, so every expert byte comes from HBM), one token at a time
through all 40 layers, the next layer's input being the previous layer's residual stream
(x <- x + MoE(x), the decoder layer's own residual add), 1024 sequential tokens by default.
A step is one token through the 40 layers; it is captured once as a HIP graph and replayed.
Reported as us per token per layer, with the HBM rate over the 8 routed + 1 shared active
experts' bytes (20,447,232 B per token-layer).

Also on the line: prefill tokens/s at T = 4096 (config 3) with MFMA utilisation against the bf16
dense peak, the roofline of the dominant decode kernel, and the CPU baseline (this repo's CPU
oracle of the same block, timed on the host on a bounded sample).

Usage: python bench.py [--gpus 1] [--steps 1024] [--warmup 16] [--layers 40] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    return ap.parse_args()


def time_stream(fn, n: int, torch) -> float:
    """Average ms of fn() over n calls, HIP events on the current stream."""
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(n):
        fn()
    b.record(st)
    b.synchronize()
    return a.elapsed_time(b) / n


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (multi-GPU "
                          "sharding is design-only, see DESIGN.md)"}))
        sys.exit(2)
    import torch
    import __graft_entry__ as ge

    pkg = ge.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    synth, abi = pkg.synth, pkg.abi
    L = args.layers

    # ---------------------------------------------------------------- decode, config 1
    t0 = time.time()
    layers = [synth.make_layer(seed=1000 + l, device=dev) for l in range(L)]
    torch.cuda.synchronize()
    resident = sum(lw.gate_up_q.numel() + lw.down_q.numel() for lw in layers)
    log(f"generated {L} layers ({resident / 1e9:.2f} GB routed Q4_K) in {time.time() - t0:.1f}s")
    x0 = synth.make_input(1, seed=0, device=dev)
    xbuf = x0.clone()

    def one_token():
        # the residual stream through 40 layers, updated in place by the block's own residual add
        for lw in layers:
            abi.block_forward(xbuf, lw, out=xbuf, residual=xbuf)
        xbuf.copy_(synth.rms_normalize(xbuf))

    for _ in range(3):
        one_token()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            one_token()
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    ms = time_stream(g.replay, args.steps, torch)
    us_tok_layer = ms * 1000.0 / L
    active = synth.decode_active_bytes(layers[0])
    gbps = active / (us_tok_layer * 1e-6) / 1e9
    log(f"decode: {ms:.3f} ms/token over {L} layers = {us_tok_layer:.2f} us/token/layer, "
        f"{gbps:.0f} GB/s on {active} active B/token-layer")

    # dominant kernel: the routed-expert contraction of one decode token (GEMV path), alone
    lw = layers[0]
    r = abi.router_topk(x0, lw.router, 8)
    gr = abi.sort_permute(r["topk_ids"], lw.n_experts)
    routed_bytes = 8 * lw.routed_bytes_per_expert()
    y = torch.empty(8, 2048, dtype=torch.float32, device=dev)

    def experts_call():
        abi.experts(x0, lw.gate_up_q, lw.gate_up_fmt, lw.down_q, lw.down_fmt, gr, 8, path=1)

    for _ in range(20):
        experts_call()
    # rotate over layers so the bytes come from HBM, not the 256 MB MALL
    lws = layers

    def experts_rot():
        for lw2 in lws:
            abi.experts(x0, lw2.gate_up_q, lw2.gate_up_fmt, lw2.down_q, lw2.down_fmt, gr, 8, path=1)

    ms_exp = time_stream(experts_rot, 20, torch) / len(lws)
    exp_gbps = routed_bytes / (ms_exp * 1e-3) / 1e9
    log(f"routed experts (gate_up + down GEMV, 8 experts): {ms_exp * 1000:.2f} us, {exp_gbps:.0f} GB/s")
    del y

    # ---------------------------------------------------------------- prefill, config 3
    prefill = {}
    if not args.no_prefill:
        lwp = layers[0]
        xp = synth.make_input(4096, seed=2, device=dev, dtype=torch.bfloat16)
        outp = torch.empty(4096, 2048, dtype=torch.float32, device=dev)
        for _ in range(2):
            abi.block_forward(xp, lwp, out=outp)
        torch.cuda.synchronize()
        ms_p = time_stream(lambda: abi.block_forward(xp, lwp, out=outp), args.prefill_steps, torch)
        flops = synth.prefill_flops(4096, lwp)
        tflops = flops / (ms_p * 1e-3) / 1e12
        prefill = {"prefill_tok_s": 4096 / (ms_p * 1e-3), "prefill_ms": ms_p,
                   "prefill_tflops": tflops, "prefill_mfma_util": tflops / BF16_PEAK_TFLOPS}
        log(f"prefill T=4096: {ms_p:.2f} ms, {prefill['prefill_tok_s']:.0f} tok/s, "
            f"{tflops:.1f} TFLOP/s ({100 * tflops / BF16_PEAK_TFLOPS:.1f}% of bf16 peak)")

    # ---------------------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu:
        from oracle import moe_oracle as O
        torch.set_num_threads(os.cpu_count() or 1)
        ow = O.from_device(layers[0])
        xc = x0.cpu()
        n, t_cpu = 0, 0.0
        t_start = time.time()
        while time.time() - t_start < args.cpu_seconds:
            t1 = time.perf_counter()
            res = O.moe_block(xc, ow)
            t_cpu += time.perf_counter() - t1
            xc = synth.rms_normalize(xc + res["combined_out"])
            n += 1
        cpu = {"value": t_cpu / n * 1e6, "unit": "us/token/layer", "cores": torch.get_num_threads(),
               "kind": "port",
               "sample": f"{n} sequential decode tokens through one layer (config 0/1 shapes): "
                         "oracle dequant of the 8 selected Q4_K experts + f32 F.linear + shared"}
        log(f"cpu baseline: {cpu['value']:.0f} us/token/layer over {n} tokens, {cpu['cores']} threads")

    result = {
        "metric": "MoE-layer us/token + HBM GB/s at bs=1 (Q4_K); prefill tok/s at 4096 tokens",
        "value": round(us_tok_layer, 3), "unit": "us/token/layer", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q4_K, N(0,1) activations)",
        "config": {"workload": f"config 1: decode bs=1, {L} resident layer instances, "
                               f"{args.steps} sequential tokens (x <- x + MoE(x) per layer, "
                               "RMS-renormalised per token)", "layers": L,
                   "tokens": args.steps, "experts": 256, "top_k": 8, "hidden": 2048,
                   "moe_intermediate": 512, "format": "Q4_K"},
        "decode_hbm_gbps": round(gbps, 1),
        "decode_hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(exp_gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(exp_gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "routed experts GEMV (k_gemv_gateup_q4k + k_gemv_down_q4k)",
                     "bytes_per_launch": routed_bytes, "avg_us": round(ms_exp * 1000, 3)},
        "cpu_baseline": cpu,
    }
    result.update({k: (round(v, 4) if isinstance(v, float) else v) for k, v in prefill.items()})
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
