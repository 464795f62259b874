"""Benchmark of the gfx950 MoE block on BASELINE.json's configs (one MI355X).

Headline (`value`): Q4_K MoE-layer decode at bs=1, config 1 — 40 independent resident layer
instances (~18.1 GB of Q4_K experts, so every expert byte comes from HBM), one token at a time
through all 40 layers as the decoder's MoE half runs them (engine/m3_forward.py:732-737):
h <- h + MoE(rmsnorm(h)) per layer, the post-attention RMSNorm and the residual add fused into the
single-launch layer, each layer's input the previous layer's output; h is rescaled to RMS 1
between tokens. 1024 sequential tokens by default. A step is one token through the 40 layers; it is captured once as a
HIP graph and replayed. Reported as us per token per layer, with the HBM rate over the 8 routed +
1 shared active experts' bytes (20,447,232 B per token-layer).

`roofline`: the dominant kernel of that path, the single-launch decode layer (k_dec_layer), timed
alone with HIP events on the stream it is launched on: a graph of 40 back-to-back launches over
the 40 layers (independent inputs), replayed; average launch period = elapsed / launches.
`traffic` comes from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of the same kernel
(`--pmc` workload, calibrated against a copy kernel of known size).

Also on the line: batched decode at T = 64 with Zipf routing (config 2), prefill tokens/s at
T = 4096 (config 3) with MFMA utilisation against the bf16 dense peak, and the CPU baseline (this
repo's CPU oracle of the same block, timed on the host on a bounded sample).

Usage:
  python bench.py [--gpus 1] [--steps 1024] [--warmup 16] [--layers 40] [--no-cpu] [--no-prefill]
  python bench.py --pmc [--no-hint]          short decode workload + copy calibration (for rocprofv3 --pmc)
  python bench.py --pmc-summary DF DW [DFH DWH]   traffic summary (markdown) from --pmc runs
  python bench.py --stats-summary DIR [CMD]   kernel table (markdown) from rocprofv3 --kernel-trace --stats
  python bench.py --pmc-prefill               config-3 prefill workload (for rocprofv3 --pmc passes)
  python bench.py --pmc-prefill-summary DIR_A DIR_T   MFMA counter summary (markdown) of the GEMMs
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
TRAFFIC_SUMMARY = ROOT / "profiles" / "k_dec_layer_c1_traffic.md"
DECODE_KERNEL = "k_dec_layer"
COPY_MIB = 512                      # calibration copy: reads and writes this many MiB
PMC_REGEX = "k_dec_layer|MulFunctor"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--kernel-reps", type=int, default=64)
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-c2", action="store_true")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the config-3 prefill timing (what the prefill profile covers)")
    ap.add_argument("--c2-only", action="store_true",
                    help="only the config-2 batched-decode timing (what the c2 profile covers)")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the dominant-kernel timing (what the kernel-trace profile covers)")
    ap.add_argument("--no-lm-head", action="store_true")
    ap.add_argument("--no-c4", action="store_true", help="skip the config-4 prefill timing")
    ap.add_argument("--c4-only", action="store_true",
                    help="only the config-4 prefill timing (what the c4 profile covers)")
    ap.add_argument("--no-artifact", action="store_true",
                    help="skip the decode chain over the shipped artifact's weight widths")
    ap.add_argument("--lm-head-only", action="store_true",
                    help="only the untied lm_head GEMV timing (what the lm_head profile covers)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--peaks-only", action="store_true",
                    help="only the measured HBM read and f16 MFMA peaks")
    ap.add_argument("--pmc", action="store_true")
    ap.add_argument("--no-hint", action="store_true",
                    help="call moe_block_forward (no next-layer L2 warm-up) in the decode runs")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="DIR_FETCH DIR_WRITE of --pmc --no-hint runs [then of --pmc runs]")
    ap.add_argument("--stats-summary", nargs="+", metavar="DIR [CMD]")
    ap.add_argument("--pmc-prefill", action="store_true",
                    help="config-3 prefill steps only, untimed (what the MFMA counter passes profile)")
    ap.add_argument("--pmc-prefill-summary", nargs=2, metavar=("DIR_PMC", "DIR_TRACE"),
                    help="MFMA counter summary from a --pmc run and a --kernel-trace run of --pmc-prefill")
    return ap.parse_args()


def time_stream(fn, n: int, torch, stream=None) -> float:
    """Average ms of fn() over n calls, HIP events on `stream` (default: the current stream)."""
    st = stream or torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(n):
        fn()
    b.record(st)
    b.synchronize()
    return a.elapsed_time(b) / n


def capture(torch, fn):
    """fn's launches captured into a HIP graph on a side stream. One eager run on that stream
    first: the library's per-stream workspace is then created (and initialised) outside the
    graph, so its one-time initialisation is not replayed with every step."""
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        fn()
    cap.synchronize()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            fn()
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    return g


# ------------------------------------------------------------------------------ rocprof helpers --
def _counter_rows(d: str):
    files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no counter_collection.csv under {d}")
    for f in files:
        with open(f) as fh:
            yield from csv.DictReader(fh)


def _per_dispatch(d: str, counter: str):
    """{kernel name: [per-dispatch value]} for one counter (summed over its dimension rows)."""
    acc: dict[tuple, float] = {}
    names: dict[tuple, str] = {}
    for r in _counter_rows(d):
        if r.get("Counter_Name") != counter:
            continue
        key = (r.get("Dispatch_Id"), r.get("Agent_Id"))
        acc[key] = acc.get(key, 0.0) + float(r["Counter_Value"])
        names[key] = r.get("Kernel_Name", "")
    out: dict[str, list] = {}
    for k, v in acc.items():
        out.setdefault(names[k], []).append(v)
    return out


def pmc_summary(dir_fetch: str, dir_write: str, dir_fetch_hint: str | None = None,
                dir_write_hint: str | None = None) -> str:
    """Markdown summary of rocprofv3 --pmc runs of `bench.py --pmc`: FETCH_SIZE / WRITE_SIZE
    (KiB per dispatch) of the decode layer kernel, scaled by what the same counters read for a
    plain copy of COPY_MIB MiB (known bytes each way). The first pair of runs is the plain entry
    (`--no-hint`) and gives the per-launch traffic; the optional second pair is the same workload
    with the next-layer L2 warm-up."""
    import statistics

    def pick(d, pat):
        ks = [k for k in d if re.search(pat, k)]
        if not ks:
            raise SystemExit(f"no kernel matching {pat!r} in {sorted(d)[:8]}")
        return max(ks, key=lambda k: len(d[k]))

    def largest(d, pat):
        vals = [(v, k) for k in d if re.search(pat, k) for v in d[k]]
        if not vals:
            raise SystemExit(f"no kernel matching {pat!r}")
        return max(vals)

    def measure(df, dw):
        f, w = _per_dispatch(df, "FETCH_SIZE"), _per_dispatch(dw, "WRITE_SIZE")
        kf, kw = pick(f, DECODE_KERNEL), pick(w, DECODE_KERNEL)
        # the calibration multiply is the largest elementwise dispatch of the run
        copy_f, cf = largest(f, r"elementwise")
        copy_w, _ = largest(w, r"elementwise")
        copy_kib = COPY_MIB * 1024.0
        sf, sw = copy_kib / copy_f, copy_kib / copy_w
        return dict(kernel=kf, n=len(f[kf]), fk=statistics.median(f[kf]), wk=statistics.median(w[kw]),
                    fetch=statistics.median(f[kf]) * sf * 1024.0,
                    write=statistics.median(w[kw]) * sw * 1024.0, sf=sf, sw=sw, copy_f=copy_f,
                    copy_w=copy_w, copy_kib=copy_kib, copy_name=cf)

    m = measure(dir_fetch, dir_write)
    mh = measure(dir_fetch_hint, dir_write_hint) if dir_fetch_hint and dir_write_hint else None
    cmd = "rocprofv3 --pmc {c} --kernel-include-regex '" + PMC_REGEX + "' --output-format csv -d {d} -o {o} -- python3 bench.py --pmc"
    lines = [
        "# k_dec_layer (config 1 decode layer): HBM traffic per launch from rocprofv3 PMC",
        "",
        "Commands (GPU box, repo root):",
        "",
        "    " + cmd.format(c="FETCH_SIZE", d="/tmp/pf", o="f") + " --no-hint",
        "    " + cmd.format(c="WRITE_SIZE", d="/tmp/pw", o="w") + " --no-hint",
    ]
    if mh:
        lines += ["    " + cmd.format(c="FETCH_SIZE", d="/tmp/pfh", o="f"),
                  "    " + cmd.format(c="WRITE_SIZE", d="/tmp/pwh", o="w"),
                  "    python3 bench.py --pmc-summary /tmp/pf /tmp/pw /tmp/pfh /tmp/pwh"]
    else:
        lines += ["    python3 bench.py --pmc-summary /tmp/pf /tmp/pw"]
    lines += [
        "",
        f"Calibration: a {COPY_MIB} MiB elementwise multiply ({m['copy_name'][:60]}) reads {m['copy_f']:.0f} KiB (FETCH_SIZE)",
        f"and writes {m['copy_w']:.0f} KiB (WRITE_SIZE) for {m['copy_kib']:.0f} KiB each way:",
        f"scale factors fetch {m['sf']:.4f}, write {m['sw']:.4f}.",
        "",
        "| entry | kernel | dispatches | FETCH_SIZE KiB (median) | WRITE_SIZE KiB (median) | scaled fetch B | scaled write B |",
        "|---|---|---|---|---|---|---|",
        f"| moe_block_forward | {m['kernel'][:60]} | {m['n']} | {m['fk']:.1f} | {m['wk']:.1f} "
        f"| {m['fetch']:.0f} | {m['write']:.0f} |",
    ]
    if mh:
        lines.append(f"| moe_block_forward_prefetch | {mh['kernel'][:60]} | {mh['n']} | {mh['fk']:.1f} | "
                     f"{mh['wk']:.1f} | {mh['fetch']:.0f} | {mh['write']:.0f} |")
    lines += [
        "",
        f"traffic_bytes_per_launch: {m['fetch'] + m['write']:.0f}",
        "",
        "Algorithmic bytes per launch: 20,447,232 (8 routed Q4_K experts + bf16 shared expert) plus",
        "1,052,672 router + shared-gate bytes = 21,499,904. Each of the 8 XCDs computes all 256",
        "router logits (no cross-XCD logit exchange), so the 1 MiB router matrix leaves L2 once per",
        f"XCD: of the {m['fetch'] + m['write'] - 21499904:.0f} B above the algorithmic bytes, 7 x 1,048,576 B are these",
        "re-reads (served from the MALL or HBM); the rest is x, the norm weight and the exchange words",
        "per XCD and the output writes.",
    ]
    if mh:
        lines += [
            "",
            "With the warm-up hint each launch also reads the next layer's router rows and norm weight",
            "into its XCD's L2; in a chain of launches the next launch then finds them there, so",
            "the bytes move from one launch to the one before it. A PMC run serialises dispatches and the",
            "warmed lines do not survive to the next one, which counts these bytes twice; the per-launch",
            "figure is therefore the plain entry's.",
        ]
    return "\n".join(lines) + "\n"


def stats_summary(d: str, cmd: str) -> str:
    """Markdown table of the kernels in a rocprofv3 --kernel-trace --stats run, by total time."""
    files = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_stats.csv under {d}")
    rows = []
    for f in files:
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    rows.sort(key=lambda r: -float(r.get("TotalDurationNs", 0) or 0))
    ours = [r for r in rows if "moe::" in r["Name"]]
    rest = [r for r in rows if "moe::" not in r["Name"]][:10]
    out = ["# rocprofv3 kernel statistics", "", "Command (GPU box, repo root):", "", f"    {cmd}", "",
           "This library's kernels (moe::) first, then the ten largest others (input generation).", "",
           "| kernel | calls | avg us | min us | max us | total ms | % |", "|---|---|---|---|---|---|---|"]
    for r in ours + rest:
        name = re.sub(r"\s+", " ", r["Name"])[:90]
        out.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                   f"{float(r['TotalDurationNs']) / 1e6:.3f} | {float(r.get('Percentage', 0) or 0):.1f} |")
    return "\n".join(out) + "\n"


PREFILL_PMC = ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_BUSY_CU_CYCLES",
               "SQ_WAVE_CYCLES", "SQ_WAIT_ANY", "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_LDS", "GRBM_GUI_ACTIVE"]
PREFILL_KERNELS = {"k_gemm4_gateup": 137438953472.0, "k_gemm4_down": 68719476736.0}   # FLOP per launch at T = 4096
N_CU, N_SIMD = 256, 4


def pmc_prefill_summary(dir_pmc: str, dir_trace: str) -> str:
    """Markdown summary of the config-3 grouped GEMMs from one rocprofv3 --pmc pass (PREFILL_PMC)
    and one --kernel-trace pass of `bench.py --pmc-prefill`: medians per dispatch of each counter,
    the f16 MFMA FLOPs the counters count (MOPS x 512) against the algorithmic FLOPs, and two
    utilisations: achieved = counted FLOPs / kernel duration / 2.5 PFLOP/s, and MFMA busy =
    SQ_VALU_MFMA_BUSY_CYCLES / (SQ_BUSY_CU_CYCLES x 4 SIMDs)."""
    import statistics
    per = {c: _per_dispatch(dir_pmc, c) for c in PREFILL_PMC}
    files = glob.glob(os.path.join(dir_trace, "**", "*kernel_stats.csv"), recursive=True)
    if not files:
        raise SystemExit(f"no kernel_stats.csv under {dir_trace}")
    dur = {}
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                dur[r["Name"]] = float(r["AverageNs"])
    lines = [
        "# Config-3 prefill grouped GEMMs: MFMA counters (rocprofv3 --pmc)", "",
        "Commands (GPU box, repo root):", "",
        "    rocprofv3 --pmc " + " ".join(PREFILL_PMC) + " --kernel-include-regex 'k_gemm4' "
        "--output-format csv -d /tmp/ppmc -o p -- python3 bench.py --pmc-prefill",
        "    rocprofv3 --kernel-trace --stats --kernel-include-regex 'k_gemm4' --output-format csv "
        "-d /tmp/ptr -o t -- python3 bench.py --pmc-prefill",
        "    python3 bench.py --pmc-prefill-summary /tmp/ppmc /tmp/ptr", "",
        "Per dispatch (median over the run's dispatches). FLOP(counted) = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512",
        "(it includes the zero rows of partly filled row tiles); issued = FLOP(counted) / average kernel",
        "duration; algorithmic = FLOP(algorithmic) / average kernel duration; % of peak uses 2.5 PFLOP/s",
        "(dense f16/bf16);",
        f"MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (SQ_BUSY_CU_CYCLES x {N_SIMD}).", "",
        "| kernel | dispatches | avg us | FLOP algorithmic | FLOP counted | algorithmic TFLOP/s | algorithmic % "
        "of peak | issued TFLOP/s | MFMA busy % | SQ_WAIT_ANY / SQ_WAVE_CYCLES | LDS bank conflicts / LDS insts |",
        "|---|---|---|---|---|---|---|---|---|---|---|"]
    out = {}
    for kname, flop_alg in PREFILL_KERNELS.items():
        med = {}
        for c in PREFILL_PMC:
            ks = [k for k in per[c] if kname in k]
            if not ks:
                raise SystemExit(f"no {kname} dispatch with counter {c}")
            med[c] = statistics.median(v for k in ks for v in per[c][k])
        n = sum(len(per[PREFILL_PMC[0]][k]) for k in per[PREFILL_PMC[0]] if kname in k)
        us = statistics.median(v for k, v in dur.items() if kname in k) / 1e3
        flop = med["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512.0
        tf = flop / (us * 1e-6) / 1e12
        tfa = flop_alg / (us * 1e-6) / 1e12
        busy = med["SQ_VALU_MFMA_BUSY_CYCLES"] / max(med["SQ_BUSY_CU_CYCLES"] * N_SIMD, 1.0)
        wait = med["SQ_WAIT_ANY"] / max(med["SQ_WAVE_CYCLES"], 1.0)
        conf = med["SQ_LDS_BANK_CONFLICT"] / max(med["SQ_INSTS_LDS"], 1.0)
        out[kname] = dict(us=us, tflops=tfa, frac=tfa / BF16_PEAK_TFLOPS, issued_tflops=tf, busy=busy)
        lines.append(f"| {kname} | {n} | {us:.1f} | {flop_alg:.4g} | {flop:.4g} | {tfa:.0f} | "
                     f"{100 * tfa / BF16_PEAK_TFLOPS:.1f} | {tf:.0f} | {100 * busy:.1f} | {wait:.3f} | {conf:.2f} |")
    lines += ["", "Raw medians per dispatch:", "", "| kernel | " + " | ".join(PREFILL_PMC) + " |",
              "|---|" + "---|" * len(PREFILL_PMC)]
    for kname in PREFILL_KERNELS:
        vals = []
        for c in PREFILL_PMC:
            vals.append(statistics.median(v for k in per[c] if kname in k for v in per[c][k]))
        lines.append(f"| {kname} | " + " | ".join(f"{v:.4g}" for v in vals) + " |")
    lines += ["", "prefill_gemm_summary: " + json.dumps({k: {kk: round(vv, 4) for kk, vv in v.items()}
                                                       for k, v in out.items()})]
    return "\n".join(lines) + "\n"


PREFILL_PMC_SUMMARY = ROOT / "profiles" / "prefill_c3_pmc.md"


PREFILL_STATS_SUMMARY = ROOT / "profiles" / "prefill_c3_kernel_stats.md"


def committed_prefill_pmc():
    """The GEMMs' counter figures from the committed summary (or None). Their "us" is the counter
    pass's own kernel trace (3 blocks of the --pmc-prefill workload); "us_kernel_stats" and
    "frac_kernel_stats" put the same algorithmic FLOPs over the average duration of the committed
    22-block kernel statistics of the timed workload, which is the figure the block time
    contains."""
    try:
        m = re.search(r"prefill_gemm_summary:\s*(\{.*\})", PREFILL_PMC_SUMMARY.read_text())
        out = json.loads(m.group(1)) if m else None
    except (OSError, ValueError):
        return None
    if out is None:
        return None
    try:
        stats = PREFILL_STATS_SUMMARY.read_text()
    except OSError:
        stats = ""
    for name, v in out.items():
        v["us_source"] = "profiles/prefill_c3_pmc.md (counter pass, 3 blocks)"
        row = re.search(r"\|\s*`[^`]*" + re.escape(name) + r"[^`]*`\s*\|\s*\d+\s*\|\s*([0-9.]+)\s*\|", stats)
        if row and v.get("us") and v.get("tflops"):
            us = float(row.group(1))
            flop = v["tflops"] * 1e12 * v["us"] * 1e-6
            v["us_kernel_stats"] = us
            v["frac_kernel_stats"] = round(flop / (us * 1e-6) / (BF16_PEAK_TFLOPS * 1e12), 4)
    return out


def committed_traffic():
    try:
        m = re.search(r"traffic_bytes_per_launch:\s*([0-9.]+)", TRAFFIC_SUMMARY.read_text())
        return float(m.group(1)) if m else None
    except OSError:
        return None


# ------------------------------------------------------------------------------------ workloads --
def pmc_workload(pkg, torch, dev, L: int, hint: bool) -> None:
    """What the PMC passes profile: 4 tokens through L decode layers (eager), then the copy."""
    synth, abi = pkg.synth, pkg.abi
    layers = [synth.make_layer(seed=1000 + l, device=dev) for l in range(L)]
    norms = [synth.make_norm_weight(seed=5000 + l, device=dev) for l in range(L)]
    x = synth.make_input(1, seed=0, device=dev)
    for _ in range(4):
        for l, (lw, nw) in enumerate(zip(layers, norms)):
            abi.block_forward(x, lw, out=x, residual=x, norm_w=nw,
                              next_layer=layers[(l + 1) % L] if hint else None,
                              next_norm_w=norms[(l + 1) % L] if hint else None)
        x.copy_(synth.rms_normalize(x))
    torch.cuda.synchronize()
    del layers
    src = torch.ones(COPY_MIB * 2 ** 20 // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.mul(src, 2.0, out=dst)         # an elementwise kernel: reads and writes COPY_MIB MiB
    torch.cuda.synchronize()
    log(f"pmc workload done: {4 * L} decode-layer launches, one {COPY_MIB} MiB elementwise copy")


def dominant_kernel_ms(torch, synth, abi, layers, norms, dev, reps: int, hint: bool = True) -> float:
    """Average launch period of the single-launch decode layer (norm fused, as in the decode
    chain): a graph of len(layers) back-to-back launches on independent inputs, replayed `reps`
    times, HIP events on the stream the graph runs on."""
    L = len(layers)
    xs = synth.make_input(L, seed=7, device=dev)
    ys = torch.empty_like(xs)

    def layer_launches():
        for l, lw in enumerate(layers):
            abi.block_forward(xs[l:l + 1], lw, out=ys[l:l + 1], residual=xs[l:l + 1],
                              norm_w=norms[l], next_layer=layers[(l + 1) % L] if hint else None,
                              next_norm_w=norms[(l + 1) % L] if hint else None)

    layer_launches()
    torch.cuda.synchronize()
    gk = capture(torch, layer_launches)
    for _ in range(4):
        gk.replay()
    torch.cuda.synchronize()
    return time_stream(gk.replay, reps, torch) / L


def c2_step(torch, synth, abi, dev, reps: int) -> dict:
    """Config 2: one block over T = 64 tokens with Zipf-skewed routing, captured in a HIP graph;
    HBM rate over the unique experts the step hits (each read once) plus the shared expert."""
    lz = synth.make_layer(seed=1, device=dev, zipf=True)
    xz = synth.make_input(64, seed=1, device=dev)
    oz = torch.empty_like(xz)
    r = abi.router_topk(xz, lz.router, lz.top_k, bias=lz.router_bias)
    uniq = int(torch.unique(r["topk_ids"]).numel())
    for _ in range(3):
        abi.block_forward(xz, lz, out=oz)
    torch.cuda.synchronize()
    gz = capture(torch, lambda: abi.block_forward(xz, lz, out=oz))
    ms_z = time_stream(gz.replay, reps, torch)
    bytes_z = uniq * lz.routed_bytes_per_expert() + lz.shared_bytes()
    out = {"c2_us_per_step": round(ms_z * 1000, 2), "c2_unique_experts": uniq,
           "c2_gbps": round(bytes_z / (ms_z * 1e-3) / 1e9, 1)}
    log(f"c2 T=64 zipf: {ms_z * 1000:.1f} us/step, {uniq} unique experts, {out['c2_gbps']:.0f} GB/s")
    return out


def prefill_c3(torch, synth, abi, lwp, dev, steps: int) -> dict:
    """Config 3: one block over T = 4096 bf16 tokens (uniform routing), HIP events."""
    xp = synth.make_input(4096, seed=2, device=dev, dtype=torch.bfloat16)
    outp = torch.empty(4096, 2048, dtype=torch.float32, device=dev)
    for _ in range(2):
        abi.block_forward(xp, lwp, out=outp)
    torch.cuda.synchronize()
    ms_p = time_stream(lambda: abi.block_forward(xp, lwp, out=outp), steps, torch)
    flops = synth.prefill_flops(4096, lwp)
    tflops = flops / (ms_p * 1e-3) / 1e12
    log(f"prefill T=4096: {ms_p:.3f} ms, {4096 / (ms_p * 1e-3):.0f} tok/s, "
        f"{tflops:.1f} TFLOP/s ({100 * tflops / BF16_PEAK_TFLOPS:.1f}% of bf16 peak)")
    return {"prefill_tok_s": 4096 / (ms_p * 1e-3), "prefill_ms": ms_p,
            "prefill_tflops": tflops, "prefill_mfma_util": tflops / BF16_PEAK_TFLOPS}


PROBE_LIB = ROOT / "qwen3.6-35b-a3b_amd" / "libmoe_peak_probe.so"


def measured_peaks(torch, dev, read_gib: int = 4) -> dict:
    """Peaks measured on this GPU with the probes of csrc/probe/peak_probe.hip (the method of the
    reference's tools/bw_probe_hip.cpp and tools/gemm_peak.cpp): the best HBM read rate over a
    sweep of grid sizes (a read_gib GiB buffer, 16 times the MALL, so every byte comes from HBM),
    and the best f16 MFMA rate (v_mfma_f32_32x32x16_f16, operands in registers) over a sweep of
    waves per CU. HIP events on the stream the probes are launched on."""
    import ctypes
    lib = ctypes.CDLL(str(PROBE_LIB))
    lib.probe_hbm_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_void_p]
    lib.probe_mfma_f16.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    st = torch.cuda.current_stream(dev)
    sp = ctypes.c_void_p(st.cuda_stream)
    sink = torch.zeros(16, dtype=torch.float32, device=dev)
    nbytes = read_gib << 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    best_bw, bw_sweep = 0.0, {}
    for blocks in (2048, 4096, 8192, 16384, 32768, 65536):
        run = lambda: lib.probe_hbm_read(ctypes.c_void_p(buf.data_ptr()), nbytes, blocks,
                                         ctypes.c_void_p(sink.data_ptr()), sp)
        if run() != 0:
            raise RuntimeError("probe_hbm_read failed")
        ms = time_stream(run, 5, torch, st)
        gbs = nbytes / (ms * 1e-3) / 1e9
        bw_sweep[blocks] = round(gbs, 1)
        best_bw = max(best_bw, gbs)
    del buf
    torch.cuda.empty_cache()
    best_tf, tf_sweep = 0.0, {}
    iters = 2048
    for blocks in (256, 512, 1024, 2048):
        run = lambda: lib.probe_mfma_f16(blocks, iters, ctypes.c_void_p(sink.data_ptr()), sp)
        if run() != 0:
            raise RuntimeError("probe_mfma_f16 failed")
        ms = time_stream(run, 5, torch, st)
        flop = blocks * 4 * 4 * iters * 32768.0
        tf = flop / (ms * 1e-3) / 1e12
        tf_sweep[blocks] = round(tf, 1)
        best_tf = max(best_tf, tf)
    log(f"measured peaks: HBM read {best_bw:.0f} GB/s (by grid {bw_sweep}); f16 MFMA "
        f"{best_tf:.0f} TFLOP/s (by grid {tf_sweep})")
    return {"hbm_read_gbps": round(best_bw, 1), "hbm_read_sweep": bw_sweep,
            "mfma_f16_tflops": round(best_tf, 1), "mfma_f16_sweep": tf_sweep}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def usable_cores() -> int:
    """Cores this process may run on (its affinity mask), not os.cpu_count()."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def cpu_baselines(torch, synth, lw_dec, x0, lw_pf, dev, seconds: float):
    """The reference's CPU path timed on this host (oracle port, BASELINE.md's plan): config-1
    decode tokens through one layer (each layer-token dequantizes its 8 selected experts), and
    config 3's 4096-token prefill block (every used expert dequantized once, grouped F.linear).
    Decode: a short probe at 1, 2, 4, 8 and all usable cores (the affinity mask), then the
    bounded sample at the fastest of them, plus a 1-thread line; the sample's mean per-token time
    is reported with the thread count that gave it. Prefill: one timed block at the usable core
    count after a warm-up call on 64 tokens."""
    from oracle import moe_oracle as O
    ncpu = usable_cores()
    model = cpu_model()
    ow = O.from_device(lw_dec)

    def decode(threads: int, budget: float, min_tokens: int = 3):
        torch.set_num_threads(threads)
        xc = x0.cpu()
        n, t_cpu, per = 0, 0.0, []
        t_start = time.time()
        while time.time() - t_start < budget or n < min_tokens:
            t1 = time.perf_counter()
            res = O.moe_block(xc, ow)
            dt = time.perf_counter() - t1
            t_cpu += dt
            per.append(dt)
            xc = synth.rms_normalize(xc + res["combined_out"])
            n += 1
        per.sort()
        return t_cpu / n, n, per

    probe = {}
    for th in sorted({1, 2, 4, 8, ncpu}):
        if th > ncpu:
            continue
        mean, _, _ = decode(th, 1.5)
        probe[th] = round(mean * 1e6, 1)
    best = min(probe, key=probe.get)
    log(f"cpu baseline probe (us/token/layer by threads, {ncpu} usable cores): {probe}; best {best}")

    def line(threads, mean, n, per, what):
        return {"value": round(mean * 1e6, 1), "unit": "us/token/layer", "cores": threads,
                "kind": "port",
                "sample": f"{n} sequential decode tokens through one config-1 layer: oracle "
                          "dequant of the 8 selected Q4_K experts + f32 F.linear + shared expert "
                          f"at {threads} torch threads ({what}; {ncpu} usable cores by the affinity "
                          f"mask, os.cpu_count()={os.cpu_count()}, {model}; per-token min "
                          f"{per[0] * 1e6:.0f} us, median {per[len(per) // 2] * 1e6:.0f} us; probe "
                          f"by threads {probe})"}

    mean, n, per = decode(best, seconds)
    cpu = line(best, mean, n, per, "the fastest thread count of the probe")
    log(f"cpu baseline: {cpu['value']:.0f} us/token/layer, {best} threads")
    mean1, n1, per1 = decode(1, max(4.0, seconds / 2))
    cpu1 = line(1, mean1, n1, per1, "one thread")
    log(f"cpu baseline, 1 thread: {cpu1['value']:.0f} us/token/layer")
    cpu_pf = None
    if lw_pf is not None:
        torch.set_num_threads(ncpu)
        owp = O.from_device(lw_pf)
        xp = synth.make_input(4096, seed=2, device=dev, dtype=torch.bfloat16).cpu()
        O.moe_block(xp[:64], owp)                               # warm-up (allocator, threads)
        t1 = time.perf_counter()
        O.moe_block(xp, owp)
        dt = time.perf_counter() - t1
        cpu_pf = {"value": round(4096 / dt, 1), "unit": "tok/s", "cores": torch.get_num_threads(),
                  "kind": "port",
                  "sample": f"config 3's 4096-token block once: oracle R1-R5, every used Q4_K expert "
                            f"dequantized once, grouped f32 F.linear, shared expert ({dt:.2f} s; "
                            f"{ncpu} usable cores, {model})"}
        log(f"cpu baseline, prefill: {cpu_pf['value']:.0f} tok/s ({dt:.2f} s for 4096 tokens)")
    torch.set_num_threads(ncpu)
    return cpu, cpu1, cpu_pf


def prefill_c4(torch, pkg, dev, steps: int, n_layers: int = 40) -> dict:
    """Config 4: T = 16384 bf16 tokens, Q4_K gate_up + Q6_K down, Zipf(1.1) routing, the step
    rotating over 40 resident layer instances (each step one block on the next instance)."""
    synth, abi = pkg.synth, pkg.abi
    layers = [synth.make_layer(seed=3000 + l, device=dev, down_fmt=pkg.quant.FMT_Q6_K, zipf=True)
              for l in range(n_layers)]
    x = synth.make_input(16384, seed=3, device=dev, dtype=torch.bfloat16)
    out = torch.empty(16384, 2048, dtype=torch.float32, device=dev)
    for l in range(2):
        abi.block_forward(x, layers[l], out=out)
    torch.cuda.synchronize()
    it = iter(range(10 ** 9))
    ms = time_stream(lambda: abi.block_forward(x, layers[next(it) % n_layers], out=out), steps, torch)
    flops = synth.prefill_flops(16384, layers[0])
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"prefill config 4 (T=16384, Q6_K down, Zipf, {n_layers} layers): {ms:.3f} ms, "
        f"{16384 / (ms * 1e-3):.0f} tok/s, {tflops:.1f} TFLOP/s ({100 * tflops / BF16_PEAK_TFLOPS:.1f}%)")
    del layers
    torch.cuda.empty_cache()
    return {"c4_prefill_ms": ms, "c4_tok_s": 16384 / (ms * 1e-3), "c4_mfma_util": tflops / BF16_PEAK_TFLOPS}


def lm_head_bench(torch, pkg, dev, reps: int = 20) -> dict:
    """The untied lm_head GEMV at the artifact's shape (248320 x 2048), one token, for each table
    width: kernel time from HIP events on the launching stream and table GB/s (each byte read
    once per call)."""
    L_, abi, Q = pkg._lib, pkg.abi, pkg.quant
    V, H = 248320, 2048
    g = torch.Generator(device=dev).manual_seed(3)
    h = torch.randn(1, H, generator=g, device=dev)
    res = {}
    for name, fmt in (("q6k", L_.MOE_FMT_Q6_K), ("q8_0", L_.MOE_FMT_Q8_0), ("bf16", L_.MOE_FMT_BF16)):
        w = torch.randn(V, H, generator=g, device=dev) * 0.02
        t = w.to(torch.bfloat16) if fmt == L_.MOE_FMT_BF16 else Q.quantize(w, fmt)
        del w
        nbytes = t.numel() * t.element_size()
        for _ in range(3):
            abi.lm_head(h, t, fmt)
        torch.cuda.synchronize()
        ms = time_stream(lambda: abi.lm_head(h, t, fmt), reps, torch)
        gbs = nbytes / (ms * 1e-3) / 1e9
        log(f"lm_head {name}: {ms * 1000:.1f} us per token, {nbytes / 1e6:.0f} MB table, "
            f"{gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBPS:.1f}% of HBM peak)")
        res[f"lm_head_{name}_us"] = ms * 1000
        res[f"lm_head_{name}_gbps"] = gbs
        del t
        torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    if args.pmc_summary:
        if len(args.pmc_summary) not in (2, 4):
            raise SystemExit("--pmc-summary takes DIR_FETCH DIR_WRITE [DIR_FETCH_HINT DIR_WRITE_HINT]")
        print(pmc_summary(*args.pmc_summary), end="")
        return
    if args.pmc_prefill_summary:
        print(pmc_prefill_summary(*args.pmc_prefill_summary), end="")
        return
    if args.stats_summary:
        d = args.stats_summary[0]
        print(stats_summary(d, " ".join(args.stats_summary[1:]) or "(not given)"), end="")
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus must be 1 (multi-GPU "
                          "sharding is design-only)"}))
        sys.exit(2)
    import torch
    import __graft_entry__ as ge

    pkg = ge.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    synth, abi = pkg.synth, pkg.abi
    L = args.layers
    if args.pmc:
        pmc_workload(pkg, torch, dev, L, not args.no_hint)
        return

    if args.peaks_only:
        print(json.dumps(measured_peaks(torch, dev)), flush=True)
        return

    if args.c2_only:
        print(json.dumps(c2_step(torch, synth, abi, dev, 50)), flush=True)
        return

    if args.lm_head_only:
        r = lm_head_bench(torch, pkg, dev)
        print(json.dumps({k: round(v, 3) for k, v in r.items()}), flush=True)
        return

    if args.pmc_prefill:
        lwp = synth.make_layer(seed=2, device=dev)
        xp = synth.make_input(4096, seed=2, device=dev, dtype=torch.bfloat16)
        outp = torch.empty(4096, 2048, dtype=torch.float32, device=dev)
        for _ in range(3):
            abi.block_forward(xp, lwp, out=outp)
        torch.cuda.synchronize()
        log("pmc prefill workload done: 3 config-3 blocks")
        return

    if args.c4_only:
        r = prefill_c4(torch, pkg, dev, args.prefill_steps)
        print(json.dumps({k: round(v, 4) for k, v in r.items()}), flush=True)
        return

    if args.prefill_only:
        lwp = synth.make_layer(seed=2, device=dev)
        r = prefill_c3(torch, synth, abi, lwp, dev, args.prefill_steps)
        print(json.dumps({k: round(v, 4) for k, v in r.items()}), flush=True)
        return

    # ---------------------------------------------------------------- measured peaks
    peaks = measured_peaks(torch, dev) if not args.kernel_only else None

    # ---------------------------------------------------------------- decode, config 1
    t0 = time.time()
    layers = [synth.make_layer(seed=1000 + l, device=dev) for l in range(L)]
    torch.cuda.synchronize()
    resident = sum(lw.gate_up_q.numel() + lw.down_q.numel() for lw in layers)
    log(f"generated {L} layers ({resident / 1e9:.2f} GB routed Q4_K) in {time.time() - t0:.1f}s")
    active = synth.decode_active_bytes(layers[0])
    if args.kernel_only:
        norms = [synth.make_norm_weight(seed=5000 + l, device=dev) for l in range(L)]
        ms_k = dominant_kernel_ms(torch, synth, abi, layers, norms, dev, args.kernel_reps,
                                  not args.no_hint)
        log(f"{DECODE_KERNEL}: {ms_k * 1000:.2f} us per launch (graph of {L} launches), "
            f"{active / (ms_k * 1e-3) / 1e9:.0f} GB/s on {active} B")
        return
    x0 = synth.make_input(1, seed=0, device=dev)
    xbuf = x0.clone()
    norms = [synth.make_norm_weight(seed=5000 + l, device=dev) for l in range(L)]

    def one_token():
        # the residual stream through L layers: h <- h + MoE(rmsnorm(h)), in place; each call
        # names the next layer so its router rows and norm weight are warmed into L2
        for l, (lw, nw) in enumerate(zip(layers, norms)):
            abi.block_forward(xbuf, lw, out=xbuf, residual=xbuf, norm_w=nw,
                              next_layer=None if args.no_hint else layers[(l + 1) % L],
                              next_norm_w=None if args.no_hint else norms[(l + 1) % L])
        xbuf.copy_(synth.rms_normalize(xbuf))

    for _ in range(3):
        one_token()
    torch.cuda.synchronize()
    g = capture(torch, one_token)
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    ms = time_stream(g.replay, args.steps, torch)
    us_tok_layer = ms * 1000.0 / L
    gbps = active / (us_tok_layer * 1e-6) / 1e9
    log(f"decode: {ms:.3f} ms/token over {L} layers = {us_tok_layer:.2f} us/token/layer, "
        f"{gbps:.0f} GB/s on {active} active B/token-layer")

    ms_k = dominant_kernel_ms(torch, synth, abi, layers, norms, dev, args.kernel_reps,
                              not args.no_hint)
    kern_gbps = active / (ms_k * 1e-3) / 1e9
    traffic = committed_traffic()
    log(f"{DECODE_KERNEL}: {ms_k * 1000:.2f} us per launch (graph of {L} launches), "
        f"{kern_gbps:.0f} GB/s on {active} B; traffic/launch {traffic}")
    err_bits = abi.device_error_bits(dev)
    if err_bits:
        log(f"WARNING: device error bits {err_bits:#x} (a bounded spin timed out)")

    # ------------------------------------------------ decode over the artifact's weight widths
    art = {}
    if not args.no_artifact:
        del layers
        torch.cuda.empty_cache()
        alayers = [synth.make_layer(seed=2000 + l, device=dev, down_fmt=pkg.quant.FMT_Q5_K,
                                    router_dtype=torch.float32, scalar_gate_dtype=torch.float32,
                                    split_gate_up=True, shared_fmt=pkg.quant.FMT_Q8_0)
                   for l in range(L)]
        xbuf.copy_(x0)

        def art_token():
            for l, (lw, nw) in enumerate(zip(alayers, norms)):
                abi.block_forward(xbuf, lw, out=xbuf, residual=xbuf, norm_w=nw,
                                  next_layer=alayers[(l + 1) % L], next_norm_w=norms[(l + 1) % L])
            xbuf.copy_(synth.rms_normalize(xbuf))

        for _ in range(3):
            art_token()
        torch.cuda.synchronize()
        ga = capture(torch, art_token)
        for _ in range(args.warmup):
            ga.replay()
        torch.cuda.synchronize()
        ms_a = time_stream(ga.replay, min(args.steps, 256), torch)
        art = {"decode_artifact_us_per_token_layer": ms_a * 1000.0 / L}
        log(f"decode, artifact widths (f32 router and scalar gate, split gate/up, Q5_K down, "
            f"Q8_0 shared expert): "
            f"{ms_a * 1000.0 / L:.2f} us/token/layer")
        del alayers, ga
        torch.cuda.empty_cache()
        layers = [synth.make_layer(seed=1000, device=dev)]

    # ---------------------------------------------------------------- batched decode, config 2
    c2 = c2_step(torch, synth, abi, dev, 50) if not args.no_c2 else {}

    # ---------------------------------------------------------------- prefill, config 3
    prefill = {}
    lwp = None
    if not args.no_prefill:
        lwp = synth.make_layer(seed=2, device=dev)              # config 3's seed
        prefill = prefill_c3(torch, synth, abi, lwp, dev, args.prefill_steps)

    # ---------------------------------------------------------------- prefill, config 4
    c4 = {} if args.no_c4 else prefill_c4(torch, pkg, dev, args.prefill_steps)

    # ---------------------------------------------------------------- untied lm_head GEMV
    lmh = lm_head_bench(torch, pkg, dev) if not args.no_lm_head else {}

    # ---------------------------------------------------------------- CPU baseline
    cpu, cpu1, cpu_pf = None, None, None
    if not args.no_cpu:
        cpu, cpu1, cpu_pf = cpu_baselines(torch, synth, layers[0], x0, lwp, dev, args.cpu_seconds)
    del lwp

    result = {
        "metric": "MoE-layer us/token + HBM GB/s at bs=1 (Q4_K); prefill tok/s at 4096 tokens",
        "value": round(us_tok_layer, 3), "unit": "us/token/layer", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q4_K, N(0,1) activations)",
        "config": {"workload": f"config 1: decode bs=1, {L} resident layer instances, "
                               f"{args.steps} sequential tokens (h <- h + MoE(rmsnorm(h)) per "
                               "layer, norm and residual fused; h RMS-renormalised per token)",
                   "layers": L,
                   "tokens": args.steps, "experts": 256, "top_k": 8, "hidden": 2048,
                   "moe_intermediate": 512, "format": "Q4_K"},
        "decode_hbm_gbps": round(gbps, 1),
        "decode_hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(kern_gbps, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(kern_gbps / HBM_PEAK_GBPS, 4),
                     "traffic": traffic, "kernel": DECODE_KERNEL,
                     "bytes_per_launch": active, "avg_us": round(ms_k * 1000, 3),
                     "peak_measured": peaks["hbm_read_gbps"],
                     "frac_of_measured": round(kern_gbps / peaks["hbm_read_gbps"], 4)},
        "peaks_measured": peaks,
        "cpu_baseline": cpu,
        "cpu_baseline_1thread": cpu1,
        "cpu_baseline_prefill": cpu_pf,
        "prefill_gemm_counters": committed_prefill_pmc(),
    }
    result.update(c2)
    result.update({k: round(v, 3) for k, v in art.items()})
    result.update({k: round(v, 3) for k, v in lmh.items()})
    result.update({k: round(v, 4) for k, v in c4.items()})
    result.update({k: (round(v, 4) if isinstance(v, float) else v) for k, v in prefill.items()})
    if prefill:
        result["prefill_mfma_util_of_measured"] = round(prefill["prefill_tflops"] / peaks["mfma_f16_tflops"], 4)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
