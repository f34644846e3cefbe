#!/usr/bin/env python3
"""Benchmark of the MXFP4 MoE expert path on one MI355X.

Workload (default): a GPT-OSS-120B-shaped MoE layer, 128 experts, top-4, hidden 2880,
expert intermediate 2880, MXFP4 weights (codes uniform 0..15, E8M0 exponents uniform
in [120, 130]), bf16 biases and router N(0, 0.02), tokens N(0, 1), clamped SwiGLU.
  * decode step  = router top-k/softmax -> expert routing -> streamed gate_up (+SwiGLU)
                   -> down -> combine, over 64 tokens (the headline ``value``);
  * prefill step = router -> blockwise mapping -> grouped gate_up GEMM -> down GEMM ->
                   combine, over 4096 tokens (reported in ``prefill``).
Synthetic data: weights are drawn on the GPU directly in the packed layout (uniform
random bytes are uniform codes in any byte order) for ``--layers`` distinct layers
that the steps rotate through, so a step never finds its weights in the 256 MB
last-level cache.  The GPT-OSS-120B-shaped workload holds all 36 MoE layers of that
model by default (its whole expert set, 61 GB, resident on the GPU); the others 8.
Inputs are resident in HBM before timing starts.

Per-kernel durations come from HIP events the library records on the launch stream
around each stage, in an eager pass of their own; the timed regions record none.  ``roofline`` covers the dominant kernel of
the headline step (decode gate_up weight streaming: HBM bound); ``prefill.roofline``
covers the prefill gate_up GEMM (MFMA bound, bf16 MFMA after in-register dequant).

Before the per-kernel timing pass and again right before each timed region the step runs
untimed for ``--settle`` seconds (0.3 by default; counts reported as ``settle_steps``): a
GPU that has been idle reaches its steady clocks only after a few hundred milliseconds of
work, and a short timed region otherwise measures the clock ramp.  The decode steps are
replayed from a HIP graph of up to 40 consecutive steps, so the timed count is the requested
steps rounded down to a multiple of the graph's length (``steps`` in the JSON is the count
timed); prefill times exactly ``--prefill-steps`` eager steps.

``other_configs`` (default workload only) times the benchmark's other workloads once each,
with their binding-roofline fractions: the MXFP4 linear (W 5760 x 2880, x 128 x 2880), the
GPT-OSS-20B-shaped layer at decode (1, 4, 16 and 64 tokens) and prefill (4,096 tokens,
uniform and Zipf(1.2) routing), and the 256-expert top-8 layer (H 7168, I 2048, Zipf(1.0)
routing) at decode (128 tokens) and prefill (8,192 tokens).

``--weights bf16`` times the bf16-expert path instead (the reference's shard_on_block
operands; moe_cte prefill and moe_block_tkg decode) and prints a line of its own.

``cpu_baseline`` times the CPU oracle (a port of the reference's CPU flow: dense
all-expert fp32 decode, dense all-expert bf16 prefill) on every affinity core of the host,
over the full expert set: decode on the whole batch, prefill on a 256-token slice (linear in
tokens).
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

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
MXFP4_PEAK_TFLOPS = 10100.0

WORKLOADS = {
    # name: (E, K, H, I, swiglu_limit, biases, decode_T, prefill_T)
    "gptoss120b": (128, 4, 2880, 2880, 7.0, True, 64, 4096),
    "gptoss20b": (32, 4, 2880, 2880, 7.0, True, 64, 4096),
    "fine256": (256, 8, 7168, 2048, None, False, 128, 8192),
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--prefill-steps", type=int, default=20)
    ap.add_argument("--workload", default="gptoss120b", choices=sorted(WORKLOADS))
    ap.add_argument("--layers", type=int, default=None,
                    help="distinct layers rotated (default: 36 for gptoss120b, 8 otherwise)")
    ap.add_argument("--decode-tokens", type=int, default=None)
    ap.add_argument("--prefill-tokens", type=int, default=None)
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--zipf", type=float, default=None,
                    help="routing skew: router bias -s*log(1 + rank) over a random expert order")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the other workloads (MXFP4 linear, 20B-shaped decode and prefill, "
                         "256-expert decode and prefill) reported in other_configs")
    ap.add_argument("--no-graph", action="store_true", help="time decode with eager launches")
    ap.add_argument("--settle", type=float, default=0.3,
                    help="seconds of untimed steps after the warmup and again right before "
                         "each timed region, so that the GPU runs at its steady clocks "
                         "(0 disables)")
    ap.add_argument("--weights", default="mxfp4", choices=["mxfp4", "bf16"],
                    help="bf16: time the bf16-expert path (moe_cte shard_on_block prefill, "
                         "moe_block_tkg decode) instead; prints its own line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run three device copies of exactly 1 GiB (the reference "
                         "kernel that scales the rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def copy_calibration():
    import torch

    a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    a.fill_(1)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": a.numel(), "copies": 3}))


def make_layer(E, K, H, I, limit, biases, dev, gen, zipf=None):
    import torch

    import pkgload

    pkgload.load()
    from vllm_neuron_amd.layer import MXFP4MoE
    from vllm_neuron_amd.weights import MXFP4Experts

    def rbytes(*shape, lo=0, hi=256):
        return torch.randint(lo, hi, shape, dtype=torch.uint8, device=dev, generator=gen)

    def rnorm(*shape, std=0.02):
        return (torch.randn(shape, device=dev, generator=gen) * std).to(torch.bfloat16)

    gu_q = rbytes(E, 2 * I // 16, 8 * H)
    gu_s = rbytes(E, (2 * I + 63) // 64, 2 * H, lo=120, hi=131)
    dn_q = rbytes(E, H // 16, 8 * I)
    dn_s = rbytes(E, (H + 63) // 64, 2 * I, lo=120, hi=131)
    gub = rnorm(E, 2, I) if biases else None
    if gub is not None and limit is not None:
        gub[:, 1] += 1.0  # the loader pre-adds +1 to the up bias (GPT-OSS)
    dnb = rnorm(E, H) if biases else None
    w = MXFP4Experts(gu_q, gu_s, dn_q, dn_s, gub, dnb, E, H, I)
    rb = None
    if zipf:
        # Zipf-skewed routing: expert of rank r (a random order) gets logit bias -s*log(1 + r)
        rank = torch.randperm(E, device=dev, generator=gen).float()
        rb = (-zipf * torch.log1p(rank)).to(torch.bfloat16)
    return MXFP4MoE(w, rnorm(E, H), rb, K, limit)


def bytes_per_expert(H, I, biases):
    b = 2 * I * H // 2 + 2 * I * H // 32 + H * I // 2 + H * I // 32
    return b + ((2 * I + H) * 2 if biases else 0)


def gate_up_bytes_per_expert(H, I, biases):
    return 2 * I * H // 2 + 2 * I * H // 32 + (2 * I * 2 if biases else 0)


def measured_traffic(workload, decode_T, prefill_T):
    """HBM bytes per launch of the decode gate_up kernel and of the prefill gate_up GEMM,
    from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes (copy-calibrated) for this
    workload and batch sizes, else None; and the summary they come from."""
    path = ROOT / "profiles" / f"decode_traffic_{workload}.json"
    if not path.exists():
        return None, None, None
    d = json.loads(path.read_text())
    dec = d["traffic_bytes"] if d.get("decode_tokens") == decode_T else None
    pre = None
    if d.get("prefill_tokens") == prefill_T and d.get("prefill_gate_up"):
        v = next(iter(d["prefill_gate_up"].values()))
        pre = v["read_bytes"] + v["write_bytes"]
    return dec, pre, d["source"]


def cpu_model() -> str:
    """The host CPU's model name as lscpu reports it (/proc/cpuinfo if lscpu fails)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for ln in out.splitlines():
            if ln.strip().lower().startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            return next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")),
                        "unknown")
    except OSError:
        return "unknown"


def cpu_baseline(wl, decode_T, prefill_T, prefill_slice=256):
    """Time the CPU oracle (the reference's CPU flows) on every affinity core of this host,
    over the workload's full expert set.  Decode: the dense all-expert fp32 flow of
    moe_block_tkg on the whole batch (its cost is the per-call fp32 cast and product of
    every expert's weights, not linear in tokens).  Prefill: the dense all-expert bf16
    _torch_moe_impl flow on a slice of the tokens, scaled linearly to the batch (every
    product in it is linear in the token count).  Weights are bf16 values of the layer's
    shapes (one random expert repeated: the arithmetic and its cost do not depend on the
    values).  Returns dicts for decode and prefill."""
    import torch

    import pkgload

    pkgload.load()
    from vllm_neuron_amd import synthetic

    from oracle.layer import RefLayer

    E, K, H, I, limit, biases, _, _ = WORKLOADS[wl]
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    model = cpu_model()
    g = torch.Generator().manual_seed(5)

    def rn(*shape, std):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)

    gu = rn(1, H, 2 * I, std=H ** -0.5).repeat(E, 1, 1)
    dn = rn(1, I, H, std=I ** -0.5).repeat(E, 1, 1)
    gub = rn(E, 2 * I, std=0.02) if biases else None
    dnb = rn(E, H, std=0.02) if biases else None
    ref = RefLayer.from_dense(gu, dn, gub, dnb, rn(E, H, std=0.02), None, K, limit)

    def timed(fn, reps):
        fn()  # warm-up
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2], len(ts)

    base = {"unit": "tokens/s", "cores": cores, "kind": "port", "cpu": model,
            "affinity_cores": cores}
    res = {}
    x = synthetic.tokens(5, decode_T, H)
    t, n = timed(lambda: ref.decode(x), 3)
    res["decode"] = dict(base, value=decode_T / t,
                         sample=f"dense all-expert fp32 decode (reference moe_block_tkg CPU flow) "
                                f"of all {decode_T} tokens over all {E} experts, median of {n} "
                                f"reps after one warm-up, {t:.2f} s per call, unscaled")
    t_s = min(prefill_T, prefill_slice)
    xp = synthetic.tokens(6, t_s, H)
    t, n = timed(lambda: ref.prefill(xp), 3)
    res["prefill"] = dict(base, value=t_s / t,
                          sample=f"dense all-expert bf16 prefill (reference _torch_moe_impl CPU "
                                 f"flow) of a {t_s}-token slice over all {E} experts, median of "
                                 f"{n} reps after one warm-up, {t:.2f} s per call; tokens/s of "
                                 f"the slice (the flow is linear in tokens, so the "
                                 f"{prefill_T}-token batch takes x{prefill_T / t_s:g} the time)")
    return res


def bench_bf16(args):
    """The bf16-expert path on one layer of random bf16 experts (gate_up [E, H, 2, I], down
    [E, I, H]): prefill = router -> mapping -> moe_cte(shard_on_block), GEMM durations from
    the library's stage events in a pass of their own; decode = moe_block_tkg (RMSNorm,
    router, experts), eager steps.  One JSON line."""
    import torch

    import pkgload

    pkgload.load()
    from vllm_neuron_amd import functional as NF

    dev = torch.device("cuda:0")
    E, K, H, I, limit, biases, dT, pT = WORKLOADS[args.workload]
    dT = args.decode_tokens or dT
    pT = args.prefill_tokens or pT
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    rn = lambda *s, std: (torch.randn(*s, device=dev, generator=g) * std).to(torch.bfloat16)  # noqa: E731
    gu, dn = rn(E, H, 2, I, std=H ** -0.5), rn(E, I, H, std=I ** -0.5)
    gb = rn(E, 2, I, std=0.02) if biases else None
    db = rn(E, H, std=0.02) if biases else None
    rw = rn(H, E, std=0.02)
    lim = {} if limit is None else dict(gate_clamp_upper_limit=limit,
                                        up_clamp_upper_limit=limit + 1,
                                        up_clamp_lower_limit=-limit + 1)
    act = "Swish" if limit is not None else "SiLU"

    def timed(fn, n):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        end = time.perf_counter() + args.settle
        while time.perf_counter() < end:
            fn()
            torch.cuda.synchronize()
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    x = torch.randn(pT, H, device=dev, generator=g).to(torch.bfloat16)

    def prefill(evs=None):
        aff = NF.router(x, rw, K, None, "softmax", computation_dtype=torch.float32)
        am, tp, b2e, _ = NF.build_blockwise_mapping(aff, E, K, 256)
        return NF.moe_cte(x, am, gu, dn, tp, b2e, 256, implementation="shard_on_block",
                          gate_and_up_proj_bias=gb, down_proj_bias=db, activation_function=act,
                          stage_events=evs, **lim)

    pms = timed(prefill, args.prefill_steps)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    stage = {"gate_up": [], "down": [], "combine": []}
    for _ in range(args.prefill_steps):
        prefill(evs)
        torch.cuda.synchronize()
        for i, k in enumerate(stage):
            stage[k].append(evs[i].elapsed_time(evs[i + 1]))
    med = {k: sorted(v)[len(v) // 2] for k, v in stage.items()}
    pairs = pT * K
    gu_tf = pairs * 4 * H * I / (med["gate_up"] * 1e-3) / 1e12
    dn_tf = pairs * 2 * H * I / (med["down"] * 1e-3) / 1e12

    xd = torch.randn(dT, H, device=dev, generator=g).to(torch.bfloat16)
    gamma = torch.ones(1, H, device=dev)
    dms = timed(lambda: NF.moe_block_tkg(
        xd.unsqueeze(0), gamma, rw, gu, dn, top_k=K, expert_gate_up_bias=gb,
        expert_down_bias=db, router_act_fn="SOFTMAX", router_pre_norm=False,
        expert_affinities_scaling_mode="POST_SCALE", hidden_act_fn=act,
        skip_router_logits=True, **lim), args.steps)
    from vllm_neuron_amd.functional.moe.moe_block_tkg import rmsnorm
    xn = rmsnorm(xd, gamma, 1e-6)
    touched = int(torch.topk(xn.float() @ rw.float(), K, dim=1).indices.unique().numel())
    dbytes = touched * 3 * H * I * 2
    out = {
        "metric": "bf16-expert MoE layer tokens/s @1 GPU (secondary path)",
        "value": dT / (dms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": 0, "ms_per_step": dms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random bf16 experts, N(0,1) tokens), weights resident in HBM",
        "config": {"workload": f"{args.workload}-shaped MoE layer, bf16 experts, decode {dT} "
                               f"tokens", "experts": E, "top_k": K, "hidden": H,
                   "intermediate": I, "weights": "bf16", "parallelism": "single GPU"},
        "decode": {"ms_per_step": dms, "experts_touched": touched, "expert_bytes": dbytes,
                   "GBps": dbytes / (dms * 1e-3) / 1e9,
                   "frac_hbm": dbytes / (dms * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "prefill": {"tokens": pT, "ms_per_step": pms, "tokens_per_s": pT / (pms * 1e-3),
                    "kernel_ms": med, "gate_up_TFLOPs": gu_tf, "down_TFLOPs": dn_tf,
                    "gate_up_frac_bf16_peak": gu_tf / BF16_PEAK_TFLOPS,
                    "expert_bytes": E * 3 * H * I * 2,
                    "frac_hbm": E * 3 * H * I * 2 / (pms * 1e-3) / 1e9 / HBM_PEAK_GBS},
    }
    print(json.dumps(out))


def _ev():
    import torch

    return torch.cuda.Event(enable_timing=True)


def settle(step_fn, seconds):
    """Untimed steps for ``seconds`` of wall time (the GPU leaves its idle clocks within a
    few hundred milliseconds of sustained work); returns the steps run."""
    import torch

    n, end = 0, time.perf_counter() + seconds
    while time.perf_counter() < end:
        for _ in range(8):
            n += step_fn(n)
        torch.cuda.synchronize()
    return n


def time_decode(layers, xs, touched, wl_shape, steps, warmup, settle_s, graph=True,
                kernel_steps=100):
    """Decode steps over the rotated layers: per-kernel durations from an eager pass with
    the library's stage events, then ``steps`` timed steps replayed from a HIP graph of up
    to 40 consecutive steps (``steps`` rounded down to a multiple of the graph's length;
    the JSON reports the count timed).  Returns the decode dict."""
    import torch

    E, K, H, I, limit, biases = wl_shape
    L = len(layers)
    dT = xs[0].shape[0]
    for s in range(warmup):
        layers[s % L].decode(xs[s % L])
    torch.cuda.synchronize()

    def eager_step(n):
        layers[n % L].decode(xs[n % L])
        return 1

    settled = settle(eager_step, settle_s)
    # Per-kernel durations: an eager pass with the library's stage events on the launch
    # stream (events recorded inside a captured graph do not time its kernels).
    n_ev = kernel_steps
    stage = [[_ev() for _ in range(6)] for _ in range(n_ev)]
    e0, e1 = _ev(), _ev()
    e0.record()
    for s in range(n_ev):
        layers[s % L].decode(xs[s % L], stage_events=stage[s])
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / n_ev

    mode = "eager"
    if graph:
        # One graph holds G consecutive steps over the rotated layers (a layer recurs at
        # least 4 steps later, across replays).
        G = min(steps, 40)
        reps = max(1, steps // G)
        steps = G * reps
        try:
            g = torch.cuda.CUDAGraph()
            cap_stream = torch.cuda.Stream()
            cap_stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(cap_stream):
                with torch.cuda.graph(g, stream=cap_stream):
                    for s in range(G):
                        layers[s % L].decode(xs[s % L])
            torch.cuda.current_stream().wait_stream(cap_stream)
            g.replay()
            torch.cuda.synchronize()
            mode = "hip-graph"
        except Exception as exc:  # capture unsupported: time eagerly
            print(f"graph capture failed ({exc}); timing eagerly", file=sys.stderr)
            torch.cuda.synchronize()
    if mode == "hip-graph":
        settled += settle(lambda n: (g.replay(), G)[1], settle_s)
    else:
        settled += settle(eager_step, settle_s)
    t0, t1 = _ev(), _ev()
    t0.record()
    if mode == "hip-graph":
        for _ in range(reps):
            g.replay()
    else:
        for s in range(steps):
            layers[s % L].decode(xs[s % L])
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps

    def stage_ms(a, b):
        return sum(stage[s][a].elapsed_time(stage[s][b]) for s in range(n_ev)) / n_ev

    avg_touched = sum(touched[s % L] for s in range(steps)) / steps
    layer_bytes = avg_touched * bytes_per_expert(H, I, biases) + E * H * 2 + 2 * dT * H * 2
    ev_touched = sum(touched[s % L] for s in range(n_ev)) / n_ev
    gu_bytes = ev_touched * gate_up_bytes_per_expert(H, I, biases) + dT * H * 2
    return {
        "tokens_per_s": dT / (ms * 1e-3), "ms_per_step": ms, "steps": steps,
        "experts_touched_avg": avg_touched,
        "layer_algorithmic_bytes": layer_bytes,
        "layer_GBps": layer_bytes / (ms * 1e-3) / 1e9,
        "layer_frac_hbm": layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "kernel_ms": {"router": stage_ms(0, 1), "route": stage_ms(1, 2),
                      "gate_up": stage_ms(2, 3), "down": stage_ms(3, 4),
                      "combine": stage_ms(4, 5)},
        "gate_up_algorithmic_bytes": gu_bytes,
        "launch": mode, "eager_ms_per_step": eager_ms, "kernel_timing_steps": n_ev,
        "settle_steps": settled, "settle_s": 2 * settle_s,
    }


def time_prefill(layers, xps, wl_shape, steps, settle_s, warmup=3):
    """Prefill steps over the rotated layers (eager launches): per-kernel durations from a
    pass with the library's stage events, then ``steps`` timed steps that record none.
    Returns the prefill dict."""
    import torch

    E, K, H, I, limit, biases = wl_shape
    L = len(layers)
    pT = xps[0].shape[0]
    for s in range(warmup):
        layers[s % L].prefill(xps[s % L])
    torch.cuda.synchronize()
    p_settled = settle(lambda n: (layers[n % L].prefill(xps[n % L]), 1)[1], settle_s)
    # Each event recorded between two kernels of the step delays the next one by a few
    # microseconds, so the timed region below records none.
    pst = [[_ev() for _ in range(5)] for _ in range(steps)]
    for s in range(steps):
        layers[s % L].prefill(xps[s % L], stage_events=pst[s])
    torch.cuda.synchronize()

    def stage_ms(i):
        return sum(pst[s][i].elapsed_time(pst[s][i + 1]) for s in range(steps)) / steps

    fe_ms, gu_ms, dn_ms, cb_ms = stage_ms(0), stage_ms(1), stage_ms(2), stage_ms(3)
    p0, p1 = _ev(), _ev()
    p0.record()
    for s in range(steps):
        layers[s % L].prefill(xps[s % L])
    p1.record()
    torch.cuda.synchronize()
    pms = p0.elapsed_time(p1) / steps
    pairs = pT * K
    flops = 6 * H * I * pairs + 2 * pT * H * E
    gu_flops = 4 * H * I * pairs
    pbytes = E * bytes_per_expert(H, I, biases) + E * H * 2 + 2 * pT * H * 2
    gu_tf = gu_flops / (gu_ms * 1e-3) / 1e12
    t_min = max(pbytes / (HBM_PEAK_GBS * 1e9), flops / (MXFP4_PEAK_TFLOPS * 1e12))
    return {
        "value": pT / (pms * 1e-3), "unit": "tokens/s", "ms_per_step": pms, "tokens": pT,
        "steps": steps, "settle_steps": p_settled, "algorithmic_flops": flops,
        "algorithmic_bytes": pbytes,
        "layer_TFLOPs": flops / (pms * 1e-3) / 1e12,
        "layer_frac_mxfp4_peak": flops / (pms * 1e-3) / 1e12 / MXFP4_PEAK_TFLOPS,
        "layer_frac_bf16_peak": flops / (pms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
        "layer_frac_binding_roofline": t_min / (pms * 1e-3),
        "binding_roofline": "hbm" if pbytes / (HBM_PEAK_GBS * 1e9) >= flops / (
            MXFP4_PEAK_TFLOPS * 1e12) else "mxfp4 mfma",
        "kernel_ms": {"router+mapping": fe_ms, "gate_up": gu_ms, "down": dn_ms,
                      "combine": cb_ms},
        "launch_gaps_ms": pms - fe_ms - gu_ms - dn_ms - cb_ms,
        "gate_up_TFLOPs": gu_tf, "gate_up_frac_bf16_peak": gu_tf / BF16_PEAK_TFLOPS,
        "gate_up_algorithmic_flops": gu_flops,
    }


def build_workload(wl, n_layers, dev, gen, zipf=None):
    E, K, H, I, limit, biases, _, _ = WORKLOADS[wl]
    return [make_layer(E, K, H, I, limit, biases, dev, gen, zipf) for _ in range(n_layers)]


def experts_touched(layers, xs):
    import torch

    out = []
    for lay, x in zip(layers, xs):
        _, _, idx, _ = lay.route(x)
        out.append(int(torch.unique(idx).numel()))
    torch.cuda.synchronize()
    return out


def time_linear(dev, gen, settle_s, n_w=64, calls=256):
    """The single MXFP4 weight-only linear: W [5760 x 2880] (codes uniform, exponents
    uniform in [120, 130]), x bf16 [128 x 2880], fp32 accumulate, bf16 out.  ``n_w``
    distinct weight matrices are rotated (560 MB, so no call finds its weights in the
    256 MB last-level cache); the calls are replayed from a HIP graph."""
    import torch

    from vllm_neuron_amd.functional.mxfp4 import mxfp4_linear

    N, K, M = 5760, 2880, 128
    ws = [(torch.randint(0, 256, (N // 16, 8 * K), dtype=torch.uint8, device=dev, generator=gen),
           torch.randint(120, 131, ((N + 63) // 64, 2 * K), dtype=torch.uint8, device=dev,
                         generator=gen)) for _ in range(n_w)]
    x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
    for q, sc in ws[:4]:
        mxfp4_linear(x, q, sc)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        with torch.cuda.graph(g, stream=cap):
            for i in range(calls):
                q, sc = ws[i % n_w]
                mxfp4_linear(x, q, sc)
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    settle(lambda n: (g.replay(), calls)[1], settle_s)
    t0, t1 = _ev(), _ev()
    t0.record()
    for _ in range(4):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    us = t0.elapsed_time(t1) * 1e3 / (4 * calls)
    nbytes = N * K // 2 + N * K // 32 + M * K * 2 + M * N * 2
    flops = 2 * M * N * K
    t_min = max(nbytes / (HBM_PEAK_GBS * 1e9), flops / (MXFP4_PEAK_TFLOPS * 1e12))
    return {"workload": "MXFP4 linear W 5760x2880, x 128x2880", "us_per_call": us,
            "tokens_per_s": M / (us * 1e-6), "algorithmic_bytes": nbytes,
            "algorithmic_flops": flops, "GBps": nbytes / (us * 1e-6) / 1e9,
            "TFLOPs": flops / (us * 1e-6) / 1e12, "binding_roofline": "hbm",
            "frac_binding_roofline": t_min / (us * 1e-6), "launch": "hip-graph",
            "calls": 4 * calls}


def other_configs(dev, gen, settle_s):
    """The other workloads of the benchmark, each timed once (hip-graph decode over 200
    steps after the same settling as the headline, eager prefill), with its
    binding-roofline fraction: the MXFP4 linear; the GPT-OSS-20B-shaped
    layer at decode (1, 4, 16, 64 tokens) and at prefill (4,096 tokens, uniform and
    Zipf(1.2) routing); the 256-expert top-8 layer with Zipf(1.0) routing at decode (128
    tokens) and prefill (8,192 tokens).  Each workload rotates over 8 layers."""
    import torch

    res = {"linear": time_linear(dev, gen, settle_s)}
    for wl, zipfs, dts in (("gptoss20b", (None, 1.2), (1, 4, 16, 64)), ("fine256", (1.0,), (128,))):
        E, K, H, I, limit, biases, _, pT = WORKLOADS[wl]
        shape = (E, K, H, I, limit, biases)
        for zipf in zipfs:
            layers = build_workload(wl, 8, dev, gen, zipf)
            tag = wl + ("" if zipf is None else f"_zipf{zipf:g}")
            if wl == "fine256" or zipf is None:
                for dT in dts:
                    xs = [torch.randn(dT, H, device=dev, generator=gen).to(torch.bfloat16)
                          for _ in range(8)]
                    d = time_decode(layers, xs, experts_touched(layers, xs), shape, 200, 10,
                                    settle_s, kernel_steps=16)
                    res[f"{tag}_decode_T{dT}"] = {
                        "tokens_per_s": d["tokens_per_s"], "ms_per_step": d["ms_per_step"],
                        "experts_touched_avg": d["experts_touched_avg"],
                        "binding_roofline": "hbm", "frac_binding_roofline": d["layer_frac_hbm"],
                        "GBps": d["layer_GBps"], "kernel_ms": d["kernel_ms"],
                        "launch": d["launch"]}
            xps = [torch.randn(pT, H, device=dev, generator=gen).to(torch.bfloat16)
                   for _ in range(8)]
            p = time_prefill(layers, xps, shape, 8, settle_s)
            res[f"{tag}_prefill_T{pT}"] = {
                k: p[k] for k in ("value", "ms_per_step", "layer_TFLOPs", "binding_roofline",
                                  "layer_frac_binding_roofline", "layer_frac_mxfp4_peak",
                                  "layer_frac_bf16_peak", "gate_up_frac_bf16_peak",
                                  "kernel_ms")}
            del layers, xps
            torch.cuda.empty_cache()
    return res


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "multi-GPU expert parallelism is not built in this tier.", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration()
        return
    if args.weights == "bf16":
        bench_bf16(args)
        return

    import torch

    dev = torch.device("cuda:0")
    E, K, H, I, limit, biases, dT, pT = WORKLOADS[args.workload]
    shape = (E, K, H, I, limit, biases)
    dT = args.decode_tokens or dT
    pT = args.prefill_tokens or pT
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    n_layers = args.layers or (36 if args.workload == "gptoss120b" else 8)
    layers = build_workload(args.workload, n_layers, dev, gen, args.zipf)
    L = len(layers)
    xs = [torch.randn(dT, H, device=dev, generator=gen).to(torch.bfloat16) for _ in range(L)]
    torch.cuda.synchronize()
    touched = experts_touched(layers, xs)  # from the actual routing

    # ---------------- decode (the headline)
    decode = time_decode(layers, xs, touched, shape, args.steps, args.warmup, args.settle,
                         graph=not args.no_graph)
    steps, ms = decode["steps"], decode["ms_per_step"]
    gu_ms = decode["kernel_ms"]["gate_up"]
    gu_bytes = decode.pop("gate_up_algorithmic_bytes")
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    traffic, traffic_pre, traffic_src = measured_traffic(args.workload, dT, pT)
    roofline = {"bound": "hbm", "kernel": "tkg_stream_kernel<4, 1, true, 2, 4> (gate_up)",
                "achieved": gu_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": gu_gbs / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": traffic_src,
                "algorithmic_bytes_per_launch": gu_bytes, "avg_launch_ms": gu_ms}

    # ---------------- prefill
    prefill = None
    if not args.skip_prefill:
        xp = [torch.randn(pT, H, device=dev, generator=gen).to(torch.bfloat16) for _ in range(L)]
        prefill = time_prefill(layers, xp, shape, args.prefill_steps, args.settle)
        gu_ms_p = prefill["kernel_ms"]["gate_up"]
        gu_flops = prefill.pop("gate_up_algorithmic_flops")
        gu_tf = prefill["gate_up_TFLOPs"]
        prefill["roofline"] = {"bound": "mfma", "kernel": "prefill_gemm_kernel<gate_up>",
                               "achieved": gu_tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                               "frac": gu_tf / BF16_PEAK_TFLOPS,
                               "frac_of_mxfp4_peak": gu_tf / MXFP4_PEAK_TFLOPS,
                               "traffic": traffic_pre, "traffic_source": traffic_src,
                               "algorithmic_flops_per_launch": gu_flops, "avg_launch_ms": gu_ms_p}
        del xp
    del layers, xs
    torch.cuda.empty_cache()

    others = None
    if not args.no_other_configs and args.workload == "gptoss120b":
        others = other_configs(dev, gen, args.settle)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.workload, dT, pT)
        if prefill is not None:
            prefill["cpu_baseline"] = cpu["prefill"]

    out = {
        "metric": "MXFP4 MoE layer tokens/s @1 GPU; decode HBM GB/s %; prefill MFMA util %",
        "value": decode["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random MXFP4 weights, N(0,1) tokens), weights resident in HBM",
        "config": {"workload": f"{args.workload}-shaped MoE layer decode, {dT} tokens",
                   "experts": E, "top_k": K, "hidden": H, "intermediate": I,
                   "decode_tokens": dT, "prefill_tokens": pT, "layers_rotated": L,
                   "routing": "uniform" if not args.zipf else f"zipf s={args.zipf}",
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": None if cpu is None else cpu["decode"],
        "decode": decode,
        "prefill": prefill,
        "other_configs": others,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
