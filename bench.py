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
work, and a short timed region otherwise measures the clock ramp.  The timed region is
exactly the requested steps.

``--weights bf16`` times the bf16-expert path instead (the reference's shard_on_block
operands; moe_cte prefill and moe_block_tkg decode) and prints a line of its own.

``cpu_baseline`` times the CPU oracle (a port of the reference's CPU flow: dense
all-expert fp32 decode, dense all-expert bf16 prefill) on the host cores over a
bounded sample of experts / tokens and scales linearly to the full workload.
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


def cpu_baseline(wl, decode_T, prefill_T):
    """Time the CPU oracle on a bounded sample; returns dicts for decode and prefill."""
    import torch

    import pkgload

    pkgload.load()
    from vllm_neuron_amd import synthetic

    from oracle.layer import RefLayer

    E, K, H, I, limit, biases, _, _ = WORKLOADS[wl]
    # The process's affinity cores, at most 16: the host share one GPU's jobs get on a
    # node of 8 GPUs, whatever the affinity mask shows.
    affinity = len(os.sched_getaffinity(0))
    cores = min(affinity, 16)
    torch.set_num_threads(cores)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")),
                         "unknown")
    except OSError:
        pass
    e_s = min(E, 16)
    shape = synthetic.MoEShape(wl + "-sample", E, min(K, e_s), H, I, limit, biases)
    ref = RefLayer(synthetic.layer_tensors(shape, 5, E=e_s))

    def timed(fn, budget_s):
        fn()  # warm-up
        ts = []
        while len(ts) < 3 or sum(ts) < budget_s:
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[len(ts) // 2], len(ts)

    res = {}
    x = synthetic.tokens(5, decode_T, H)
    t, n = timed(lambda: ref.decode(x), 8.0)
    t *= E / e_s
    res["decode"] = {"value": decode_T / t, "unit": "tokens/s", "cores": cores, "kind": "port",
                     "cpu": model, "affinity_cores": affinity,
                     "sample": f"dense all-expert fp32 decode (reference moe_block_tkg CPU flow) "
                               f"of {decode_T} tokens over {e_s} of {E} experts, median of {n} "
                               f"reps (about 8 s), time scaled x{E / e_s:g} (linear in experts)"}
    t_s = min(prefill_T, 512)
    xp = synthetic.tokens(6, t_s, H)
    t, n = timed(lambda: ref.prefill(xp), 8.0)
    t *= (E / e_s) * (prefill_T / t_s)
    res["prefill"] = {"value": prefill_T / t, "unit": "tokens/s", "cores": cores, "kind": "port",
                      "cpu": model, "affinity_cores": affinity,
                      "sample": f"dense all-expert bf16 prefill (reference _torch_moe_impl CPU "
                                f"flow) of {t_s} tokens over {e_s} of {E} experts, median of {n} "
                                f"reps (about 8 s), time scaled x{E / e_s:g} (experts) "
                                f"x{prefill_T / t_s:g} (tokens)"}
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
    dT = args.decode_tokens or dT
    pT = args.prefill_tokens or pT
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    n_layers = args.layers or (36 if args.workload == "gptoss120b" else 8)
    layers = [make_layer(E, K, H, I, limit, biases, dev, gen, args.zipf) for _ in range(n_layers)]
    L = len(layers)
    xs = [torch.randn(dT, H, device=dev, generator=gen).to(torch.bfloat16) for _ in range(L)]
    torch.cuda.synchronize()

    # experts touched by each (layer, batch) pair, from the actual routing
    touched = []
    for lay, x in zip(layers, xs):
        _, _, idx, _ = lay.route(x)
        touched.append(int(torch.unique(idx).numel()))
    torch.cuda.synchronize()

    def ev():
        return torch.cuda.Event(enable_timing=True)

    def settle(step_fn, seconds):
        """Untimed steps for ``seconds`` of wall time (the GPU leaves its idle clocks within
        a few hundred milliseconds of sustained work); returns the steps run."""
        n, end = 0, time.perf_counter() + seconds
        while time.perf_counter() < end:
            for _ in range(8):
                n += step_fn(n)
            torch.cuda.synchronize()
        return n

    def eager_step(n):
        layers[n % L].decode(xs[n % L])
        return 1

    # ---------------- decode
    for s in range(args.warmup):
        layers[s % L].decode(xs[s % L])
    torch.cuda.synchronize()
    settled = settle(eager_step, args.settle)

    # Per-kernel durations: an eager pass with the library's stage events on the launch
    # stream (events recorded inside a captured graph do not time its kernels).
    n_ev = 100
    stage = [[ev() for _ in range(6)] for _ in range(n_ev)]
    e0, e1 = ev(), ev()
    e0.record()
    for s in range(n_ev):
        layers[s % L].decode(xs[s % L], stage_events=stage[s])
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / n_ev

    steps = args.steps
    mode = "eager"
    if not args.no_graph:
        # One graph holds G consecutive steps over the rotated layers (a layer recurs at
        # least 4 steps later, across replays); the timed region replays it, so ``steps``
        # is rounded to a multiple of G.
        G = min(steps, 40)
        reps = max(1, steps // G)
        steps = G * reps
        try:
            graph = torch.cuda.CUDAGraph()
            cap_stream = torch.cuda.Stream()
            cap_stream.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(cap_stream):
                with torch.cuda.graph(graph, stream=cap_stream):
                    for s in range(G):
                        layers[s % L].decode(xs[s % L])
            torch.cuda.current_stream().wait_stream(cap_stream)
            graph.replay()
            torch.cuda.synchronize()
            mode = "hip-graph"
        except Exception as exc:  # capture unsupported: time eagerly
            print(f"graph capture failed ({exc}); timing eagerly", file=sys.stderr)
            torch.cuda.synchronize()
    if mode == "hip-graph":
        settled += settle(lambda n: (graph.replay(), G)[1], args.settle)
    else:
        settled += settle(eager_step, args.settle)
    t0, t1 = ev(), ev()
    if mode == "hip-graph":
        t0.record()
        for _ in range(reps):
            graph.replay()
        t1.record()
    else:
        t0.record()
        for s in range(steps):
            layers[s % L].decode(xs[s % L])
        t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps

    def stage_ms(a, b):
        return sum(stage[s][a].elapsed_time(stage[s][b]) for s in range(n_ev)) / n_ev

    rt_ms, route_ms, gu_ms = stage_ms(0, 1), stage_ms(1, 2), stage_ms(2, 3)
    dn_ms, cb_ms = stage_ms(3, 4), stage_ms(4, 5)
    avg_touched = sum(touched[s % L] for s in range(steps)) / steps
    bpe = bytes_per_expert(H, I, biases)
    layer_bytes = avg_touched * bpe + E * H * 2 + 2 * dT * H * 2
    # the roofline kernel's duration comes from the eager pass over n_ev steps
    ev_touched = sum(touched[s % L] for s in range(n_ev)) / n_ev
    gu_bytes = ev_touched * gate_up_bytes_per_expert(H, I, biases) + dT * H * 2
    decode = {
        "tokens_per_s": dT / (ms * 1e-3), "ms_per_step": ms,
        "experts_touched_avg": avg_touched,
        "layer_algorithmic_bytes": layer_bytes,
        "layer_GBps": layer_bytes / (ms * 1e-3) / 1e9,
        "layer_frac_hbm": layer_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "kernel_ms": {"router": rt_ms, "route": route_ms, "gate_up": gu_ms, "down": dn_ms,
                      "combine": cb_ms},
        "launch": mode, "eager_ms_per_step": eager_ms, "kernel_timing_steps": n_ev,
        "settle_steps": settled, "settle_s": 2 * args.settle,
    }
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
        for s in range(3):
            layers[s % L].prefill(xp[s % L])
        torch.cuda.synchronize()
        p_settled = settle(lambda n: (layers[n % L].prefill(xp[n % L]), 1)[1], args.settle)
        ps = args.prefill_steps
        # Per-kernel durations from a pass with the library's stage events; the timed
        # region below records none (each event recorded between two kernels of the step
        # delays the next one by a few microseconds).
        pst = [[ev() for _ in range(4)] for _ in range(ps)]
        for s in range(ps):
            layers[s % L].prefill(xp[s % L], stage_events=pst[s])
        torch.cuda.synchronize()
        gu_ms_p = sum(pst[s][0].elapsed_time(pst[s][1]) for s in range(ps)) / ps
        dn_ms_p = sum(pst[s][1].elapsed_time(pst[s][2]) for s in range(ps)) / ps
        cb_ms_p = sum(pst[s][2].elapsed_time(pst[s][3]) for s in range(ps)) / ps
        p0, p1 = ev(), ev()
        p0.record()
        for s in range(ps):
            layers[s % L].prefill(xp[s % L])
        p1.record()
        torch.cuda.synchronize()
        pms = p0.elapsed_time(p1) / ps
        pairs = pT * K
        flops = 6 * H * I * pairs + 2 * pT * H * E
        gu_flops = 4 * H * I * pairs
        pbytes = E * bpe + E * H * 2 + 2 * pT * H * 2
        gu_tf = gu_flops / (gu_ms_p * 1e-3) / 1e12
        t_min = max(pbytes / (HBM_PEAK_GBS * 1e9), flops / (MXFP4_PEAK_TFLOPS * 1e12))
        prefill = {
            "value": pT / (pms * 1e-3), "unit": "tokens/s", "ms_per_step": pms, "tokens": pT,
            "steps": ps, "settle_steps": p_settled, "algorithmic_flops": flops,
            "algorithmic_bytes": pbytes,
            "layer_TFLOPs": flops / (pms * 1e-3) / 1e12,
            "layer_frac_mxfp4_peak": flops / (pms * 1e-3) / 1e12 / MXFP4_PEAK_TFLOPS,
            "layer_frac_binding_roofline": t_min / (pms * 1e-3),
            "kernel_ms": {"gate_up": gu_ms_p, "down": dn_ms_p, "combine": cb_ms_p,
                          "router+mapping": pms - gu_ms_p - dn_ms_p - cb_ms_p},
            "roofline": {"bound": "mfma", "kernel": "prefill_gemm_kernel<gate_up>",
                         "achieved": gu_tf, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": gu_tf / BF16_PEAK_TFLOPS,
                         "frac_of_mxfp4_peak": gu_tf / MXFP4_PEAK_TFLOPS,
                         "traffic": traffic_pre, "traffic_source": traffic_src,
                         "algorithmic_flops_per_launch": gu_flops, "avg_launch_ms": gu_ms_p},
        }

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
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
