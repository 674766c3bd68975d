"""Benchmark: MoE route -> dispatch -> combine on one MI355X.

A step is one pass of the whole path over one batch of synthetic input that
is already resident in HBM: router GEMM + scoring/top-k + histogram
(moe_route), stable permutation + gather (moe_permute), weighted combine
(moe_combine).  Default workload: the DeepSeek-V3 shape (C4: T=32768,
H=7168, E=256, top-8, sigmoid + bias, 8 groups keep 4, x2.5).

Prints ONE JSON line: routed tokens/s, ms/step, the roofline of the dominant
kernel (algorithmic bytes / HIP-event-timed launch duration vs 8 TB/s),
per-stage times, the end-to-end HBM fraction, and the CPU oracle's rate on a
bounded sample of the same workload (rank 0, N=1).

    python bench.py [--steps K] [--warmup W] [--config C4|C5|C2|C3] [--no-cpu]
    python bench.py --layer [T ...] [--layer-int8]   # the drop-in run() at the reference's workloads

--layer times the reference entry point run() (route, dispatch, SwiGLU
experts and shared expert on the grouped GEMM, combine) at the reference's
own workload shapes (NE=64, H=8192, Ni=3584, SNi=7168, top-8; T from its
9-workload mix, kernel.cu:133-136) and prints ONE JSON line with per-T
latency and the mix-weighted sum the reference quotes (35.92 ms on B200,
kernel.cu:146-151).
"""
import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [REPO, os.path.join(REPO, "ernie-evolve-results_amd")]

import numpy as np  # noqa: E402
import torch  # noqa: E402

import moe_route as M  # noqa: E402
from moe_route.configs import CONFIGS  # noqa: E402

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def algorithmic_bytes(c):
    """Bytes each stage must move at minimum (x read by the router and again
    by the permute; each routed row written once and read once)."""
    T, H, E, k = c.T, c.H, c.E, c.k
    xb = 2
    wb = 4 if c.x_dtype == torch.float32 else 2  # an fp32 router weight is read whole
    db = 1 if c.fp8 else 2
    route = T * H * xb + E * H * wb + T * E * 4 + T * k * 8
    gather = T * H * xb + T * k * H * db + (T * k * (H // 128) * 4 if c.fp8 else 0) + T * k * 8
    combine = T * k * H * 2 + T * H * 2 + T * k * 8
    return dict(route=route, gather=gather, combine=combine)


TRAFFIC_FILES = {"C4": "c4_hbm_traffic.md", "C5": "c5_fp8_dispatch_hbm_traffic.md"}


def measured_traffic(config):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    (copy-calibrated), read from the committed summary of this workload:
    lines `traffic <kernel> <bytes>` of profiles/<file>."""
    out = {}
    if config not in TRAFFIC_FILES:
        return out
    try:
        with open(os.path.join(REPO, "profiles", TRAFFIC_FILES[config])) as f:
            for line in f:
                p = line.split()
                if len(p) == 3 and p[0] == "traffic":
                    out[p[1]] = float(p[2])
    except OSError:
        pass
    return out


def cpu_baseline(c, sample_T, threads=0):
    """The CPU oracle (oracle/moe_oracle.py) on `sample_T` tokens of the same
    workload: router GEMM (torch fp32), scoring/top-k, permutation, gather /
    fp8 quantisation and combine.  1 warm-up + median of 3."""
    from oracle import moe_oracle as O
    ncores = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    sample_T = min(sample_T, c.T)
    x, w, bias, y = M.make_inputs(c, T=sample_T, seed=0)
    cfg = O.RouteCfg(c.cfg.scoring, c.cfg.renormalize, c.cfg.n_group, c.cfg.topk_group,
                     c.cfg.route_scale, c.cfg.norm_min)
    b = None if bias is None else bias.numpy()

    def once():
        """The oracle's route_dispatch_combine, stage by stage: seconds per stage."""
        t = [time.perf_counter()]
        r = O.route(x, w, b, c.k, cfg)
        t.append(time.perf_counter())
        row_token, pair_row = O.permutation(r["ids"])
        if c.fp8:
            O.permute_fp8(x, row_token)
            xg = None
        else:
            xg = O.gather_rows(x, row_token)
        t.append(time.perf_counter())
        O.combine(xg if y is None else y, pair_row, r["weights"])  # y None: identity experts
        t.append(time.perf_counter())
        return [t[i + 1] - t[i] for i in range(3)]

    once()
    runs = [once() for _ in range(3)]
    med = statistics.median(sum(r) for r in runs)
    stages = {n: round(statistics.median(r[i] for r in runs), 4)
              for i, n in enumerate(("route", "permute", "combine"))}
    return {"value": sample_T / med, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port", "stages_s": stages,
            "sample": "%d tokens of %s (T,H,E,k = %d,%d,%d,%d), oracle route+permute+combine, "
                      "median of 3 = %.3f s" % (sample_T, c.name, sample_T, c.H, c.E, c.k, med)}


LAYER_MIX = {1571: 1, 2048: 1, 4096: 3, 4904: 1, 8192: 3}  # kernel.cu:133-136


def layer_bench(Ts, steps, warmup, dispatch="bf16", experts="bf16", cold=True):
    """run() latency per T (HIP events around each call, median of `steps`).
    cold: before each timed call a 1 GiB buffer is rewritten, evicting L2 and
    the 256 MB MALL, as the reference's harness times each call with a cold
    L2 (kernel.cu:146-151)."""
    dev = torch.device("cuda:0")
    H, E, Ni, SNi = 8192, 64, 3584, 7168
    g = torch.Generator(device=dev).manual_seed(0)
    r = lambda *sh: torch.randn(*sh, generator=g, device=dev)
    gw = r(E, H) / H ** 0.5
    bias = r(E)
    eg = (r(E, Ni, H) / H ** 0.5).to(torch.bfloat16)
    eu = (r(E, Ni, H) / H ** 0.5).to(torch.bfloat16)
    ed = (r(E, H, Ni) / Ni ** 0.5).to(torch.bfloat16)
    sg = (r(SNi, H) / H ** 0.5).to(torch.bfloat16)
    su = (r(SNi, H) / H ** 0.5).to(torch.bfloat16)
    sd = (r(H, SNi) / SNi ** 0.5).to(torch.bfloat16)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev) if cold else None
    ms = {}
    for T in Ts:
        hs = r(1, T, H).to(torch.bfloat16)
        args = (hs, gw, bias, eg, eu, ed, sg, su, sd, 1e-6)
        run = lambda: M.run(*args, dispatch=dispatch, experts=experts)
        for _ in range(warmup):
            run()
        torch.cuda.synchronize()
        ts = []
        for _ in range(steps):
            if flush is not None:
                flush.fill_(1)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            run()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b))
        ms[T] = statistics.median(ts)
        print("layer T=%d: %.3f ms" % (T, ms[T]), file=sys.stderr, flush=True)
    line = {
        "metric": "reference run() layer latency (route+dispatch+SwiGLU experts+shared+combine)",
        "value": round(sum(LAYER_MIX.get(T, 1) * ms[T] for T in Ts), 4), "unit": "ms",
        "n_gpus": 1, "steps": steps, "warmup": warmup, "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 experts, bf16 shared expert" if experts == "int8" else "bf16",
        "data": "synthetic (seeded randn, the reference harness's distributions)",
        "config": {"workload": "kernel.cu run(): NE=64 H=8192 Ni=3584 SNi=7168 top-8; value = "
                               "sum over T of mix weight x latency",
                   "dispatch": dispatch, "experts": experts,
                   "cache": "cold (1 GiB rewritten before each timed call)" if cold else "warm",
                   "mix": {str(T): LAYER_MIX.get(T, 1) for T in Ts}},
        "per_T_ms": {str(T): round(v, 4) for T, v in ms.items()},
        "reference_b200_mix_sum_ms": 35.92,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C4")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=0,
                    help="tokens of the CPU baseline sample (0: the whole configuration)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads for the CPU baseline (0: every core of this process)")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run one plain 1 GiB device copy (untimed), the known-size "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE scaling")
    ap.add_argument("--layer", nargs="*", type=int, default=None,
                    help="time run() at the reference's workload T values (default: its mix)")
    ap.add_argument("--layer-fp8", action="store_true",
                    help="with --layer: run(..., dispatch='fp8')")
    ap.add_argument("--layer-warm", action="store_true",
                    help="with --layer: no cache flush between the timed calls")
    ap.add_argument("--layer-int8", action="store_true",
                    help="with --layer: run(..., experts='int8'), the reference's expert precision")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this path runs on one GPU only (no sharding, no collectives); "
              "--gpus %d is not supported" % args.gpus, file=sys.stderr)
        sys.exit(2)

    if args.layer is not None:
        layer_bench(args.layer or sorted(LAYER_MIX), max(args.steps // 2, 5), 2,
                    "fp8" if args.layer_fp8 else "bf16", "int8" if args.layer_int8 else "bf16",
                    cold=not args.layer_warm)
        return

    c = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    x, w, bias, y = M.make_inputs(c, seed=0, device=dev)
    # The router takes bf16 hidden states (K:4327-4339); an fp32 config (C1)
    # hands the GPU path bf16(x), cast once here, and keeps its fp32 router
    # weight, which moe_route splits into bf16 hi/lo on the device.
    x = x.to(torch.bfloat16)
    plan = M.MoePlan(c.T, c.H, c.E, c.k, c.cfg, dev, fp8=c.fp8, w_dtype=w.dtype)
    torch.cuda.synchronize()

    for _ in range(args.warmup):
        plan.step(x, w, bias, y)
    torch.cuda.synchronize()
    if args.copy_calib:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- timed region: exactly K steps, whole path, inputs resident in HBM.
    # Each step runs cold: before it, a 1 GiB buffer is rewritten (outside the
    # step's HIP events), evicting L2 and the 256 MB MALL, so no step finds the
    # previous one's data in the caches.  ms_per_step = the median of the K
    # event-timed steps.
    ev = lambda: torch.cuda.Event(enable_timing=True)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    evs = [(ev(), ev()) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in evs:
        flush.fill_(1)
        e0.record()
        plan.step(x, w, bias, y)
        e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    cold = [e0.elapsed_time(e1) for e0, e1 in evs]
    ms_per_step = statistics.median(cold)
    del flush

    # ---- the same K steps back to back (no rewrite between them): wall clock
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        plan.step(x, w, bias, y)
    torch.cuda.synchronize()
    warm_ms = (time.perf_counter() - t1) * 1e3 / args.steps

    # ---- per-stage HIP-event timing (on the stream the kernels run on).
    # permute = index kernels + the gather launch; an index-only permute (no
    # rows) isolates the gather.  route = the router GEMM and the scoring (one
    # fused kernel at the DeepSeek-V3 shape, plus its weight re-layout pass).
    st = {"route": [], "permute": [], "permute_index": [], "combine": []}
    for _ in range(args.steps):
        e = [ev() for _ in range(5)]
        e[0].record()
        plan.route(x, w, bias)
        e[1].record()
        plan.permute(x)
        e[2].record()
        plan.combine(y)
        e[3].record()
        plan.permute(x, index_only=True)
        e[4].record()
        torch.cuda.synchronize()
        st["route"].append(e[0].elapsed_time(e[1]) * 1e3)
        st["permute"].append(e[1].elapsed_time(e[2]) * 1e3)
        st["combine"].append(e[2].elapsed_time(e[3]) * 1e3)
        st["permute_index"].append(e[3].elapsed_time(e[4]) * 1e3)
    us = {k2: statistics.mean(v) for k2, v in st.items()}

    us["gather"] = us["permute"] - us["permute_index"]

    ab = algorithmic_bytes(c)
    traffic = measured_traffic(c.name)
    kern = {"combine": ("combine_wave_kernel", ab["combine"], us["combine"]),
            "gather": ("gather_fp8_kernel" if c.fp8 else "gather_kernel", ab["gather"],
                       us["gather"])}
    dom = max(kern, key=lambda n: kern[n][2])
    kname, kbytes, kus = kern[dom]
    gbs = kbytes / (kus * 1e-6) / 1e9
    tr = traffic.get(kname)
    roofline = {"kernel": kname, "bound": "hbm", "achieved": round(gbs, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                "traffic": tr, "algorithmic_bytes": kbytes, "avg_launch_us": round(kus, 2)}
    total_bytes = ab["route"] + ab["gather"] + ab["combine"]
    e2e_gbs = total_bytes / (ms_per_step * 1e-3) / 1e9
    flops = 2.0 * c.T * c.H * c.E
    # the router stage as a whole (GEMM + scoring): MFMA and HBM fractions
    route = {"us": round(us["route"], 2),
             "tflops": round(flops / (us["route"] * 1e-6) / 1e12, 1),
             "mfma_frac": round(flops / (us["route"] * 1e-6) / 1e12 / BF16_PEAK_TFLOPS, 4),
             "hbm_frac": round(ab["route"] / (us["route"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(c, args.cpu_tokens or c.T, args.cpu_threads)

    tok_s = c.T / (ms_per_step * 1e-3)
    line = {
        "metric": "routed tokens/sec + achieved HBM GB/s (% of peak) at DSV3 shape, 1 MI355X",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded randn inputs generated on the GPU)",
        "config": {"workload": "%s route+dispatch+combine: %s" % (c.name, c.description),
                   "T": c.T, "H": c.H, "E": c.E, "k": c.k, "fp8_dispatch": c.fp8,
                   "x": "bf16", "router_weight": str(w.dtype).replace("torch.", "")},
        "roofline": roofline,
        "e2e_hbm": {"algorithmic_bytes": total_bytes, "achieved": round(e2e_gbs, 1),
                    "unit": "GB/s", "frac": round(e2e_gbs / HBM_PEAK_GBS, 4)},
        "stages_us": {k2: round(v, 2) for k2, v in us.items()},
        "stage_hbm_frac": {
            "route": round(ab["route"] / (us["route"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "permute": round(ab["gather"] / (us["permute"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "gather": round(ab["gather"] / (us["gather"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "combine": round(ab["combine"] / (us["combine"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)},
        "route_mfma": route,
        "timing": {"protocol": "value and ms_per_step: median of the K steps, each timed with HIP "
                               "events after a 1 GiB rewrite (cold L2 and MALL)",
                   "cold_steps_ms": {"median": round(ms_per_step, 4), "min": round(min(cold), 4),
                                     "max": round(max(cold), 4)},
                   "timed_region_wall_s": round(wall, 4),
                   "back_to_back": {"ms_per_step": round(warm_ms, 4),
                                    "tokens_per_s": round(c.T / (warm_ms * 1e-3), 1),
                                    "note": "the same K steps with no rewrite between them "
                                            "(wall clock)"}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
