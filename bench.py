#!/usr/bin/env python3
"""Benchmark of the MiMo-V2.6-Flash MoE block on one MI355X.

Headline (`value`): MoE-layer decode throughput at 1 row on a MiMo-shaped layer (H=4096, E=256 experts all
resident, I=2048, top-8, MXFP4 group 32), in algorithmic GB/s: per step the bytes of the distinct experts
read (U x 13,369,344) plus the router weight (256 x 4096 x 2) plus the row in and out.  One step = one fused
MoE-layer decode (router -> top-8 -> grouping -> experts -> combine) on a freshly routed row; steps rotate over
`--layers` distinct resident layers so no step finds its experts in L2 / MALL.  The timed region is one replay
of a HIP graph holding exactly --steps steps, inputs resident in HBM.

Also reported (field "extra"): decode at 2, 4, 8 rows with controlled routing (consecutive rows share ~2.6
of 8 experts), prefill at 512 / 2048 tokens with Zipf(1.1) expert popularity and at 2048 tokens with every route
on 16 popular experts (the GEMMs' compute-bound tiles on their own), a 48-layer stack decode at 1 and 4 rows,
the MoE half of a decoder layer (post-attention RMSNorm + block + residual) against the block alone at 1 row and
2048 tokens, and the per-kernel durations measured with HIP events.  "cpu_baseline" times an fp32 PyTorch CPU
restatement of the one-row decode (oracle/cpu_decode.py) on every host thread, on a bounded sample of the same
workload.

    python bench.py [--gpus 1] [--steps 500] [--warmup 20]

HBM traffic of the dominant kernel (the "traffic" field of "roofline") comes from two rocprofv3 counter runs
of `python bench.py --traffic-run` (FETCH_SIZE, then WRITE_SIZE), reduced by `--traffic-parse` against a
plain elementwise copy of known size measured in the same runs; the result is committed under profiles/.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mimo-on-a-mac_amd"))
sys.path.insert(0, ROOT)

METRIC = "MoE-layer decode GB/s (% HBM peak) at 1–8 rows; prefill tokens/sec"
HBM_PEAK_GBS = 8000.0
MXFP4_PEAK_TFLOPS = 10100.0
FP8_PEAK_TFLOPS = 5000.0
H, I, E, K = 4096, 2048, 256, 8
ROUTER_BYTES = E * H * 2
GATEUP_BYTES_PER_EXPERT = 2 * (I * H // 2 + I * H // 32)      # 8,912,896
FLOPS_PER_ROUTE = 2 * (2 * I * H + H * I)                      # 50,331,648
PF_HOT_EXPERTS = 16          # concentrated prefill: every token's 8 experts among 16 (1,024 routes each at 2048)
HILO_CEILING_TFLOPS = 2500.0  # useful flops when each product takes two fp8 x fp4 MFMAs at the 5.0 PF fp8 peak
ISSUE_RATE_TFLOPS = 3310.0    # issued fp8 x fp4 MFMA flops at the rate a throughput probe measured (48.6 cycles)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=48, help="resident MoE layers (48 = the MiMo stack)")
    ap.add_argument("--no-extra", action="store_true", help="headline only")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic-run", action="store_true",
                    help="profiling payload: a 1 GiB calibration copy, 1-row decode steps over 8 layers, then "
                         "2048-token prefill layers")
    ap.add_argument("--traffic-parse", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="reduce two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of --traffic-run to "
                         "profiles/traffic.json")
    ap.add_argument("--mfma-parse", metavar="PMC_DIR",
                    help="summarise a rocprofv3 --pmc run of --traffic-run with SQ_INSTS_MFMA, "
                         "SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE, using the kernel durations of a "
                         "--kernel-trace run of the same payload (second argument)")
    ap.add_argument("--mfma-trace", metavar="TRACE_DIR", help="kernel-trace directory for --mfma-parse")
    ap.add_argument("--pipe-parse", nargs=2, metavar=("LDS_DIR", "WAIT_DIR"),
                    help="summarise two rocprofv3 --pmc runs of --traffic-run (LDS counters, then wave wait and "
                         "issue counters) for the prefill GEMMs")
    ap.add_argument("--trace-parse", metavar="TRACE_DIR",
                    help="summarise a rocprofv3 --kernel-trace run of this benchmark: a markdown table per kernel "
                         "and grid on stdout, and the headline kernel's average duration (and its interval from "
                         "the previous kernel's end, what the live HIP events measure) to profiles/trace.json")
    return ap.parse_args()


class Layers:
    """`n` resident MoE layers: 256-slot MXFP4 banks from seeded N(0, 0.02) weights, random bf16 routers."""

    def __init__(self, n, device):
        import torch
        from mimo_stream import pools, kernels, Router, MoEBlock
        self.blocks, self.W = [], []
        for l in range(n):
            bank = pools.random_bank(E, seed=1000 + l, device=device)
            r = Router(H, E, K, device=device)
            r.weight.copy_(kernels.random_bf16((E, H), seed=5000 + l, stddev=0.02, device=device))
            self.blocks.append(MoEBlock(r, bank))
            self.W.append(r.weight.float().cpu().numpy())
        torch.cuda.synchronize()


def steered_rows(rng, W, sets, alpha=6.0):
    """Rows x ~ N(0, 1) plus alpha * sum of the unit router rows of `sets[i]` (float32; the caller rounds to
    bf16): the router picks (almost always exactly) the experts in sets[i]; the realised routing is
    measured and reported."""
    import numpy as np
    Wn = W / np.linalg.norm(W, axis=1, keepdims=True)
    x = rng.standard_normal((len(sets), W.shape[1])).astype(np.float32)
    for i, s in enumerate(sets):
        x[i] += alpha * Wn[list(s)].sum(0)
    return x


def controlled_sets(rng, M, shared_cycle=(3, 2, 3, 3, 2)):
    """Row 0: 8 random experts; row i keeps shared_cycle[i-1 mod 5] of row i-1's experts (mean 2.6) and draws
    the rest fresh (the verify-width routing statistics of bench/results/raw/mimo-cache-sim.json:313-338)."""
    import numpy as np
    sets = [list(rng.choice(E, K, replace=False))]
    for i in range(1, M):
        keep = shared_cycle[(i - 1) % len(shared_cycle)]
        kept = list(rng.choice(sets[-1], keep, replace=False))
        pool = np.setdiff1d(np.arange(E), sets[-1])
        sets.append(kept + list(rng.choice(pool, K - keep, replace=False)))
    return sets


def time_graph(fn, steps, warmup):
    """W eager warm-up steps, capture `steps` steps in one HIP graph, one untimed replay, then one timed
    replay bracketed by synchronisation.  Returns ms per step."""
    import torch
    for s in range(warmup):
        fn(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for s in range(steps):
            fn(s)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    del g
    return ms / steps


def kernel_times(fn, steps):
    """Per-kernel average durations (ms) over `steps` eager steps, from HIP events the library records on
    its launch stream."""
    import torch
    from mimo_stream import _lib
    torch.cuda.synchronize()
    _lib.profile_enable(True)
    for s in range(steps):
        fn(s)
    prof = _lib.profile_read()
    _lib.profile_enable(False)
    return {k: (t / n, n) for k, (t, n) in prof.items()}


def decode_case(layers, M, steps, warmup, seed, device):
    """Fused decode of M rows per step, layers rotated.  Returns dict with ms/step, realised U, GB/s."""
    import numpy as np
    import torch
    rng = np.random.default_rng(seed)
    n = len(layers.blocks)
    nin = steps
    X = np.zeros((nin, M, H), np.float32)
    for s in range(nin):
        l = s % n
        sets = controlled_sets(rng, M)
        X[s] = steered_rows(rng, layers.W[l], sets)
    Xd = torch.from_numpy(X).to(torch.bfloat16).to(device)
    blocks = layers.blocks

    def fn(s):
        blocks[s % n](Xd[s % nin])

    # realised routing on a sample of steps
    Us, shared = [], []
    for s in range(min(nin, 64)):
        _, inds, _ = blocks[s % n](Xd[s], return_routes=True)
        ii = inds.cpu().numpy()
        Us.append(len(np.unique(ii)))
        for r in range(1, M):
            shared.append(len(set(ii[r]) & set(ii[r - 1])))
    U = float(np.mean(Us))
    ms = time_graph(fn, steps, warmup)
    nbytes = U * 13369344 + ROUTER_BYTES + 2 * M * H * 2
    return {"rows": M, "ms_per_layer": ms, "distinct_experts": U,
            "shared_with_previous_row": float(np.mean(shared)) if shared else None,
            "naive_per_row_experts": M * K,
            "GBps": nbytes / (ms * 1e-3) / 1e9, "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "experts_only_GBps": U * 13369344 / (ms * 1e-3) / 1e9, "_fn": fn, "_U": U}


def zipf_routes(T, seed, nin):
    """`nin` routings of T tokens: top-8 distinct experts per token drawn with Zipf(1.1) popularity over a
    seeded permutation of the 256 experts (Gumbel top-k on log p), and normalised random weights."""
    import numpy as np
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    logp = np.log(p / p.sum())
    out = []
    for _ in range(nin):
        g = rng.gumbel(size=(T, E)) + logp[None, :]
        inds = perm[np.argsort(-g, axis=1)[:, :K]].astype(np.int32)
        w = rng.random((T, K)).astype(np.float32)
        w /= w.sum(1, keepdims=True)
        out.append((inds, w))
    return out


def profile_counts():
    """Measured per-layer expert popularity of MiMo-V2.6-Flash (tests/golden/expert_profile.npz, the reference's
    engine/mimo_stream/data/expert_profile.npz): int64 [47, 256] selection counts, row i = MoE layer i + 1."""
    import numpy as np
    with np.load(os.path.join(ROOT, "tests", "golden", "expert_profile.npz"), allow_pickle=False) as z:
        return z["counts"]


def profile_routes(T, seed, layer_rows):
    """One routing of T tokens per entry of layer_rows: top-8 distinct experts per token drawn with that layer's
    measured popularity (Gumbel top-k on log(count), experts never selected in the profile excluded), and
    normalised random weights."""
    import numpy as np
    rng = np.random.default_rng(seed)
    counts = profile_counts()
    out = []
    for l in layer_rows:
        c = counts[l].astype(np.float64)
        with np.errstate(divide="ignore"):
            logp = np.log(c / c.sum())
        g = rng.gumbel(size=(T, E)) + logp[None, :]
        inds = np.argsort(-g, axis=1)[:, :K].astype(np.int32)
        w = rng.random((T, K)).astype(np.float32)
        w /= w.sum(1, keepdims=True)
        out.append((inds, w))
    return out


def hot_routes(T, seed, nin, n_hot=PF_HOT_EXPERTS):
    """`nin` routings of T tokens concentrated on `n_hot` experts (a seeded subset): each token takes 8 of them
    uniformly at random, so every expert gets about T * 8 / n_hot routes and every row tile is a full wide tile
    of a popular expert (the compute-bound part of a Zipf prefill, measured on its own)."""
    import numpy as np
    rng = np.random.default_rng(seed)
    hot = rng.permutation(E)[:n_hot]
    out = []
    for _ in range(nin):
        pick = np.argsort(rng.random((T, n_hot)), axis=1)[:, :K]
        w = rng.random((T, K)).astype(np.float32)
        w /= w.sum(1, keepdims=True)
        out.append((hot[pick].astype(np.int32), w))
    return out


def prefill_case(layers, T, steps, warmup, seed, device, timed=True, routes=None):
    """Expert path of prefill (dispatch + grouped GEMMs + combine) with Zipf(1.1) routes (or the given routings),
    layers rotated.  With timed=False only the step function and the routing statistics are returned."""
    import numpy as np
    import torch
    n = min(len(layers.blocks), 8)
    nin = 4
    Xs, Is, Ws, Us = [], [], [], []
    for inds, w in (routes if routes is not None else zipf_routes(T, seed, nin)):
        Xs.append(torch.randn(T, H, device=device).to(torch.bfloat16))
        Is.append(torch.from_numpy(inds).to(device))
        Ws.append(torch.from_numpy(w).to(device))
        Us.append(len(np.unique(inds)))
    blocks = layers.blocks

    def fn(s):
        blocks[s % n]._moe_prefill(Xs[s % nin], Is[s % nin], Ws[s % nin])

    if not timed:
        return {"_fn": fn, "distinct_experts": float(np.mean(Us)), "inds": [i.cpu().numpy() for i in Is]}
    ms = time_graph(fn, steps, warmup)
    U = float(np.mean(Us))
    nbytes = U * 13369344 + 2 * T * H * 2
    flops = T * K * FLOPS_PER_ROUTE
    return {"tokens": T, "ms_per_layer": ms, "tokens_per_s": T / (ms * 1e-3), "distinct_experts": U,
            "GBps": nbytes / (ms * 1e-3) / 1e9, "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "TFLOPs": flops / (ms * 1e-3) / 1e12,
            "mxfp4_mfma_frac": flops / (ms * 1e-3) / 1e12 / MXFP4_PEAK_TFLOPS, "_fn": fn}


def hot_prefill_case(layers, T, device):
    """Prefill with every route on PF_HOT_EXPERTS experts (hot_routes): only full wide tiles of popular experts,
    the GEMMs' compute-bound case.  Per GEMM: useful TFLOP/s (one product = 2 flops per multiply-add), against
    the hi/lo ceiling (2 fp8 x fp4 MFMAs per product at the 5.0 PF fp8 peak) and, as issued MFMA flops (hi + lo),
    against the issue rate a throughput probe of the same instruction measured."""
    r = prefill_case(layers, T, 20, 3, seed=0, device=device, routes=hot_routes(T, 60 + T, 4))
    kt = kernel_times(r.pop("_fn"), 4)
    r["kernel_us"] = {k: round(v[0] * 1e3, 1) for k, v in kt.items()}
    r["hot_experts"] = PF_HOT_EXPERTS
    r["routes_per_expert"] = T * K / PF_HOT_EXPERTS
    for tag, kern, flops in (("gateup", "prefill_gateup", T * K * 2 * (2 * I * H)),
                             ("down", "prefill_down", T * K * 2 * (H * I))):
        us = kt[kern][0] * 1e3
        useful = flops / (us * 1e-6) / 1e12
        r[tag] = {"us": round(us, 1), "useful_TFLOPs": useful, "hilo_ceiling_frac": useful / HILO_CEILING_TFLOPS,
                  "issued_vs_probe_rate": 2 * useful / ISSUE_RATE_TFLOPS,
                  "mxfp4_mfma_frac": useful / MXFP4_PEAK_TFLOPS}
    return r


def stack_case(layers, M, tokens, device, seed, popularity="zipf"):
    """One decode step through every resident layer (48 = the MiMo stack): per-layer steered hidden states
    whose experts follow Zipf(1.1) popularity, or (popularity="profile") the measured popularity of the matching
    MiMo layer (layer l uses profile row l mod 47); reports MoE time per token and aggregate GB/s."""
    import numpy as np
    import torch
    rng = np.random.default_rng(seed)
    n = len(layers.blocks)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    counts = profile_counts() if popularity == "profile" else None
    Xd, Us = [], []
    for t in range(tokens):
        for l in range(n):
            if counts is not None:
                pl = counts[l % len(counts)] / counts[l % len(counts)].sum()
                sets = [list(rng.choice(E, K, replace=False, p=pl)) for _ in range(M)]
            else:
                perm = np.random.default_rng(10 * l + 1).permutation(E)
                sets = [list(perm[rng.choice(E, K, replace=False, p=p)]) for _ in range(M)]
            Xd.append(torch.from_numpy(steered_rows(rng, layers.W[l], sets)).to(torch.bfloat16).to(device))
            Us.append(len(np.unique(np.concatenate(sets))))
    blocks = layers.blocks

    def fn(s):
        blocks[s % n](Xd[s % len(Xd)])

    steps = n * tokens
    ms = time_graph(fn, steps, warmup=n)
    U = float(np.mean(Us))
    nbytes = U * 13369344 + ROUTER_BYTES + 2 * M * H * 2
    return {"layers": n, "rows": M, "ms_per_token": ms * n, "distinct_experts_per_layer": U,
            "GBps": nbytes * n / (ms * n * 1e-3) / 1e9,
            "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}


HEADLINE_KERNEL = ("decode_gateup_kernel<8, true, false, true>", 32768, 8)   # 1-row decode: 128 x 8 blocks of 256


def trace_parse(d, out_path=None):
    """rocprofv3 kernel trace of bench.py -> markdown on stdout, headline figures to profiles/trace.json (or
    out_path)."""
    import collections
    import csv
    rows = []
    for name in os.listdir(d):
        if name.endswith("kernel_trace.csv"):
            with open(os.path.join(d, name)) as f:
                rows += list(csv.DictReader(f))
    if not rows:
        raise SystemExit(f"{d}: no kernel_trace.csv")
    rows.sort(key=lambda r: (r["Queue_Id"], int(r["Start_Timestamp"])))
    acc = collections.defaultdict(list)
    gap = []
    prev_end = {}
    for r in rows:
        q, t0, t1 = r["Queue_Id"], int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        n = r["Kernel_Name"]
        if "mimo::" in n:
            key = (n.split("(")[0].replace("void ", "").replace("mimo::", ""), int(r["Grid_Size_X"]),
                   int(r["Grid_Size_Y"]), int(r["Workgroup_Size_X"]))
            acc[key].append((t1 - t0) / 1e3)
            if key[:3] == HEADLINE_KERNEL and q in prev_end:
                gap.append((t1 - prev_end[q]) / 1e3)
        prev_end[q] = t1
    print("| kernel | grid (threads) | block | dispatches | avg µs | min µs | max µs |\n|---|---|---|---|---|---|---|")
    for (n, gx, gy, wx), v in sorted(acc.items()):
        print(f"| `{n}` | {gx}×{gy} | {wx} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} |")
    head = [v for k, v in acc.items() if k[:3] == HEADLINE_KERNEL]
    if head:
        v = head[0]
        out = {"decode_gateup_kernel:decode_m1": {
            "avg_us": sum(v) / len(v), "launches": len(v),
            "after_previous_end_us": sum(gap) / len(gap) if gap else None}}
        print(f"\nHeadline kernel `{HEADLINE_KERNEL[0]}` (grid {HEADLINE_KERNEL[1]}×{HEADLINE_KERNEL[2]}): "
              f"{len(v)} dispatches, average duration {out['decode_gateup_kernel:decode_m1']['avg_us']:.2f} µs; "
              f"average interval from the previous kernel's end on its queue to its own end "
              f"{out['decode_gateup_kernel:decode_m1']['after_previous_end_us']:.2f} µs (the interval the "
              f"benchmark's chained HIP events measure).")
        with open(out_path or os.path.join(ROOT, "profiles", "trace.json"), "w") as f:
            json.dump(out, f, indent=1)


def trace_from_profiles(key):
    path = os.path.join(ROOT, "profiles", "trace.json")
    try:
        with open(path) as f:
            return json.load(f).get(key)
    except (OSError, ValueError):
        return None


def traffic_from_profiles(kernel, workload):
    """HBM bytes per launch measured with rocprofv3 counters (committed summary), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            d = json.load(f)
        return d.get(f"{kernel}:{workload}")
    except (OSError, ValueError):
        return None


def cpu_baseline(layers, seconds, n_layers=2):
    """The one-row MoE-layer decode (Router + _gather_m1, model.py:58-65, :173-182) on the host CPU: the fp32
    PyTorch restatement oracle.cpu_decode on every thread PyTorch is given (OMP_NUM_THREADS), over host copies
    of `n_layers` whole resident layers (3.42 GB each, so the experts come from DRAM, not cache), for about
    `seconds` split between its two forms of the expert products: per-32-group sums times the group scale
    (group_dot, no fp32 weight matrix; the reported value) and the whole-matrix dequantise-then-multiply port.
    Returns GB/s with the same byte accounting as the GPU figure."""
    import numpy as np
    import torch
    from oracle import cpu_decode as cd, mxfp4 as oq
    threads = torch.get_num_threads()
    rng = np.random.default_rng(7)
    host = []
    for l in range(min(n_layers, len(layers.blocks))):     # staging, not timed
        b = layers.blocks[l]
        host.append(({k: v.cpu() for k, v in b.bank.items()}, torch.from_numpy(layers.W[l]),
                     b.router.e_score_correction_bias.cpu()))
    res = {}
    for grouped, budget in ((True, 0.6 * seconds), (False, 0.4 * seconds)):
        cd.decode_step(torch.zeros(H), host[0][1], host[0][2], host[0][0], K, grouped)   # warm-up, not timed
        done, t_cpu, nbytes = 0, 0.0, 0.0
        while t_cpu < budget and done < 200:
            pools, W, bias = host[done % len(host)]
            x = torch.from_numpy(oq.round_bf16(steered_rows(rng, W.numpy(), controlled_sets(rng, 1)))[0])
            t0 = time.perf_counter()
            _, inds, _ = cd.decode_step(x, W, bias, pools, K, grouped)
            t_cpu += time.perf_counter() - t0
            done += 1
            nbytes += len(np.unique(inds.numpy())) * 13369344 + ROUTER_BYTES + 2 * H * 2
        res[grouped] = (nbytes / t_cpu / 1e9, done, t_cpu)
    (g_val, g_n, g_t), (p_val, p_n, p_t) = res[True], res[False]
    return {"value": g_val, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{g_n} one-row MoE-layer decode steps (router + 8 MXFP4 experts + combine) over host copies "
                      f"of {len(host)} of the same layers, fp32 PyTorch restatement (oracle/cpu_decode.py, "
                      f"per-32-group sums times the group scale), {threads} threads, {g_t:.1f} s; host: "
                      f"{os.cpu_count()} logical CPUs ({_cpu_model()})",
            "dequant_matrix_port": {"value": p_val, "unit": "GB/s", "steps": p_n, "seconds": round(p_t, 2),
                                    "is": "the same steps with each expert matrix dequantised to fp32, then "
                                          "multiplied"}}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


CALIB_BYTES = 1 << 30        # the calibration copy reads and writes this many bytes
PF_HOT_STEPS = 4             # prefill layers with routes concentrated on PF_HOT_EXPERTS experts


PF_TRAFFIC_T = 2048
PF_TRAFFIC_STEPS = 8


def traffic_run():
    """Workload for the counter runs: the calibration copy (an elementwise multiply by one over 1 GiB, so a
    kernel, not a DMA copy), then 24 one-row decode steps rotating over 8 resident layers (8 x 103 MB, more
    than the 256 MB MALL holds), then 8 prefill layers of 2048 tokens with Zipf(1.1) routes, one per layer, then 4
    prefill layers of 2048 tokens with every route on 16 popular experts (hot_routes)."""
    import numpy as np
    import torch
    src = torch.ones(CALIB_BYTES // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1, out=dst)
    torch.cuda.synchronize()
    del src, dst
    layers = Layers(8, "cuda")
    rng = np.random.default_rng(5)
    xs = [torch.from_numpy(steered_rows(rng, layers.W[l % 8], controlled_sets(rng, 1))).to(torch.bfloat16).cuda()
          for l in range(24)]
    for s in range(24):
        layers.blocks[s % 8](xs[s])
    torch.cuda.synchronize()
    r = prefill_case(layers, PF_TRAFFIC_T, 0, 0, seed=20 + PF_TRAFFIC_T, device="cuda", timed=False)
    for s in range(PF_TRAFFIC_STEPS):
        r["_fn"](s)
    torch.cuda.synchronize()
    r = prefill_case(layers, PF_TRAFFIC_T, 0, 0, seed=0, device="cuda", timed=False,
                     routes=hot_routes(PF_TRAFFIC_T, 60 + PF_TRAFFIC_T, 4))
    for s in range(PF_HOT_STEPS):
        r["_fn"](s)
    torch.cuda.synchronize()
    log("[traffic] done")


def _counter_rows(d):
    import csv
    import glob
    rows = []
    for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            rows += list(csv.DictReader(f))
    if not rows:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    return rows


def gemm_kernels(gate):
    """Kernel-name tests for the two launches of one prefill GEMM: (narrow tiles, wide tiles)."""
    g = "true" if gate else "false"
    return (lambda n: f"prefill_gemm_kernel<{g}, false>" in n), (lambda n: f"prefill_gemm_kernel<{g}, true>" in n)


def per_layer(vals_narrow, vals_wide, combine=lambda a, b: a + b):
    """One value per prefill layer from the per-dispatch values of its narrow and wide launches (dispatch
    order; a layer without narrow tiles has no narrow launch only when no layer has one)."""
    if not vals_narrow:
        return list(vals_wide)
    if len(vals_narrow) != len(vals_wide):
        raise SystemExit(f"{len(vals_narrow)} narrow vs {len(vals_wide)} wide launches")
    return [combine(a, b) for a, b in zip(vals_narrow, vals_wide)]


def traffic_parse(fetch_dir, write_dir):
    """Per-dispatch FETCH_SIZE / WRITE_SIZE (KiB) averaged per kernel; each scaled by bytes / counter of the
    calibration copy.  Writes profiles/traffic.json and prints a markdown summary."""
    def per_kernel(d, counter):   # per kernel, values in dispatch order
        acc = {}
        for r in sorted(_counter_rows(d), key=lambda r: int(r["Dispatch_Id"])):
            if r.get("Counter_Name") != counter:
                continue
            acc.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]) * 1024.0)
        return acc
    f = per_kernel(fetch_dir, "FETCH_SIZE")
    w = per_kernel(write_dir, "WRITE_SIZE")
    def pick(acc, key):
        names = [n for n in acc if key(n)]
        if not names:
            raise SystemExit(f"kernel not found among {sorted(acc)[:20]}")
        vals = [v for n in names for v in acc[n]]
        return names[0], vals
    cal = lambda n: "elementwise" in n and "Mul" in n
    gu = lambda n: "decode_gateup_kernel" in n
    _, cf = pick(f, cal)
    _, cw = pick(w, cal)
    fetch_scale = CALIB_BYTES / (sum(cf) / len(cf))
    write_scale = CALIB_BYTES / (sum(cw) / len(cw))
    name, gf = pick(f, gu)
    _, gw = pick(w, gu)
    fetch = sum(gf) / len(gf) * fetch_scale
    write = sum(gw) / len(gw) * write_scale
    algo = 8 * GATEUP_BYTES_PER_EXPERT
    out = {"decode_gateup_kernel:decode_m1": fetch + write,
           "_detail": {"kernel": name, "dispatches": len(gf), "fetch_bytes": fetch, "write_bytes": write,
                       "algorithmic_bytes": algo, "fetch_scale": fetch_scale, "write_scale": write_scale,
                       "calibration": "elementwise multiply by one over 1 GiB: reads and writes 1 GiB"}}
    rows = [("decode_gateup_kernel (1 row, 8 experts)", len(gf), fetch, write, algo)]
    # prefill GEMMs of the payload: algorithmic bytes = distinct experts' weights and scales + activation codes
    # and scales read + results written (hi/lo E4M3 h with scales, or bf16 Y)
    import numpy as np
    T, P = PF_TRAFFIC_T, PF_TRAFFIC_T * K
    routes = zipf_routes(T, 20 + T, 4)
    U = float(np.mean([len(np.unique(routes[s % 4][0])) for s in range(PF_TRAFFIC_STEPS)]))
    split = lambda rows_, cols: 2 * rows_ * cols + 2 * rows_ * cols // 32          # hi + lo codes and scales
    algo_pf = {True: U * GATEUP_BYTES_PER_EXPERT + split(T, H) + split(P, I),
               False: U * (H * I // 2 + H * I // 32) + split(P, I) + P * H * 2}
    def layer_vals(acc, gate):
        kn, kw = gemm_kernels(gate)
        vn = [v for n in acc if kn(n) for v in acc[n]]
        _, vw = pick(acc, kw)
        return per_layer(vn, vw)
    for gate in (True, False):
        pname = f"prefill_gemm_kernel<{'true' if gate else 'false'}, narrow + wide>"
        pf_ = layer_vals(f, gate)[:PF_TRAFFIC_STEPS]                  # the Zipf layers come first
        pw_ = layer_vals(w, gate)[:PF_TRAFFIC_STEPS]
        pfetch = sum(pf_) / len(pf_) * fetch_scale
        pwrite = sum(pw_) / len(pw_) * write_scale
        tag = "prefill_gateup" if gate else "prefill_down"
        out[f"prefill_gemm_kernel<{'true' if gate else 'false'}>:prefill_t{T}"] = pfetch + pwrite
        out[f"_detail_{tag}"] = {"kernel": pname, "dispatches": len(pf_), "fetch_bytes": pfetch,
                                 "write_bytes": pwrite, "algorithmic_bytes": algo_pf[gate],
                                 "distinct_experts": U}
        rows.append((f"prefill {'gate/up' if gate else 'down'} GEMM, narrow + wide launches ({T} tokens, {U:.1f} experts)",
                     len(pf_), pfetch, pwrite, algo_pf[gate]))
    with open(os.path.join(ROOT, "profiles", "traffic.json"), "w") as fh:
        json.dump(out, fh, indent=1)
    print(f"| kernel | dispatches | FETCH (MB/launch) | WRITE (MB/launch) | algorithmic (MB/launch) | "
          f"(fetch + write) / algorithmic |")
    print(f"|---|---|---|---|---|---|")
    for nm, nd, fe, wr, al in rows:
        print(f"| {nm} | {nd} | {fe / 1e6:.2f} | {wr / 1e6:.3f} | {al / 1e6:.2f} | {(fe + wr) / al:.3f} |")
    print(f"\ncalibration: FETCH_SIZE scale {fetch_scale:.4f}, WRITE_SIZE scale {write_scale:.4f} (bytes per counted "
          f"byte, from the 1 GiB elementwise copy)")


def mfma_parse(pmc_dir, trace_dir):
    """MFMA work of the prefill GEMMs from a --pmc run (SQ_INSTS_MFMA, SQ_VALU_MFMA_BUSY_CYCLES,
    GRBM_GUI_ACTIVE) and their durations from a --kernel-trace run of the same payload: the Zipf(1.1) layers
    (the first PF_TRAFFIC_STEPS of each GEMM) and the layers on PF_HOT_EXPERTS experts (the next PF_HOT_STEPS).
    A GEMM is two concurrent launches (narrow and wide tiles): instructions are summed, its time runs from the
    first start to the last end of the pair in the trace run."""
    import csv
    import glob
    cnt = {}
    for r in sorted(_counter_rows(pmc_dir), key=lambda r: int(r["Dispatch_Id"])):
        k = r["Kernel_Name"]
        if "prefill_gemm_kernel" in k:
            cnt.setdefault(k, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    spans = {}
    trows = []
    for path in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        with open(path) as f:
            trows += [r for r in csv.DictReader(f) if "prefill_gemm_kernel" in r["Kernel_Name"]]
    for r in sorted(trows, key=lambda r: int(r["Dispatch_Id"])):
        spans.setdefault(r["Kernel_Name"], []).append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    groups = ((f"2048 tokens, Zipf(1.1)", 0, PF_TRAFFIC_STEPS),
              (f"2048 tokens on {PF_HOT_EXPERTS} experts", PF_TRAFFIC_STEPS, PF_TRAFFIC_STEPS + PF_HOT_STEPS))
    print("| GEMM | routes | layers | MFMA instr / layer | avg µs | MFMA TFLOP/s issued (hi + lo) | "
          "useful TFLOP/s | issued / probe rate | useful / hi-lo ceiling | busy cycles / instr |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for gate in (True, False):
        kn, kw = gemm_kernels(gate)
        sel = lambda src, key, c=None: [v for n in src if key(n) for v in (src[n][c] if c else src[n])]
        inst = per_layer(sel(cnt, kn, "SQ_INSTS_MFMA"), sel(cnt, kw, "SQ_INSTS_MFMA"))
        busy = per_layer(sel(cnt, kn, "SQ_VALU_MFMA_BUSY_CYCLES"), sel(cnt, kw, "SQ_VALU_MFMA_BUSY_CYCLES"))
        span = per_layer(sel(spans, kn), sel(spans, kw), lambda a, b: (min(a[0], b[0]), max(a[1], b[1])))
        for label, a, b in groups:
            n = len(inst[a:b])
            if not n or not span[a:b]:
                continue
            ins = sum(inst[a:b]) / n
            bz = sum(busy[a:b]) / n
            d = sum((e - st) * 1e-9 for st, e in span[a:b]) / len(span[a:b])
            issued = ins * 16 * 16 * 128 * 2 / d / 1e12
            print(f"| {'gate/up' if gate else 'down'} | {label} | {n} | {ins:,.0f} | {d * 1e6:.1f} | {issued:.0f} | "
                  f"{issued / 2:.0f} | {issued / ISSUE_RATE_TFLOPS:.2f} | {issued / 2 / HILO_CEILING_TFLOPS:.2f} | "
                  f"{bz / ins:.1f} |")


def pipe_parse(lds_dir, wait_dir):
    """Where the prefill GEMMs' waves spend their cycles, per launch (narrow or wide tiles; counter runs serialise
    the two launches of a GEMM) and routing group (as mfma_parse):
    LDS utilisation (SQ_LDS_IDX_ACTIVE over GRBM_GUI_ACTIVE of one XCD x 256 CUs), bank conflicts per access,
    MFMA pipe busy per SIMD, and the fractions of wave-cycles waiting (SQ_WAIT_ANY: s_waitcnt and barriers;
    SQ_WAIT_INST_ANY: an instruction waiting to issue) or issuing (SQ_ACTIVE_INST_ANY / _LDS)."""
    def load(d):
        cnt = {}
        for r in sorted(_counter_rows(d), key=lambda r: int(r["Dispatch_Id"])):
            if "prefill_gemm_kernel" in r["Kernel_Name"]:
                cnt.setdefault(r["Kernel_Name"], {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        return cnt
    lds, wt = load(lds_dir), load(wait_dir)
    groups = ((f"2048 tokens, Zipf(1.1)", 0, PF_TRAFFIC_STEPS),
              (f"2048 tokens on {PF_HOT_EXPERTS} experts", PF_TRAFFIC_STEPS, PF_TRAFFIC_STEPS + PF_HOT_STEPS))
    print("| kernel | routes | LDS busy | bank conflicts / access | MFMA busy / SIMD | waiting (waitcnt, barrier) | "
          "waiting to issue | issuing | issuing LDS |")
    print("|---|---|---|---|---|---|---|---|---|")
    for k in sorted(lds):
        for label, a, b in groups:
            m = lambda c, src: sum(src[k][c][a:b]) / len(src[k][c][a:b])
            grbm = m("GRBM_GUI_ACTIVE", lds) / 8          # summed over the 8 XCDs
            ia, bc = m("SQ_LDS_IDX_ACTIVE", lds), m("SQ_LDS_BANK_CONFLICT", lds)
            g2 = m("GRBM_GUI_ACTIVE", wt) / 8
            wc = m("SQ_WAVE_CYCLES", wt)
            if ia <= bc or wc <= 0:                      # a launch with no tiles of its shape in these layers
                continue
            print(f"| {k.split('(')[0].replace('void mimo::', '')} | {label} | {ia / (grbm * 256):.2f} | {bc / (ia - bc):.2f} | "
                  f"{m('SQ_VALU_MFMA_BUSY_CYCLES', wt) / (g2 * 1024):.2f} | {m('SQ_WAIT_ANY', wt) / wc:.2f} | "
                  f"{m('SQ_WAIT_INST_ANY', wt) / wc:.2f} | {m('SQ_ACTIVE_INST_ANY', wt) / wc:.2f} | "
                  f"{m('SQ_ACTIVE_INST_LDS', wt) / wc:.2f} |")


def layer_case(layers, T, steps, warmup, seed, device):
    """The MoE half of a decoder layer (post-attention RMSNorm, block, residual added in the combine) against the
    block alone on the normalised rows (so both route identically), layers rotated; the difference is what the
    norm and the residual cost."""
    import numpy as np
    import torch
    from mimo_stream import MoELayer
    rng = np.random.default_rng(seed)
    n = len(layers.blocks)
    nin = min(steps, 64) if T <= 8 else 4
    if T <= 8:
        X = np.stack([steered_rows(rng, layers.W[s % n], controlled_sets(rng, T)) for s in range(nin)])
        Xd = torch.from_numpy(X).to(torch.bfloat16).to(device)
    else:
        Xd = torch.randn(nin, T, H, device=device).to(torch.bfloat16)
    g = torch.Generator(device=device).manual_seed(seed)
    lays = [MoELayer(b, (1.0 + 0.1 * torch.randn(H, device=device, generator=g)).to(torch.bfloat16), 1e-5)
            for b in layers.blocks]
    blocks = layers.blocks
    Rd = {(j, i): lays[j].norm(Xd[i]) for j in range(n) for i in range(nin)}
    ms_l = time_graph(lambda s: lays[s % n](Xd[s % nin]), steps, warmup)
    ms_b = time_graph(lambda s: blocks[s % n](Rd[(s % n, s % nin)]), steps, warmup)
    return {"rows": T, "layer_us": ms_l * 1e3, "block_us": ms_b * 1e3, "norm_and_residual_us": (ms_l - ms_b) * 1e3}


def main():
    args = parse()
    if args.mfma_parse:
        mfma_parse(args.mfma_parse, args.mfma_trace)
        return
    if args.pipe_parse:
        pipe_parse(*args.pipe_parse)
        return
    if args.traffic_parse:
        traffic_parse(*args.traffic_parse)
        return
    if args.trace_parse:
        trace_parse(args.trace_parse)
        return
    if args.traffic_run:
        traffic_run()
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "bench.py measures one GPU only: the MoE block runs on a single MI355X "
                                   "(multi-GPU sharding is designed, not implemented)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device"}))
        sys.exit(1)
    device = "cuda:0"
    torch.cuda.set_device(0)
    t0 = time.time()
    layers = Layers(args.layers, device)
    log(f"[bench] {args.layers} layers resident ({args.layers * E * 13369344 / 1e9:.1f} GB) in {time.time() - t0:.1f}s")

    head = decode_case(layers, 1, args.steps, args.warmup, seed=1, device=device)
    log(f"[bench] decode M=1: {head['ms_per_layer'] * 1e3:.1f} us/layer, {head['GBps']:.0f} GB/s")
    kt = kernel_times(head["_fn"], min(args.steps, 200))
    gu_ms, gu_n = kt.get("decode_gateup", (float("nan"), 0))
    bpl = head["_U"] * GATEUP_BYTES_PER_EXPERT
    live_us = gu_ms * 1e3
    tr = trace_from_profiles("decode_gateup_kernel:decode_m1")
    # The kernel's own duration comes from the committed rocprofv3 kernel trace of this benchmark (profiles/): HIP
    # events on the launch stream cannot isolate it (an event completes when the previous kernel does, so the live
    # interval includes the dispatch gap before the kernel).  The live figure is kept beside it.
    avg_us = tr["avg_us"] if tr else live_us
    achieved = bpl / (avg_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "kernel": "decode_gateup_kernel", "achieved": achieved, "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                "traffic": traffic_from_profiles("decode_gateup_kernel", "decode_m1"),
                "bytes_per_launch": bpl, "avg_us": avg_us,
                "avg_us_is": ("rocprofv3 kernel-trace average duration of this kernel in this benchmark "
                              "(profiles/bench_kernels_trace.md, profiles/trace.json)") if tr else
                             "live HIP events (no committed trace found)",
                "avg_us_live": live_us, "launches_timed_live": gu_n,
                "frac_live": bpl / (live_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
                "avg_us_live_is": "live HIP events on the launch stream, from the previous kernel's end to this "
                                  "kernel's end (the dispatch gap before the kernel included)"}
    if tr:
        roofline["after_previous_end_us_trace"] = tr.get("after_previous_end_us")
        roofline["trace_launches"] = tr.get("launches")

    extra = {"kernel_us_decode_m1": {k: round(v[0] * 1e3, 2) for k, v in kt.items()}}
    if not args.no_extra:
        for M in (2, 4, 8):
            try:
                r = decode_case(layers, M, min(args.steps, 300), args.warmup, seed=10 + M, device=device)
                r.pop("_fn"), r.pop("_U")
                extra[f"decode_m{M}"] = r
                log(f"[bench] decode M={M}: {r['ms_per_layer'] * 1e3:.1f} us/layer, U={r['distinct_experts']:.1f}, {r['GBps']:.0f} GB/s")
            except Exception as e:    # an extra measurement never hides the headline
                extra[f"decode_m{M}"] = {"error": repr(e)}
        for T, pop in ((512, "zipf"), (2048, "zipf"), (2048, "profile")):
            key = f"prefill_t{T}" + ("_profile" if pop == "profile" else "")
            try:
                routes = profile_routes(T, 20 + T, (0, 14, 29, 43)) if pop == "profile" else None
                r = prefill_case(layers, T, 20, 3, seed=20 + T, device=device, routes=routes)
                kt2 = kernel_times(r.pop("_fn"), 4)
                r["kernel_us"] = {k: round(v[0] * 1e3, 1) for k, v in kt2.items()}
                if pop == "profile":
                    r["routing"] = "measured MiMo popularity, profile layers 1, 15, 30, 44"
                extra[key] = r
                log(f"[bench] prefill T={T} ({pop}): {r['ms_per_layer']:.3f} ms/layer, {r['tokens_per_s']:.0f} tok/s")
            except Exception as e:
                extra[key] = {"error": repr(e)}
        key = f"prefill_t2048_hot{PF_HOT_EXPERTS}"
        try:
            extra[key] = hot_prefill_case(layers, 2048, device)
            log(f"[bench] prefill T=2048 on {PF_HOT_EXPERTS} experts: {extra[key]['ms_per_layer']:.3f} ms/layer, "
                f"gate/up {extra[key]['gateup']['useful_TFLOPs']:.0f} useful TFLOP/s")
        except Exception as e:
            extra[key] = {"error": repr(e)}
        for M, pop in ((1, "zipf"), (4, "zipf"), (1, "profile"), (4, "profile")):
            key = f"stack{args.layers}_m{M}" + ("_profile" if pop == "profile" else "")
            try:
                r = stack_case(layers, M, tokens=4, device=device, seed=30 + M, popularity=pop)
                extra[key] = r
                log(f"[bench] stack M={M} ({pop}): {r['ms_per_token']:.3f} ms/token, {r['GBps']:.0f} GB/s")
            except Exception as e:
                extra[key] = {"error": repr(e)}
        for T, st in ((1, min(args.steps, 300)), (2048, 10)):
            try:
                r = layer_case(layers, T, st, 3, seed=40 + T, device=device)
                extra[f"layer_t{T}"] = r
                log(f"[bench] layer T={T}: {r['layer_us']:.1f} us (block alone {r['block_us']:.1f} us)")
            except Exception as e:
                extra[f"layer_t{T}"] = {"error": repr(e)}
    head.pop("_fn"), head.pop("_U")
    extra["decode_m1"] = head

    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(layers, args.cpu_seconds)
        except Exception as e:
            cpu = {"error": repr(e)}

    out = {
        "metric": METRIC, "value": head["GBps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_layer"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "mxfp4 x bf16 -> fp32 (block-scaled fp8/fp4 MFMA)", "data": "synthetic",
        "config": {"workload": "MiMo-V2.6-Flash MoE layer decode, 1 row: router 4096->256 bf16, top-8, 256 "
                               "resident MXFP4 experts (I=2048, group 32), SwiGLU, fixed-order combine",
                   "hidden": H, "experts": E, "top_k": K, "intermediate": I, "rows": 1,
                   "resident_layers": args.layers, "hbm_frac": head["hbm_frac"]},
        "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
