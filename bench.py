#!/usr/bin/env python3
"""Streamed-MoE layer benchmark on one MI355X.

Headline (`value`): decode tokens/s through one full-width MoE layer --
d_model 4096, 256 routed experts (top-6, sqrt-softplus router) + 1 shared
expert, d_ff 2048, 2-bit affine weights (group 64, bf16 scales/biases), all
257 expert slots resident in an HBM arena, 1 token per step, uniform-random
routing. A step is one token through router, experts, combine and shared
expert. Steps are replayed from a captured HIP graph (inputs already in HBM).

Also reported:
  roofline      the dominant kernel (decode gate/up + SwiGLU), its average
                launch duration from HIP events around a graph of back-to-back
                launches on the replay stream, achieved algorithmic GB/s
                against the 8 TB/s peak, and `traffic`: HBM bytes per launch
                measured by two rocprofv3 --pmc passes (FETCH_SIZE, then
                WRITE_SIZE), each scaled by what the counter reads for a
                reference kernel of known bytes -- a 256 MiB reduction and a
                256 MiB fill (`--copy-calibration`) -- summarised by
                `--summarize-pmc` into profiles/gateup_diag_kernel_decode_traffic.json
  prefill64     64-token prefill on the same layer with Zipf(1.1) expert
                popularity (grouped path), tokens/s and algorithmic GB/s
  cpu_baseline  the C oracle (oracle/expert_ref.c, OpenMP) on the host cores
                over a bounded sample of the same decode workload; a stand-in
                for the reference's MLX-CPU path, which cannot run here

`python bench.py --gpus N` with N > 1 exits: this path is measured on one GPU.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from locali_amd import ops, synth  # noqa: E402

METRIC = "MoE-layer tokens/s at 1 GPU (decode & 64-tok prefill); achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "gateup_diag_kernel_decode_traffic.json"
GATEUP_KERNEL = "gateup_diag_kernel<2, true>"
COPY_BYTES = 256 << 20
D, E, DFF, K_TOP, GROUP, BITS = 4096, 256, 2048, 6, 64, 2


def proj_bytes(rows, cols, bits=BITS, group=GROUP):
    return rows * cols * bits // 8 + 2 * 2 * rows * (cols // group)


EXPERT_BYTES = 2 * proj_bytes(DFF, D) + proj_bytes(D, DFF)          # 7,864,320
GATEUP_ROUTE_BYTES = 2 * proj_bytes(DFF, D)                           # 5,242,880
ROUTER_BYTES = E * D * 2
# per decode gate/up launch: 7 routes' gate+up slots, x read once, h written
GATEUP_ALG_BYTES = (K_TOP + 1) * GATEUP_ROUTE_BYTES + D * 2 + (K_TOP + 1) * DFF * 2   # 36,737,024


def layer(dev, seed=1):
    arena = synth.expert_arena(E + 1, D, DFF, bits_gate_up=BITS, group=GROUP, dtype=torch.bfloat16,
                               seed=seed, device=dev)
    shared = synth.expert_arena(1, D, DFF, bits_gate_up=BITS, group=GROUP, dtype=torch.bfloat16,
                                seed=seed + 1, device=dev, zero_slot=False)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=dev)
    return arena, shared, slot_of


def decode_graph_run(spec, arena, shared, slot_of, X, ws, steps, warmup, use_graph):
    """Returns elapsed seconds for exactly `steps` decode steps."""
    n_in = X.shape[0]
    outs = torch.empty_like(X)
    idx = torch.empty(n_in, K_TOP, dtype=torch.int32, device=X.device)
    wts = torch.empty(n_in, K_TOP, dtype=torch.float32, device=X.device)

    def step(i):
        j = i % n_in
        ops.forward(spec, arena, shared, slot_of, X[j:j + 1], ws, out=outs[j:j + 1],
                    idx=idx[j:j + 1], weights=wts[j:j + 1])

    for i in range(max(warmup, 1)):
        step(i)
    torch.cuda.synchronize()
    graphs = []
    if use_graph:
        chunk = min(n_in, steps)
        sizes = [chunk] * (steps // chunk) + ([steps % chunk] if steps % chunk else [])
        cache = {}
        for n in sizes:
            if n not in cache:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for i in range(n):
                        step(i)
                cache[n] = g
            graphs.append(cache[n])
        for g in set(graphs):       # one untimed replay of each graph
            g.replay()
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    if use_graph:
        for g in graphs:
            g.replay()
    else:
        for i in range(steps):
            step(i)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / 1e3, wall, idx


def stage_timing(spec, arena, shared, slot_of, X, ws, m=40, replays=5):
    """Average device time (s) of one router / gate-up / down+combine launch.

    Each stage is captured m times back to back (inputs 0..m-1, so every
    launch streams different experts) into its own HIP graph; HIP events on
    the replay stream bracket `replays` replays, and the per-launch average
    is elapsed / (replays * m) -- the same quantity rocprofv3 reports as a
    kernel's average duration."""
    dev = X.device
    n_in = X.shape[0]
    xs = [X[i % n_in:i % n_in + 1] for i in range(m)]
    hidden = torch.empty(K_TOP + 1, DFF, dtype=torch.bfloat16, device=dev)
    out = torch.empty(1, D, dtype=torch.bfloat16, device=dev)
    dws = ops.Workspace(dev)
    dws.reserve(1, D, DFF, 1, K_TOP, True)
    routed = [ops.router(spec, x, ws, slot_of_expert=slot_of, n_slots=E + 1) for x in xs]
    stages = {
        "router": lambda i: ops.router(spec, xs[i], ws, slot_of_expert=slot_of, n_slots=E + 1),
        "gateup": lambda i: ops.decode_gateup(arena, shared, xs[i], routed[i][2], hidden, dws),
        "down_combine": lambda i: ops.decode_down_combine(arena, shared, routed[i][2], routed[i][1],
                                                          out, dws),
    }
    res = {}
    for name, fn in stages.items():
        for i in range(2):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(m):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        res[name] = e0.elapsed_time(e1) / 1e3 / (replays * m)
    return res


def prefill_run(arena, shared, slot_of, dev, tokens, calls, seed):
    """Zipf(1.1) routing through the real router (x . Wg == Zipf logits)."""
    batches = []
    for c in range(calls):
        x, w = synth.zipf_router_inputs(tokens, E, D, 1.1, torch.bfloat16, seed=seed + c, device=dev)
        batches.append(x)
    spec = ops.RouterSpec(w, K_TOP, routed_scale=1.5)
    ws = ops.Workspace(dev)
    out = torch.empty(tokens, D, dtype=torch.bfloat16, device=dev)
    idx = torch.empty(tokens, K_TOP, dtype=torch.int32, device=dev)
    wts = torch.empty(tokens, K_TOP, dtype=torch.float32, device=dev)
    for x in batches[:2]:
        ops.forward(spec, arena, shared, slot_of, x, ws, out=out, idx=idx, weights=wts)
    torch.cuda.synchronize()
    distinct = []
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for x in batches:
        ops.forward(spec, arena, shared, slot_of, x, ws, out=out, idx=idx, weights=wts)
    e1.record()
    torch.cuda.synchronize()
    secs = e0.elapsed_time(e1) / 1e3
    for x in batches:                      # distinct experts per call (untimed)
        i, _, _ = ops.router(spec, x, ws)
        distinct.append(int(torch.unique(i).numel()))
    u = sum(distinct) / len(distinct)
    algo = (u + 1) * EXPERT_BYTES + ROUTER_BYTES + tokens * D * 2 * 2
    per_call = secs / calls
    return {"tokens": tokens, "calls": calls, "value": tokens * calls / secs, "unit": "tokens/s",
            "ms_per_call": per_call * 1e3, "distinct_experts": u,
            "algorithmic_bytes_per_call": int(algo),
            "achieved_GBps": algo / per_call / 1e9, "frac_of_hbm_peak": algo / per_call / 1e9 / HBM_PEAK_GBS}


def cpu_baseline(arena, shared, spec, X, seconds):
    """C oracle on the host cores, decode tokens until `seconds` elapse."""
    import numpy as np
    from oracle import cref
    lib_path = ROOT / "oracle" / "liboracle.so"
    if not lib_path.exists():
        import subprocess
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "oracle"], check=True)
    ref = cref.load()

    def host(p):
        return (p.weight.cpu().view(torch.int32).numpy().view(np.uint32),
                p.scales.cpu().view(torch.int16).numpy().view(np.uint16),
                p.biases.cpu().view(torch.int16).numpy().view(np.uint16), p.bits, p.group_size)

    names = ("gate_proj", "up_proj", "down_proj")
    ha = {n: host(p) for n, p in zip(names, (arena.gate, arena.up, arena.down))}
    hs = {n: host(p) for n, p in zip(names, (shared.gate, shared.up, shared.down))}
    wg = spec.weight.float().cpu().numpy()
    xs = X.float().cpu().numpy()
    n = 0
    t0 = time.perf_counter()
    while True:
        x = xs[n % xs.shape[0]:n % xs.shape[0] + 1]
        idx, w = ref.router(x, wg, None, K_TOP, 0, True, spec.routed_scale)
        ref.moe_layer(x, idx + 1, w, ha, "bf16", shared=hs)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 2:
            break
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
    return {"value": n / el, "unit": "tokens/s", "cores": min(threads, len(os.sched_getaffinity(0))),
            "kind": "port",
            "sample": f"{n} decode tokens of the same layer (router + 6 routed + shared experts), "
                      f"{el:.1f} s, C oracle oracle/expert_ref.c with OpenMP; stand-in for the "
                      "reference dsv4_arena path on MLX's CPU backend (not runnable here)"}


def copy_calibration(dev):
    """Reference kernels of known traffic for the FETCH_SIZE / WRITE_SIZE
    counters: a reduction that reads COPY_BYTES (and writes one scalar) and a
    fill that writes COPY_BYTES (and reads nothing). A plain copy is not used:
    its stores allocate lines in L2 and read them first, so its FETCH_SIZE
    counts the destination as well."""
    src = torch.ones(COPY_BYTES // 2, dtype=torch.bfloat16, device=dev)
    for _ in range(3):
        src.sum()
        src.fill_(0.5)
    torch.cuda.synchronize()


def summarize_pmc(fetch_csv, write_csv, out_path=TRAFFIC_FILE):
    """Turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE pass,
    WRITE_SIZE pass) into HBM bytes per launch of the decode gate/up kernel,
    each counter scaled by its reading for a reference kernel of known bytes
    (reduction for FETCH_SIZE, fill for WRITE_SIZE)."""
    import csv

    def per_kernel(path, counter, ref_name):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
        refs = [float(r["Counter_Value"]) for r in rows
                if ref_name in r["Kernel_Name"] and int(r["Grid_Size"]) >= 1 << 16]
        target = [float(r["Counter_Value"]) for r in rows if GATEUP_KERNEL in r["Kernel_Name"]]
        if not refs or not target:
            raise SystemExit(f"{path}: no {counter} rows for {ref_name} and/or {GATEUP_KERNEL}")
        ref_kib = sorted(refs)[len(refs) // 2]
        scale = (COPY_BYTES / 1024) / ref_kib        # true KiB per counted KiB
        kib = sum(target) / len(target)
        return {"counter_kib_per_launch": kib, "reference_kernel": ref_name,
                "reference_counter_kib": ref_kib, "reference_true_kib": COPY_BYTES / 1024,
                "scale": scale, "bytes_per_launch": kib * 1024 * scale, "launches": len(target)}

    fetch = per_kernel(fetch_csv, "FETCH_SIZE", "reduce_kernel")
    write = per_kernel(write_csv, "WRITE_SIZE", "FillFunctor")
    res = {"kernel": GATEUP_KERNEL, "fetch": fetch, "write": write,
           "traffic_bytes_per_launch": fetch["bytes_per_launch"] + write["bytes_per_launch"],
           "algorithmic_bytes_per_launch": GATEUP_ALG_BYTES}
    Path(out_path).write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res, indent=1))
    return res


def measured_traffic():
    try:
        t = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    return t.get("traffic_bytes_per_launch") if t.get("kernel") == GATEUP_KERNEL else None


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-graph", action="store_true", help="launch steps eagerly")
    ap.add_argument("--prefill-calls", type=int, default=20)
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run 256 MiB read and write reference kernels first (for --pmc byte counters)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc runs into HBM bytes per gate/up launch")
    args = ap.parse_args(argv)
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures the streamed-MoE layer on one GPU; expert-parallel runs over "
              "several GPUs are not implemented.", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        copy_calibration(dev)
    print(f"[bench] building layer d={D} E={E} dff={DFF} {BITS}-bit g{GROUP}", file=sys.stderr, flush=True)
    arena, shared, slot_of = layer(dev, args.seed)
    w, _ = synth.uniform_router(E, D, torch.bfloat16, seed=args.seed + 2, device=dev)
    spec = ops.RouterSpec(w, K_TOP, routed_scale=1.5)
    n_inputs = 200   # 200 distinct tokens x 57 MB per step >> 256 MB MALL
    X = synth.activations(n_inputs, D, torch.bfloat16, seed=args.seed + 3, device=dev)
    ws = ops.Workspace(dev)
    ws.reserve(1, D, DFF, E, K_TOP, True)

    print("[bench] decode", file=sys.stderr, flush=True)
    secs, wall, idx = decode_graph_run(spec, arena, shared, slot_of, X, ws, args.steps, args.warmup,
                                       not args.no_graph)
    value = args.steps / secs
    layer_bytes = 7 * EXPERT_BYTES + ROUTER_BYTES

    print("[bench] stage timing", file=sys.stderr, flush=True)
    st = stage_timing(spec, arena, shared, slot_of, X, ws)
    gate_bytes = GATEUP_ALG_BYTES
    achieved = gate_bytes / st["gateup"] / 1e9
    result = {
        "metric": METRIC,
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": secs / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "full-width decode MoE layer: d_model 4096, 256 routed experts top-6 "
                        "(sqrt-softplus, scale 1.5) + 1 shared expert, d_ff 2048, 2-bit affine "
                        "group-64 weights with bf16 scales/biases, fp32 accumulation, all 257 "
                        "slots resident in HBM, 1 token per step, uniform-random routing",
            "tokens_per_step": 1,
            "graph_replay": not args.no_graph,
            "wall_s": wall,
            "layer_bytes_per_token": layer_bytes,
            "layer_GBps": layer_bytes * value / 1e9,
            "layer_frac_of_hbm_peak": layer_bytes * value / 1e9 / HBM_PEAK_GBS,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gateup_diag_kernel (decode gate/up + clamped SwiGLU on the matrix cores, 7 routes)",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(),
            "algorithmic_bytes_per_launch": gate_bytes,
            "avg_launch_us": st["gateup"] * 1e6,
            "stage_us": {k: v * 1e6 for k, v in st.items()},
        },
    }
    if not args.skip_prefill:
        print("[bench] prefill 64", file=sys.stderr, flush=True)
        result["prefill64"] = prefill_run(arena, shared, slot_of, dev, 64, args.prefill_calls,
                                          args.seed + 100)
    if not args.skip_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(arena, shared, spec, X, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
