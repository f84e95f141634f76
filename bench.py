#!/usr/bin/env python3
"""Streamed-MoE layer benchmark on one MI355X.

Headline (`value`): decode tokens/s through one full-width MoE layer --
d_model 4096, 256 routed experts (top-6, sqrt-softplus router) + 1 shared
expert, d_ff 2048, 2-bit affine weights (group 64, bf16 scales/biases), all
257 expert slots resident in an HBM arena, 1 token per step, uniform-random
routing. A step is one token through router, experts, combine and shared
expert. Steps are replayed from a captured HIP graph (inputs already in HBM)
and rotate over 64 copies of the router and shared expert, so that no step
finds them in the 256 MB MALL (a model's layers each have their own).

Also reported:
  roofline      the dominant kernel, the step's first launch (router rows,
                gate/up + SwiGLU, top-6 selection), its average launch
                duration from HIP events around graphs of back-to-back steps
                and of back-to-back down kernels on the replay stream,
                achieved algorithmic GB/s against the 8 TB/s peak, and
                `traffic`: HBM bytes per launch
                measured by two rocprofv3 --pmc passes (FETCH_SIZE, then
                WRITE_SIZE), each scaled by what the counter reads for a
                reference kernel of known bytes -- a 256 MiB reduction and a
                256 MiB fill (`--copy-calibration`) -- summarised by
                `--summarize-pmc` into profiles/gateup_diag_kernel_decode_traffic.json
  decode_g128   the decode leg with the real checkpoint's 2-bit experts in
                groups of 128 (7,077,888 B per expert)
  decode_3bit_g128
                the decode leg with the DSpark/MTP tier's experts: 3-bit codes
                in groups of 128 (10,223,616 B per expert)
  prefill64, prefill512
                64- and 512-token prefill on the same layer with Zipf(1.1)
                expert popularity (grouped path): tokens/s, algorithmic GB/s
                against 8 TB/s, and matrix-core utilisation (flops against
                the 2.5 PFLOP/s dense bf16 peak)
  prefill64_3bit_g128, prefill512_3bit_g128
                the same prefill calls on the DSpark/MTP tier's experts (3-bit
                codes in groups of 128, the 64-position matrix-core kernels
                for tiles of every size)
  prefill512_heavy_tiles
                matrix-core utilisation on the heavy tiles alone: a 512-token
                call's routes to experts with 64 or more positions, plus the
                shared expert over those tokens
  mixed32       batched decode of 32 tokens on a layer with 2-bit gate/up
                and 4-bit down projections, uniform routing: tokens/s and GB/s
  stack43       a 43-layer stack of full-width layers decoding through one
                bounded arena (96 usable slots per layer, 4129 slots, 32.5 GB):
                the compiled SLRU planner (and LFU-decay) picks evictions on
                the host, or the same planner on the GPU (no per-layer host
                round trip), misses copied from pinned host memory;
                Zipf(1.1) routing with AR(1) cross-layer noise (rho 0.6);
                hit rate, bytes moved, tokens/s and host -> HBM GB/s
  cpu_baseline  the C oracle (oracle/expert_ref.c, OpenMP) on the host cores
                over a bounded sample of the same decode workload, on every
                core and on one; a stand-in for the reference's MLX-CPU path,
                which cannot run here

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
MFMA_PEAK_TFLOPS = 2500.0          # dense bf16
TRAFFIC_FILE = ROOT / "profiles" / "gateup_diag_kernel_decode_traffic.json"
# the decode step's first launch: router rows, gate/up + SwiGLU and the top-6
# selection in one kernel
GATEUP_KERNEL = "gateup_diag_kernel<2, true, true, true>"
COPY_BYTES = 256 << 20
D, E, DFF, K_TOP, GROUP, BITS = 4096, 256, 2048, 6, 64, 2


def proj_bytes(rows, cols, bits=BITS, group=GROUP):
    return rows * cols * bits // 8 + 2 * 2 * rows * (cols // group)


EXPERT_BYTES = 2 * proj_bytes(DFF, D) + proj_bytes(D, DFF)          # 7,864,320
# the real checkpoint's 2-bit experts come in groups of 128
G128_EXPERT_BYTES = 2 * proj_bytes(DFF, D, group=128) + proj_bytes(D, DFF, group=128)   # 7,077,888
MIXED_EXPERT_BYTES = 2 * proj_bytes(DFF, D) + proj_bytes(D, DFF, bits=4)   # 9,961,472
# the checkpoint's DSpark/MTP tier: 3-bit experts in groups of 128
B3_EXPERT_BYTES = 2 * proj_bytes(DFF, D, bits=3, group=128) + proj_bytes(D, DFF, bits=3, group=128)   # 10,223,616
GATEUP_ROUTE_BYTES = 2 * proj_bytes(DFF, D)                           # 5,242,880
ROUTER_BYTES = E * D * 2
# copula correlation between the next layer's gate applied to the current
# input and that layer's own routing logits (the stack's lookahead); 0.9
# puts about two thirds of a lookahead top-6 among the next layer's top-6
LOOKAHEAD_RHO = 0.9
# per decode gate/up launch: 7 routes' gate+up slots, x read once, h written
GATEUP_ALG_BYTES = (K_TOP + 1) * GATEUP_ROUTE_BYTES + D * 2 + (K_TOP + 1) * DFF * 2   # 36,737,024
# the decode step's gate/up kernel also reads the token's logits and writes its
# routes (expert, weight, slot)
SELECT_ALG_BYTES = GATEUP_ALG_BYTES + E * 4 + 3 * K_TOP * 4                            # 36,738,120
# ... and with its router rows it reads the router weight and hands the logits
# over itself (one 8-byte tagged word per expert written; the routes read them)
STEP_GATEUP_ALG_BYTES = GATEUP_ALG_BYTES + ROUTER_BYTES + E * 8 + 3 * K_TOP * 4         # 38,836,296


def layer_flops(tokens):
    """Multiply-adds x 2 of the routed and shared experts for `tokens` tokens."""
    return 2 * tokens * (K_TOP + 1) * 3 * D * DFF


# The decode leg rotates its steps over this many copies of the layer's router
# and shared expert (as a model's layers each have their own): 64 x 9.96 MB
# is well past the 256 MB MALL, so every step reads its router and shared
# expert from HBM like its routed experts, instead of re-reading one copy.
DECODE_LAYERS = 64


def layer(dev, seed=1):
    arena = synth.expert_arena(E + 1, D, DFF, bits_gate_up=BITS, group=GROUP, dtype=torch.bfloat16,
                               seed=seed, device=dev)
    shared = synth.expert_arena(1, D, DFF, bits_gate_up=BITS, group=GROUP, dtype=torch.bfloat16,
                                seed=seed + 1, device=dev, zero_slot=False)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=dev)
    return arena, shared, slot_of


def decode_layers(dev, seed, shared0, spec0, n=DECODE_LAYERS):
    """n (router, shared expert) pairs; the first are the layer's own."""
    specs, shareds = [spec0], [shared0]
    for i in range(1, n):
        shareds.append(synth.expert_arena(1, D, DFF, bits_gate_up=BITS, group=GROUP, dtype=torch.bfloat16,
                                          seed=seed + 1000 + 2 * i, device=dev, zero_slot=False))
        w, _ = synth.uniform_router(E, D, torch.bfloat16, seed=seed + 1001 + 2 * i, device=dev)
        specs.append(ops.RouterSpec(w, K_TOP, routed_scale=1.5))
    return specs, shareds


def decode_graph_run(specs, arena, shareds, slot_of, X, ws, steps, warmup, use_graph):
    """Returns elapsed seconds for exactly `steps` decode steps (step j uses
    router and shared expert j % len(specs))."""
    n_in = X.shape[0]
    outs = torch.empty_like(X)
    idx = torch.empty(n_in, K_TOP, dtype=torch.int32, device=X.device)
    wts = torch.empty(n_in, K_TOP, dtype=torch.float32, device=X.device)

    def step(i):
        j = i % n_in
        ops.forward(specs[j % len(specs)], arena, shareds[j % len(specs)], slot_of, X[j:j + 1], ws,
                    out=outs[j:j + 1],
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


def stage_timing(specs, arena, shareds, slot_of, X, ws, m=40, replays=5):
    """Average device time (s) per launch of the decode step and of its
    kernels. The step (`decode_step`, locali_moe_forward) is two launches:
    gateup_diag_kernel<2, true, true, true> -- router rows, gate/up + SwiGLU
    and the top-6 selection -- then down_combine_kernel. The first cannot run
    alone (its router rows tag the logits with a generation the down kernel
    advances), so its average is the step's less the down kernel's
    (`gateup_router_select`). Also timed, for reference: the separate stages
    of the same step (router logits kernel, gate/up selecting from those
    logits, the gate/up kernel fed with chosen routes).

    Each stage is captured m times back to back (inputs 0..m-1, so every
    launch streams different experts) into its own HIP graph; HIP events on
    the replay stream bracket `replays` replays, and the per-launch average
    is elapsed / (replays * m) -- the same quantity rocprofv3 reports as a
    kernel's average duration (plus the launch gap). Launch i uses router
    and shared expert i % len(specs), as the decode leg does."""
    dev = X.device
    nl = len(specs)
    n_in = X.shape[0]
    xs = [X[i % n_in:i % n_in + 1] for i in range(m)]
    hidden = torch.empty(K_TOP + 1, DFF, dtype=torch.bfloat16, device=dev)
    out = torch.empty(1, D, dtype=torch.bfloat16, device=dev)
    dws = ops.Workspace(dev)
    dws.reserve(1, D, DFF, 1, K_TOP, True)
    routed = [ops.router(specs[i % nl], x, ws, slot_of_expert=slot_of, n_slots=E + 1) for i, x in enumerate(xs)]
    logits = [ops.router_logits(specs[i % nl], x) for i, x in enumerate(xs)]
    lbuf = torch.empty(E, dtype=torch.float32, device=dev)
    sel = [tuple(torch.empty(1, K_TOP, dtype=dt, device=dev) for dt in (torch.int32, torch.float32, torch.int32))
           for _ in range(m)]
    outs = torch.empty(m, D, dtype=torch.bfloat16, device=dev)
    sidx = torch.empty(m, K_TOP, dtype=torch.int32, device=dev)
    swts = torch.empty(m, K_TOP, dtype=torch.float32, device=dev)
    stages = {
        "decode_step": lambda i: ops.forward(specs[i % nl], arena, shareds[i % nl], slot_of, xs[i], ws,
                                             out=outs[i:i + 1], idx=sidx[i:i + 1], weights=swts[i:i + 1]),
        "router_logits": lambda i: ops.router_logits(specs[i % nl], xs[i], lbuf),
        "gateup_select": lambda i: ops.decode_gateup_select(specs[i % nl], arena, shareds[i % nl], slot_of, xs[i],
                                                            logits[i], hidden, dws, idx=sel[i][0],
                                                            weights=sel[i][1], route_slot=sel[i][2]),
        "down_combine": lambda i: ops.decode_down_combine(arena, shareds[i % nl], routed[i][2], routed[i][1],
                                                          out, dws),
        "gateup_chosen_routes": lambda i: ops.decode_gateup(arena, shareds[i % nl], xs[i], routed[i][2], hidden,
                                                            dws),
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
    res["gateup_router_select"] = res["decode_step"] - res["down_combine"]
    return res


def prefill_run(arena, shared, slot_of, dev, tokens, calls, seed, expert_bytes=EXPERT_BYTES):
    """Zipf(1.1) routing through the real router (x . Wg == Zipf logits);
    expert_bytes: bytes of one expert in the arena's format."""
    batches = []
    for c in range(calls):
        x, w = synth.zipf_router_inputs(tokens, E, D, 1.1, torch.bfloat16, seed=seed + c, device=dev)
        batches.append(x)
    spec = ops.RouterSpec(w, K_TOP, routed_scale=1.5)
    ws = ops.Workspace(dev)
    out = torch.empty(tokens, D, dtype=torch.bfloat16, device=dev)
    idx = torch.empty(tokens, K_TOP, dtype=torch.int32, device=dev)
    wts = torch.empty(tokens, K_TOP, dtype=torch.float32, device=dev)
    # one untimed pass over the same calls first: the timed pass then sees
    # the steady state of a serving loop (address translation of the arena's
    # pages and clocks warm after the legs before it), not a cold start
    for x in batches:
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
    algo = (u + 1) * expert_bytes + ROUTER_BYTES + tokens * D * 2 * 2
    per_call = secs / calls
    flops = layer_flops(tokens)
    t_roof = max(algo / (HBM_PEAK_GBS * 1e9), flops / (MFMA_PEAK_TFLOPS * 1e12))
    return {"tokens": tokens, "calls": calls, "value": tokens * calls / secs, "unit": "tokens/s",
            "ms_per_call": per_call * 1e3, "distinct_experts": u,
            "algorithmic_bytes_per_call": int(algo),
            "achieved_GBps": algo / per_call / 1e9, "frac_of_hbm_peak": algo / per_call / 1e9 / HBM_PEAK_GBS,
            "flops_per_call": flops, "achieved_TFLOPs": flops / per_call / 1e12,
            "mfma_utilisation": flops / per_call / 1e12 / MFMA_PEAK_TFLOPS,
            "roofline_frac": t_roof / per_call}


def mixed_run(dev, tokens, calls, seed):
    """Batched decode on a 2-bit gate/up, 4-bit down layer, uniform routing."""
    arena = synth.expert_arena(E + 1, D, DFF, bits_gate_up=2, bits_down=4, group=GROUP,
                               dtype=torch.bfloat16, seed=seed, device=dev)
    shared = synth.expert_arena(1, D, DFF, bits_gate_up=2, bits_down=4, group=GROUP,
                                dtype=torch.bfloat16, seed=seed + 1, device=dev, zero_slot=False)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=dev)
    w, _ = synth.uniform_router(E, D, torch.bfloat16, seed=seed + 2, device=dev)
    spec = ops.RouterSpec(w, K_TOP, routed_scale=1.5)
    ws = ops.Workspace(dev)
    xs = [synth.activations(tokens, D, torch.bfloat16, seed=seed + 10 + c, device=dev)
          for c in range(calls)]
    out = torch.empty(tokens, D, dtype=torch.bfloat16, device=dev)
    idx = torch.empty(tokens, K_TOP, dtype=torch.int32, device=dev)
    wts = torch.empty(tokens, K_TOP, dtype=torch.float32, device=dev)
    for x in xs:                           # one untimed pass first (as prefill_run)
        ops.forward(spec, arena, shared, slot_of, x, ws, out=out, idx=idx, weights=wts)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for x in xs:
        ops.forward(spec, arena, shared, slot_of, x, ws, out=out, idx=idx, weights=wts)
    e1.record()
    torch.cuda.synchronize()
    secs = e0.elapsed_time(e1) / 1e3
    distinct = [int(torch.unique(ops.router(spec, x, ws)[0]).numel()) for x in xs]
    u = sum(distinct) / len(distinct)
    per_call = secs / calls
    algo = (u + 1) * MIXED_EXPERT_BYTES + ROUTER_BYTES + tokens * D * 2 * 2
    del arena, shared
    torch.cuda.empty_cache()
    return {"tokens": tokens, "calls": calls, "value": tokens * calls / secs, "unit": "tokens/s",
            "ms_per_call": per_call * 1e3, "distinct_experts": u,
            "expert_bytes": MIXED_EXPERT_BYTES, "algorithmic_bytes_per_call": int(algo),
            "achieved_GBps": algo / per_call / 1e9, "frac_of_hbm_peak": algo / per_call / 1e9 / HBM_PEAK_GBS,
            "workload": "d_model 4096, 256 experts top-6 + shared, d_ff 2048, gate/up 2-bit + "
                        "down 4-bit affine g64 bf16, 32 tokens per call, uniform routing"}


def stack_run(dev, steps, warmup, policy, seed, layers=43, per_layer=96, prefetch_k=None,
              lookahead_rho=LOOKAHEAD_RHO, device_planner=False, mark=None):
    """Decode through a stack of full-width layers sharing one bounded arena,
    misses copied from pinned host memory (V4ArenaStore host_source).

    Even layers' gates read the routing logits from x[:, :E], odd layers'
    from x[:, E:2E]; a layer's input carries its own logits in its slice and,
    in the other, a lookahead view of the next layer's logits (Gumbel noise
    with copula correlation lookahead_rho to that layer's), which is what the
    next layer's gate sees when it is applied to the current input.

    prefetch_k: each layer also routes its input through the next layer's
    gate and prefetches that call's prefetch_k highest-weight experts
    (cross-layer prefetch at depth 1).

    device_planner: the planner runs on the GPU (same decisions), so a
    layer's router, planner, fills and expert kernels queue on the stream
    with no per-layer host round trip.

    mark(suffix): called (after a device synchronize) when the timed tokens
    start and when they end, for the bench's phase log."""
    import tempfile
    from locali_amd.dsv4_arena import V4ArenaMoE, V4ArenaStore, V4Gate
    tmp = tempfile.TemporaryDirectory()
    index = Path(tmp.name) / "stack.idx"
    index.write_text(json.dumps(synth.stack_index(layers, E, K_TOP, D, DFF, bits=BITS, group=GROUP)))
    payload = synth.expert_arena(E, D, DFF, bits_gate_up=BITS, group=GROUP, dtype=torch.bfloat16,
                                 seed=seed, device=dev, zero_slot=False)
    host = synth.host_payloads(payload)          # 256 distinct experts, pinned
    del payload
    n_slots = layers * per_layer + 1
    store = V4ArenaStore(index, ceiling_gb=n_slots * EXPERT_BYTES / 1e9 + 1e-6, threads=1,
                         cache_policy=policy, device=dev, device_planner=device_planner,
                         host_source=lambda layer, e: host[e])
    shared = synth.expert_arena(layers, D, DFF, bits_gate_up=BITS, group=GROUP, dtype=torch.bfloat16,
                                seed=seed + 1, device=dev, zero_slot=False)

    def shared_of(layer):
        return ops.ExpertArenaT(*(ops.ProjArena(p.weight[layer:layer + 1], p.scales[layer:layer + 1],
                                                p.biases[layer:layer + 1], p.bits, p.group_size)
                                  for p in (shared.gate, shared.up, shared.down)))

    w_even = synth.identity_router(E, D, torch.bfloat16, dev)
    gates = [V4Gate(w, top_k=K_TOP, routed_scaling_factor=1.5)
             for w in (w_even, torch.roll(w_even, E, dims=1).contiguous())]
    mods = [V4ArenaMoE(store, layer, gates[layer % 2], K_TOP, shared_expert=shared_of(layer))
            for layer in range(layers)]
    if prefetch_k:
        for cur, nxt in zip(mods, mods[1:]):
            cur.nxt, cur.prefetch_k = nxt, prefetch_k
    n_tok = warmup + steps
    X = synth.activations(n_tok * layers, D, torch.bfloat16, seed=seed + 2, device=dev).view(n_tok, layers, D)
    logits, ahead = synth.layered_zipf_lookahead(n_tok, layers, E, 1.1, 0.6, lookahead_rho, seed=seed + 3)
    for layer in range(layers):
        own = (layer % 2) * E
        X[:, layer, own:own + E] = logits[:, layer].to(dev, torch.bfloat16)
        if layer + 1 < layers:
            other = E - own
            X[:, layer, other:other + E] = ahead[:, layer].to(dev, torch.bfloat16)
    # how often a lookahead top-j expert is among the next layer's top-k
    # (timed tokens; bf16 rounding of the inputs aside)
    act = logits[warmup:, 1:].topk(K_TOP, dim=-1).indices
    precision = {j: (ahead[warmup:].topk(j, dim=-1).indices.unsqueeze(-1) == act.unsqueeze(-2))
                 .any(-1).float().mean().item() for j in sorted({1, 3, K_TOP, prefetch_k or K_TOP})}
    # The layers run on a stream of their own: on this runtime a launch on
    # the legacy default stream waits on the host for a running kernel that
    # reads host memory on another stream (the prefetch's fills).
    compute = torch.cuda.Stream(device=dev)
    compute.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(compute):
        for t in range(warmup):
            for layer in range(layers):
                mods[layer](X[t, layer:layer + 1])
    torch.cuda.synchronize()
    store.reset_stats()
    if mark:
        mark("timed tokens")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(compute):
        e0.record()
        for t in range(warmup, n_tok):
            for layer in range(layers):
                mods[layer](X[t, layer:layer + 1])
        e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if mark:
        mark("teardown")
    secs = e0.elapsed_time(e1) / 1e3
    st = store.stats()
    store.close()
    del store, shared, host, mods
    tmp.cleanup()
    torch.cuda.empty_cache()
    moved = st["bytes_read"]
    return {"layers": layers, "slots": n_slots, "usable_slots_per_layer": per_layer,
            "arena_GB": n_slots * EXPERT_BYTES / 1e9, "cache_policy": policy,
            "planner": "device" if device_planner else "host",
            "prefetch": (None if not prefetch_k else
                         {"depth": 1, "top": prefetch_k, "prefetched": st["prefetched"],
                          "used": st["prefetch_used"], "wasted": st["prefetch_wasted"]}),
            "lookahead": {"rho": lookahead_rho,
                          "precision_at": {str(j): round(p, 4) for j, p in precision.items()}},
            "steps": steps, "warmup_tokens": warmup, "value": steps / secs, "unit": "tokens/s",
            "ms_per_token": secs / steps * 1e3, "wall_s": wall, "hit_rate": st["hit_rate"],
            "hits": st["hits"], "misses": st["misses"], "evictions": st["evictions"],
            "h2d_bytes": moved, "h2d_bytes_per_token": moved / steps,
            "h2d_GBps": moved / secs / 1e9, "host_stall_s": st["t_stall"],
            "hbm_expert_bytes_per_token": layers * (K_TOP + 1) * EXPERT_BYTES + layers * ROUTER_BYTES,
            "demand_miss_bytes_per_token": st["misses"] * EXPERT_BYTES / steps,
            "workload": "43 full-width layers (d 4096, 256 experts top-6 + shared, d_ff 2048, 2-bit "
                        "g64), one arena of 43 x 96 + 1 slots, Zipf(1.1) routing with a per-layer "
                        "expert ranking and AR(1) cross-layer noise rho 0.6, misses from pinned host "
                        "memory (256 distinct expert payloads; expert e of every layer copies "
                        f"payload e); next-layer gate on the current input sees the next layer's "
                        f"logits through copula noise of correlation {lookahead_rho}"}


DOWN_ROUTE_BYTES = proj_bytes(D, DFF)                                 # 2,621,440


def streaming_floor_run(dev, m=40, replays=5, rotate=16):
    """The decode step's memory traffic with nothing else: per step three
    dependent launches of locali_moe_stream_read (16-byte non-temporal loads,
    no arithmetic) over the router's 2 MiB, the 7 routes' gate/up bytes and
    the 7 routes' down bytes, each from its own buffer; steps rotate over
    `rotate` buffer sets (914 MB, far past the 256 MB MALL) so every read is
    cold, as the decode leg's are. Graphs of m steps (and of m launches of
    each stage alone) are timed with HIP events on the replay stream."""
    from locali_amd import _lib
    lib = _lib.lib()
    sizes = {"router": ROUTER_BYTES, "gateup": (K_TOP + 1) * GATEUP_ROUTE_BYTES,
             "down": (K_TOP + 1) * DOWN_ROUTE_BYTES}
    bufs = [{k: torch.empty(v, dtype=torch.uint8, device=dev) for k, v in sizes.items()} for _ in range(rotate)]
    sink = torch.zeros(65535, dtype=torch.int32, device=dev)

    def launch(buf):
        blocks = min(65535, (buf.numel() // 16 + 1023) // 1024)
        _lib.check(lib.locali_moe_stream_read(buf.data_ptr(), buf.numel(), sink.data_ptr(), blocks, ops._stream()),
                   "locali_moe_stream_read")

    def timed(fn):
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
        return e0.elapsed_time(e1) / 1e3 / (replays * m)

    def step(i):
        for k in ("router", "gateup", "down"):
            launch(bufs[i % rotate][k])

    out = {"step_us": timed(step) * 1e6}
    for k in sizes:
        t = timed(lambda i, k=k: launch(bufs[i % rotate][k]))
        out[f"{k}_us"] = t * 1e6
        out[f"{k}_GBps"] = sizes[k] / t / 1e9
    out["bytes_per_step"] = sum(sizes.values())
    out["step_GBps"] = out["bytes_per_step"] / (out["step_us"] * 1e-6) / 1e9
    out["workload"] = ("three dependent streaming reads per step (router 2 MiB, 7 routes' gate/up "
                       "36.7 MB, 7 routes' down 18.4 MB), cold buffers, no arithmetic")
    del bufs
    torch.cuda.empty_cache()
    return out


def decode_format_run(specs, X, dev, steps, warmup, use_graph, seed, bits, group, expert_bytes, workload):
    """The decode leg on experts of another format (`bits`-bit codes in
    groups of `group`, expert_bytes per expert): same router copies, inputs
    and step as the headline leg, one shared expert of that format per
    router copy."""
    arena = synth.expert_arena(E + 1, D, DFF, bits_gate_up=bits, group=group, dtype=torch.bfloat16,
                               seed=seed, device=dev)
    shareds = [synth.expert_arena(1, D, DFF, bits_gate_up=bits, group=group, dtype=torch.bfloat16,
                                  seed=seed + 1000 + 2 * i, device=dev, zero_slot=False) for i in range(len(specs))]
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=dev)
    ws = ops.Workspace(dev)
    ws.reserve(1, D, DFF, E, K_TOP, True)
    secs, wall, _ = decode_graph_run(specs, arena, shareds, slot_of, X, ws, steps, warmup, use_graph)
    del arena, shareds
    torch.cuda.empty_cache()
    layer = 7 * expert_bytes + ROUTER_BYTES
    value = steps / secs
    return {"value": value, "unit": "tokens/s", "ms_per_step": secs / steps * 1e3, "steps": steps,
            "expert_bytes": expert_bytes, "layer_bytes_per_token": layer,
            "layer_GBps": layer * value / 1e9, "layer_frac_of_hbm_peak": layer * value / 1e9 / HBM_PEAK_GBS,
            "workload": workload}


def heavy_tiles_run(arena, shared, slot_of, dev, tokens, calls, seed):
    """Matrix-core utilisation on the heavy tiles alone: the routes of one
    Zipf(1.1) call of `tokens` tokens whose expert has at least 64 positions,
    each as a one-route token (so every heavy expert keeps its tiles), plus
    the shared expert over those tokens (full 64-position tiles)."""
    x, w = synth.zipf_router_inputs(tokens, E, D, 1.1, torch.bfloat16, seed=seed, device=dev)
    spec = ops.RouterSpec(w, K_TOP, routed_scale=1.5)
    ws = ops.Workspace(dev)
    idx, _, _ = ops.router(spec, x, ws)
    counts = torch.bincount(idx.reshape(-1).long(), minlength=E)
    heavy = (counts >= 64).nonzero().reshape(-1)
    sel = torch.isin(idx.long(), heavy)
    tok = sel.nonzero()[:, 0]
    xh = x[tok].contiguous()
    ih = idx[sel].reshape(-1, 1).contiguous()
    n = xh.shape[0]
    ones = torch.ones(n, 1, device=dev)
    for _ in range(2):
        ops.expert_grouped(arena, shared, xh, ih, slot_of, ones, ws, n_experts=E)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(calls):
        ops.expert_grouped(arena, shared, xh, ih, slot_of, ones, ws, n_experts=E)
    e1.record()
    torch.cuda.synchronize()
    per_call = e0.elapsed_time(e1) / 1e3 / calls
    flops = 2 * (2 * n) * 3 * D * DFF            # n routed routes + n shared routes
    tiles = int(sum((int(c) + 63) // 64 for c in counts[heavy].tolist())) + (n + 63) // 64
    return {"from_tokens": tokens, "heavy_experts": int(heavy.numel()),
            "positions_per_heavy_expert": sorted(counts[heavy].tolist(), reverse=True),
            "routes": 2 * n, "tiles": tiles, "ms_per_call": per_call * 1e3,
            "achieved_TFLOPs": flops / per_call / 1e12,
            "mfma_utilisation": flops / per_call / 1e12 / MFMA_PEAK_TFLOPS,
            "bytes_per_call": int((heavy.numel() + 1) * EXPERT_BYTES),
            "frac_of_hbm_peak": (heavy.numel() + 1) * EXPERT_BYTES / per_call / 1e9 / HBM_PEAK_GBS}


def cpu_baseline(arena, shared, spec, X, seconds):
    """C oracle on the host cores, decode tokens until `seconds` elapse on
    every core, then for half as long on one core."""
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

    def timed(threads, budget):
        ref.set_threads(threads)
        n = 0
        t0 = time.perf_counter()
        while True:
            x = xs[n % xs.shape[0]:n % xs.shape[0] + 1]
            idx, w = ref.router(x, wg, None, K_TOP, 0, True, spec.routed_scale)
            ref.moe_layer(x, idx + 1, w, ha, "bf16", shared=hs)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget and n >= 2:
                return n, el

    cores = len(os.sched_getaffinity(0))
    threads = min(int(os.environ.get("OMP_NUM_THREADS", "0")) or cores, cores)
    n, el = timed(threads, seconds)
    n1, el1 = timed(1, seconds / 2)
    ref.set_threads(0)
    return {"value": n / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "one_core": {"value": n1 / el1, "unit": "tokens/s", "cores": 1,
                         "sample": f"{n1} decode tokens, {el1:.1f} s"},
            "sample": f"{n} decode tokens of the same layer (router + 6 routed + shared experts), "
                      f"{el:.1f} s on {threads} threads, C oracle oracle/expert_ref.c with OpenMP; "
                      "stand-in for the reference dsv4_arena path on MLX's CPU backend (not "
                      "runnable here)"}


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
        # the reference launches are the run's only ones of this name that
        # count at least a quarter of COPY_BYTES (other fills and
        # reductions of the run are far smaller)
        refs = [float(r["Counter_Value"]) for r in rows
                if ref_name in r["Kernel_Name"] and int(r["Grid_Size"]) >= 1 << 16
                and float(r["Counter_Value"]) >= COPY_BYTES / 1024 / 4]
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
           "algorithmic_bytes_per_launch": STEP_GATEUP_ALG_BYTES}
    Path(out_path).write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res, indent=1))
    return res


def summarize_trace(trace_csv, phases_json):
    """Per-phase kernel table (markdown) from a rocprofv3 --kernel-trace CSV of
    a run made with --phase-log: kernels are assigned to the bench phase
    whose [start, next start) window holds their start timestamp (both
    clocks are CLOCK_MONOTONIC nanoseconds).

    Each phase also gets the occupancy of the library's kernels over their
    span (first start to last end): the time some host-to-HBM copy launch
    (the fill kernels and the device planner's plan-and-copy launch) is
    running, the time any library kernel is running, and the time no copy
    launch is running."""
    import csv
    marks = json.loads(Path(phases_json).read_text())["phases"]
    bounds = [(name, t0, marks[i + 1][1] if i + 1 < len(marks) else float("inf"))
              for i, (name, t0) in enumerate(marks)]
    per = {name: {} for name, _, _ in bounds}
    spans = {name: {"copy": [], "all": [], "wide": [], "small": [], "combine": 0} for name, _, _ in bounds}
    unassigned = 0
    for r in csv.DictReader(open(trace_csv)):
        t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        name = r["Kernel_Name"].replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")
        for ph, a, b in bounds:
            if a <= t0 < b:
                per[ph].setdefault(name, []).append((t1 - t0) / 1e3)
                if "locali" in name or "dplan" in name:
                    spans[ph]["all"].append((t0, t1))
                    if "fill_kernel" in name or "dplan_kernel<true>" in name:
                        spans[ph]["copy"].append((t0, t1))
                    if "wide_" in name:
                        spans[ph]["wide"].append((t0, t1))
                    elif "_small" in name:
                        spans[ph]["small"].append((t0, t1))
                    elif "combine8" in name:
                        spans[ph]["combine"] += 1
                break
        else:
            unassigned += 1

    def union(iv):
        tot, end = 0, None
        for a, b in sorted(iv):
            if end is None or a > end:
                tot += b - a
                end = b
            elif b > end:
                tot += b - end
                end = b
        return tot

    out = []
    for ph, _, _ in bounds:
        ks = per[ph]
        if not ks:
            continue
        total = sum(sum(v) for v in ks.values())
        out += [f"### {ph}", ""]
        iv = spans[ph]
        if iv["copy"]:
            span = max(b for _, b in iv["all"]) - min(a for a, _ in iv["all"])
            cu, au = union(iv["copy"]), union(iv["all"])
            out += [f"Library kernels span {span / 1e6:.2f} ms: a host-to-HBM copy launch runs {cu / 1e6:.2f} ms "
                    f"({100 * cu / span:.1f} %), some library kernel {au / 1e6:.2f} ms ({100 * au / span:.1f} %); "
                    f"no copy launch runs for {(span - cu) / 1e6:.2f} ms ({100 * (span - cu) / span:.1f} %).", ""]
        if iv["wide"] and iv["small"] and iv["combine"]:
            # grouped calls (one combine each): kernel time against the time
            # some library kernel runs, and the time a 64-position and a
            # small-tile kernel run together (the second stream's overlap)
            n = iv["combine"]
            both = union(iv["wide"]) + union(iv["small"]) - union(iv["wide"] + iv["small"])
            ksum = sum(b - a for a, b in iv["all"])
            out += [f"Grouped calls: {n}; library kernel time {ksum / n / 1e3:.1f} us per call, some library kernel "
                    f"running {union(iv['all']) / n / 1e3:.1f} us per call, a 64-position and a small-tile kernel "
                    f"running together {both / n / 1e3:.1f} us per call.", ""]
        out += ["| kernel | calls | avg us | min us | max us | share of phase kernel time |",
                "|---|---:|---:|---:|---:|---:|"]
        for name, v in sorted(ks.items(), key=lambda kv: -sum(kv[1])):
            if "locali" not in name and sum(v) < 0.01 * total:
                continue
            out.append(f"| `{name[:90]}` | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
                       f"{100 * sum(v) / total:.1f}% |")
        out.append("")
    out.append(f"({unassigned} dispatches outside the logged phases)")
    print("\n".join(out))


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
    ap.add_argument("--prefill-sizes", default="64,512", help="tokens per prefill call, comma-separated")
    ap.add_argument("--skip-mixed", action="store_true")
    ap.add_argument("--skip-g128", action="store_true")
    ap.add_argument("--skip-3bit", action="store_true")
    ap.add_argument("--skip-heavy", action="store_true")
    ap.add_argument("--skip-stack", action="store_true")
    ap.add_argument("--stack-steps", type=int, default=128)
    ap.add_argument("--stack-warmup", type=int, default=16)
    ap.add_argument("--stack-policies", default="slru-all,lfu-decay",
                    help="comma-separated arena cache policies for the 43-layer stack")
    ap.add_argument("--stack-prefetch", default="5",
                    help="comma-separated prefetch widths for extra slru-all stack legs with "
                         "cross-layer prefetch at depth 1 (0: none)")
    ap.add_argument("--stack-device-prefetch", default="1,5",
                    help="comma-separated prefetch widths for extra slru-all stack legs planned on the GPU "
                         "with cross-layer prefetch at depth 1 (0: none)")
    ap.add_argument("--stack-device-planner", default="slru-all,lfu-decay",
                    help="comma-separated cache policies for extra stack legs planned on the GPU")
    ap.add_argument("--stack-lookahead-rho", type=float, default=LOOKAHEAD_RHO,
                    help="correlation of the stack's lookahead routing with the next layer's")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run 256 MiB read and write reference kernels first (for --pmc byte counters)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc runs into HBM bytes per gate/up launch")
    ap.add_argument("--phase-log", metavar="JSON",
                    help="write the start time (CLOCK_MONOTONIC ns) of every bench phase")
    ap.add_argument("--summarize-trace", nargs=2, metavar=("TRACE_CSV", "PHASES_JSON"),
                    help="per-phase kernel table of a rocprofv3 kernel trace of a --phase-log run")
    args = ap.parse_args(argv)
    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return 0
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace)
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
    marks = []

    def phase(name):
        torch.cuda.synchronize()
        marks.append((name, time.monotonic_ns()))
        print(f"[bench] {name}", file=sys.stderr, flush=True)

    phase("setup")
    if args.copy_calibration:
        copy_calibration(dev)
    arena, shared, slot_of = layer(dev, args.seed)
    w, _ = synth.uniform_router(E, D, torch.bfloat16, seed=args.seed + 2, device=dev)
    spec = ops.RouterSpec(w, K_TOP, routed_scale=1.5)
    n_inputs = 200   # 200 distinct tokens x 57 MB per step >> 256 MB MALL
    X = synth.activations(n_inputs, D, torch.bfloat16, seed=args.seed + 3, device=dev)
    ws = ops.Workspace(dev)
    ws.reserve(1, D, DFF, E, K_TOP, True)

    specs, shareds = decode_layers(dev, args.seed, shared, spec)

    phase("decode (graph replay)")
    secs, wall, idx = decode_graph_run(specs, arena, shareds, slot_of, X, ws, args.steps, args.warmup,
                                       not args.no_graph)
    value = args.steps / secs
    layer_bytes = 7 * EXPERT_BYTES + ROUTER_BYTES

    phase("stage timing (decode step, down + combine, separate stages)")
    st = stage_timing(specs, arena, shareds, slot_of, X, ws)
    gate_bytes = STEP_GATEUP_ALG_BYTES
    achieved = gate_bytes / st["gateup_router_select"] / 1e9
    phase("streaming floor of the decode step (three dependent streaming reads)")
    floor = streaming_floor_run(dev)
    g128 = b3 = None
    if not args.skip_g128:
        phase("decode, experts in groups of 128 (graph replay)")
        g128 = decode_format_run(specs, X, dev, args.steps, args.warmup, not args.no_graph, args.seed + 50,
                                 BITS, 128, G128_EXPERT_BYTES,
                                 "the headline decode layer with 2-bit affine experts in groups of 128 "
                                 "(bf16 scales/biases), the real checkpoint's expert layout")
    if not args.skip_3bit:
        phase("decode, 3-bit experts in groups of 128 (graph replay)")
        b3 = decode_format_run(specs, X, dev, args.steps, args.warmup, not args.no_graph, args.seed + 60,
                               3, 128, B3_EXPERT_BYTES,
                               "the headline decode layer with 3-bit affine experts in groups of 128 "
                               "(bf16 scales/biases), the checkpoint's DSpark/MTP tier layout")
    del specs, shareds
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
                        "slots resident in HBM, 1 token per step, uniform-random routing; steps "
                        f"rotate over {DECODE_LAYERS} copies of the router and shared expert "
                        "(cold in the MALL, as a model's layers)",
            "tokens_per_step": 1,
            "router_shared_copies": DECODE_LAYERS,
            "graph_replay": not args.no_graph,
            "wall_s": wall,
            "layer_bytes_per_token": layer_bytes,
            "layer_GBps": layer_bytes * value / 1e9,
            "layer_frac_of_hbm_peak": layer_bytes * value / 1e9 / HBM_PEAK_GBS,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{GATEUP_KERNEL}: the decode step's first launch -- the shared expert's "
                      "workgroups compute the router logits first (2 MiB gate), then the gate/up + clamped "
                      "SwiGLU of 7 routes on the matrix cores, each routed workgroup selecting its "
                      "token's top-6 from the logits",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(),
            "algorithmic_bytes_per_launch": gate_bytes,
            "avg_launch_us": st["gateup_router_select"] * 1e6,
            "measured_as": "decode_step - down_combine: HIP events around graphs of 40 back-to-back launches",
            "stage_us": {k: v * 1e6 for k, v in st.items()},
            "chosen_routes_variant": {
                "kernel": "gateup_diag_kernel<2, true, false, false> (the same kernel fed with chosen routes)",
                "avg_launch_us": st["gateup_chosen_routes"] * 1e6,
                "achieved": GATEUP_ALG_BYTES / st["gateup_chosen_routes"] / 1e9,
                "frac": GATEUP_ALG_BYTES / st["gateup_chosen_routes"] / 1e9 / HBM_PEAK_GBS},
        },
    }
    result["decode_streaming_floor"] = floor
    if g128 is not None:
        result["decode_g128"] = g128
    if b3 is not None:
        result["decode_3bit_g128"] = b3
    if not args.skip_prefill:
        for tokens in (int(v) for v in args.prefill_sizes.split(",")):
            phase(f"prefill {tokens} tokens")
            result[f"prefill{tokens}"] = prefill_run(arena, shared, slot_of, dev, tokens,
                                                     args.prefill_calls, args.seed + 100)
        if not args.skip_3bit:
            a3 = synth.expert_arena(E + 1, D, DFF, bits_gate_up=3, group=128, dtype=torch.bfloat16,
                                    seed=args.seed + 61, device=dev)
            s3 = synth.expert_arena(1, D, DFF, bits_gate_up=3, group=128, dtype=torch.bfloat16,
                                    seed=args.seed + 62, device=dev, zero_slot=False)
            for tokens in (int(v) for v in args.prefill_sizes.split(",")):
                phase(f"prefill {tokens} tokens, 3-bit experts in groups of 128")
                result[f"prefill{tokens}_3bit_g128"] = prefill_run(a3, s3, slot_of, dev, tokens, args.prefill_calls,
                                                                   args.seed + 100, B3_EXPERT_BYTES)
            del a3, s3
            torch.cuda.empty_cache()
        if not args.skip_heavy:
            phase("heavy tiles of a 512-token prefill")
            result["prefill512_heavy_tiles"] = heavy_tiles_run(arena, shared, slot_of, dev, 512,
                                                               args.prefill_calls, args.seed + 100)
    if not args.skip_mixed:
        phase("mixed 2/4-bit, 32 tokens")
        result["mixed32"] = mixed_run(dev, 32, args.prefill_calls, args.seed + 200)
    if not args.skip_stack:
        result["stack43"] = []
        def leg(label, policy, **kw):
            phase(label)
            result["stack43"].append(stack_run(dev, args.stack_steps, args.stack_warmup, policy, args.seed + 300,
                                               lookahead_rho=args.stack_lookahead_rho,
                                               mark=lambda what: phase(f"{label}: {what}"), **kw))

        for policy in (v for v in args.stack_policies.split(",") if v.strip()):
            leg(f"43-layer bounded arena, {policy}", policy)
        for policy in (v for v in args.stack_device_planner.split(",") if v.strip()):
            leg(f"43-layer bounded arena, {policy}, device planner", policy, device_planner=True)
        for k in (int(v) for v in args.stack_prefetch.split(",") if v.strip() and int(v)):
            leg(f"43-layer bounded arena, slru-all, prefetch top-{k} at depth 1", "slru-all", prefetch_k=k)
        for k in (int(v) for v in args.stack_device_prefetch.split(",") if v.strip() and int(v)):
            leg(f"43-layer bounded arena, slru-all, device planner, prefetch top-{k} at depth 1", "slru-all",
                prefetch_k=k, device_planner=True)
    if not args.skip_cpu:
        phase("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(arena, shared, spec, X, args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    phase("end")
    if args.phase_log:
        Path(args.phase_log).write_text(json.dumps({"phases": marks}) + "\n")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
