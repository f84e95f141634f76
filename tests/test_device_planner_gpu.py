"""Device-resident planner (locali_dplan_*) against the host planner.

The same call sequence goes through NativeCache.plan_each with the calling
convention of V4ArenaStore._place_keys (the previous demand call's slots
pinned, hits touched, the LFU token tick before layer-0 calls of at most
top_k experts) and through DevicePlanner.plan on the GPU; every per-key
result (key, slot, evicted key, hit, placed), every route's slot and the
counters must be identical. The host planner is pinned separately against
the reference planner's traces (test_planner_*.py), so equality here carries
that parity to the device. The fill kernel's copies are checked byte for
byte against the pinned payloads.
"""

import numpy as np
import pytest
import torch

from locali_amd.native import DevicePlanner, NativeCache

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def zipf_calls(rng, n_calls, layers, E, top_k, multi_every=0):
    """(layer, expert ids of one call's routes) with Zipf-skewed experts per
    layer; every multi_every-th call carries three tokens (duplicates)."""
    ranks = [rng.permutation(E) for _ in range(layers)]
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    calls = []
    for c in range(n_calls):
        layer = c % layers
        tokens = 3 if multi_every and c % multi_every == multi_every - 1 else 1
        routes = []
        for _ in range(tokens):
            routes.extend(int(ranks[layer][i]) for i in rng.choice(E, size=top_k, replace=False, p=p))
        calls.append((layer, routes))
    return calls


def host_run(calls, layers, E, slots, pcap, policy, top_k):
    cache = NativeCache(layers * E, slots, pcap, policy=policy)
    pinned = ()
    out = []
    for layer, routes in calls:
        want = list(dict.fromkeys(routes))
        if layer == 0 and len(want) <= top_k:
            cache.note_token()
        res = cache.plan_each([layer * E + e for e in want], pinned_slots=pinned, touch_hits=True)
        pinned = tuple(r.slot for r in res if r.placed)
        out.append(res)
    return out


@pytest.mark.parametrize("policy,slots,pcap,multi", [
    ("slru", 40, 12, 0),
    ("slru", 40, 0, 0),
    ("slru", 64, 20, 4),
    ("lfu-decay", 40, 0, 0),
    ("lfu-decay", 64, 0, 5),
])
def test_device_planner_matches_host_planner(policy, slots, pcap, multi):
    layers, E, top_k, n_calls = 5, 64, 6, 400
    rng = np.random.default_rng(slots * 7 + pcap + multi)
    calls = zipf_calls(rng, n_calls, layers, E, top_k, multi)
    expect = host_run(calls, layers, E, slots, pcap, policy, top_k)
    dp = DevicePlanner(layers * E, slots, pcap, n_experts=E, policy=policy, max_routes=64, device=DEV)
    hits = misses = evictions = 0
    for c, ((layer, routes), want_res) in enumerate(zip(calls, expect)):
        idx = torch.tensor(routes, dtype=torch.int32, device=DEV)
        rs = dp.plan(idx, layer, top_k)
        counters, got = dp.read(max_results=len(want_res))
        assert counters["error"] == 0, (c, counters)
        assert [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in got] == \
               [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in want_res], f"call {c} layer {layer}"
        slot_of = {r.key - layer * E: r.slot for r in want_res}
        assert rs.cpu().tolist() == [slot_of[e] for e in routes], f"route slots of call {c}"
        hits += sum(r.hit for r in want_res)
        misses += sum(not r.hit for r in want_res)
        evictions += sum(r.evicted_key >= 0 for r in want_res)
    counters, _ = dp.read()
    assert (counters["hits"], counters["misses"], counters["evictions"], counters["calls"]) == \
           (hits, misses, evictions, n_calls)
    assert evictions > 50        # the arena is small enough to churn


def test_device_planner_placement_failure_matches_host():
    """A tier with fewer unpinned slots than a call needs: the keys the host
    planner cannot place come back unplaced, their routes get slot 0 and the
    sticky error is set; the rest is identical."""
    layers, E, top_k = 2, 32, 6
    slots = 9                       # 8 usable: six pinned by the previous call leave two
    calls = [(0, [0, 1, 2, 3, 4, 5]), (1, [6, 7, 8, 9, 10, 11])]
    expect = host_run(calls, layers, E, slots, 0, "slru", top_k)
    assert not all(r.placed for r in expect[1])
    dp = DevicePlanner(layers * E, slots, 0, n_experts=E, policy="slru", max_routes=16, device=DEV)
    for (layer, routes), want_res in zip(calls, expect):
        rs = dp.plan(torch.tensor(routes, dtype=torch.int32, device=DEV), layer, top_k)
        counters, got = dp.read(max_results=len(want_res))
        assert [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in got] == \
               [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in want_res]
        placed = {r.key - layer * E: (r.slot if r.placed else 0) for r in want_res}
        assert rs.cpu().tolist() == [placed[e] for e in routes]
    assert counters["error"] == 2     # LOCALI_DPLAN_E_PLACE


@pytest.mark.parametrize("fused", [False, True])
def test_device_planner_fill_copies_each_miss(fused):
    """Three records per expert of unequal sizes; after every call each
    resident slot of the routed experts holds its expert's payload (fused:
    plan and copies in one launch)."""
    layers, E, top_k, slots = 3, 16, 4, 12
    sizes = [4096, 256, 1024]                   # bytes per slot of each record
    total = sum(sizes)
    payload = torch.randint(0, 256, (layers * E, total), dtype=torch.uint8).pin_memory()
    arrays = [torch.zeros(slots, s, dtype=torch.uint8, device=DEV) for s in sizes]
    table = ([a.data_ptr() for a in arrays], sizes)
    ptrs = DevicePlanner.host_view([payload[k].data_ptr() for k in range(layers * E)])
    host_src = torch.tensor(ptrs, dtype=torch.uint64, device=DEV)
    dp = DevicePlanner(layers * E, slots, 3, n_experts=E, policy="slru", max_routes=16, device=DEV)
    rng = np.random.default_rng(5)
    for c in range(60):
        layer = c % layers
        routes = [int(e) for e in rng.choice(E, size=top_k, replace=False)]
        idx = torch.tensor(routes, dtype=torch.int32, device=DEV)
        if fused:
            rs = dp.plan_fill(idx, layer, top_k, table, host_src)
        else:
            rs = dp.plan(idx, layer, top_k)
            dp.fill(table, host_src, layer, len(routes))
        got = torch.cat([a[rs.long()].cpu() for a in arrays], dim=1)
        want = payload[[layer * E + e for e in routes]]
        assert torch.equal(got, want), f"call {c}"
    counters, _ = dp.read()
    assert counters["error"] == 0 and counters["evictions"] > 0


@pytest.mark.parametrize("policy,multi", [("slru", 3), ("lfu-decay", 2)])
def test_fused_plan_fill_equals_plan_then_fill(policy, multi):
    """plan_fill against plan + fill on two planners fed the same calls
    (single-token calls and calls of several tokens, so several misses per
    call): per-key results, route slots, counters and every slot's bytes are
    identical, and the decisions equal the host planner's."""
    layers, E, top_k, slots, pcap = 4, 48, 6, 40, (10 if policy == "slru" else 0)
    sizes = [8192, 4096, 256]
    total = sum(sizes)
    payload = torch.randint(0, 256, (layers * E, total), dtype=torch.uint8).pin_memory()
    ptrs = DevicePlanner.host_view([payload[k].data_ptr() for k in range(layers * E)])
    host_src = torch.tensor(ptrs, dtype=torch.uint64, device=DEV)
    rng = np.random.default_rng(11 + multi)
    calls = zipf_calls(rng, 160, layers, E, top_k, multi)
    expect = host_run(calls, layers, E, slots, pcap, policy, top_k)
    planners, arenas = [], []
    for _ in range(2):
        arrays = [torch.zeros(slots, sz, dtype=torch.uint8, device=DEV) for sz in sizes]
        arenas.append((arrays, ([a.data_ptr() for a in arrays], sizes)))
        planners.append(DevicePlanner(layers * E, slots, pcap, n_experts=E, policy=policy, max_routes=64,
                                      device=DEV))
    n_multi_miss = 0
    for c, ((layer, routes), want_res) in enumerate(zip(calls, expect)):
        idx = torch.tensor(routes, dtype=torch.int32, device=DEV)
        rs_a = planners[0].plan(idx, layer, top_k)
        planners[0].fill(arenas[0][1], host_src, layer, len(routes))
        rs_b = planners[1].plan_fill(idx, layer, top_k, arenas[1][1], host_src)
        assert torch.equal(rs_a, rs_b), f"route slots of call {c}"
        ca, ra = planners[0].read(max_results=len(want_res))
        cb, rb = planners[1].read(max_results=len(want_res))
        assert ca == cb and cb["error"] == 0, (c, ca, cb)
        assert ra == rb == want_res, f"results of call {c}"
        for a, b in zip(arenas[0][0], arenas[1][0]):
            assert torch.equal(a, b), f"arena bytes after call {c}"
        got = torch.cat([a[rs_b.long()].cpu() for a in arenas[1][0]], dim=1)
        assert torch.equal(got, payload[[layer * E + e for e in routes]]), f"payload of call {c}"
        n_multi_miss += sum(not r.hit for r in want_res) > 1
    assert n_multi_miss > 20


@pytest.mark.parametrize("policy,slots,n_calls,tokens", [
    ("slru", 43 * 96 + 1, 43 * 14, (1, 1, 4, 16)),
    ("lfu-decay", 43 * 96 + 1, 43 * 14, (1, 1, 4, 16)),
    ("slru", 43 * 192 + 1, 43 * 30, (1, 4, 16, 16)),
])
def test_device_planner_at_the_stack_geometry(policy, slots, n_calls, tokens):
    """The geometry the 43-layer bench leg runs: 43 layers x 256 experts
    (11,008 keys) over 4,129 slots (and 8,257 under SLRU, beyond 8,000), the
    store's protected segment (slots - 1) // 2 under SLRU. Each thread of
    the planner workgroup then scans several slots per victim search, and the
    slot state fills most of the LDS. Zipf(1.1) calls of 1 to 16 tokens
    through the layers in order; every per-key result, every route's slot
    and the counters equal the host planner's, and the arena churns."""
    layers, E, top_k = 43, 256, 6
    pcap = (slots - 1) // 2 if policy == "slru" else 0
    rng = np.random.default_rng(slots + (1 if policy == "slru" else 2))
    ranks = [rng.permutation(E) for _ in range(layers)]
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    calls = []
    for c in range(n_calls):
        routes = []
        for _ in range(int(rng.choice(tokens))):
            routes.extend(int(ranks[c % layers][i]) for i in rng.choice(E, size=top_k, replace=False, p=p))
        calls.append((c % layers, routes))
    expect = host_run(calls, layers, E, slots, pcap, policy, top_k)
    dp = DevicePlanner(layers * E, slots, pcap, n_experts=E, policy=policy, max_routes=16 * top_k, device=DEV)
    hits = misses = evictions = 0
    for c, ((layer, routes), want_res) in enumerate(zip(calls, expect)):
        rs = dp.plan(torch.tensor(routes, dtype=torch.int32, device=DEV), layer, top_k)
        counters, got = dp.read(max_results=len(want_res))
        assert counters["error"] == 0, (c, counters)
        assert [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in got] == \
               [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in want_res], f"call {c} layer {layer}"
        slot_of = {r.key - layer * E: r.slot for r in want_res}
        assert rs.cpu().tolist() == [slot_of[e] for e in routes], f"route slots of call {c}"
        hits += sum(r.hit for r in want_res)
        misses += sum(not r.hit for r in want_res)
        evictions += sum(r.evicted_key >= 0 for r in want_res)
    counters, _ = dp.read()
    assert (counters["hits"], counters["misses"], counters["evictions"], counters["calls"]) == \
           (hits, misses, evictions, n_calls)
    assert evictions > 500 and hits > 1000, (hits, misses, evictions)


def prefetch_calls(rng, n_calls, layers, E, top_k, tokens=(1, 1, 3)):
    """Alternating demand and prefetch calls, as a layer call with a depth-1
    cross-layer prefetch makes them: ("demand", layer, routes) then
    ("prefetch", layer + 1, (idx [T, top_k], weights [T, top_k])) for a
    lookahead routing of T tokens whose weights come from a few values, so
    that equal weights are common."""
    ranks = [rng.permutation(E) for _ in range(layers)]
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    seq = []
    for c in range(n_calls):
        layer = c % layers
        routes = [int(ranks[layer][i]) for i in rng.choice(E, size=top_k, replace=False, p=p)]
        seq.append(("demand", layer, routes))
        nxt = (layer + 1) % layers
        T = int(rng.choice(tokens))
        idx = np.stack([ranks[nxt][rng.choice(E, size=top_k, replace=False, p=p)] for _ in range(T)])
        w = rng.choice(np.array([0.05, 0.1, 0.2, 0.3], np.float32), size=(T, top_k))
        seq.append(("prefetch", nxt, (idx.astype(np.int32), w.astype(np.float32))))
    return seq


def host_prefetch_run(seq, layers, E, slots, pcap, policy, top_k, take_k):
    """The host store's convention (V4ArenaStore.submit / _place_keys and
    ArenaStore's prefetch counters): a demand call pins the previous demand
    call's slots, touches hits and replaces the pinned set; a prefetch call
    plans the lookahead's take_k highest-weight experts per row
    (_lookahead_experts, deduplicated in order) with hits untouched and the
    same pins, and leaves the pinned set alone. Counters: hits and misses of
    demand calls, evictions of both, placed prefetch misses, demand hits on a
    prefetched key (used) and evictions of one before such a hit (wasted)."""
    from locali_amd.arena import _lookahead_experts
    cache = NativeCache(layers * E, slots, pcap, policy=policy)
    pinned, flag, out = (), {}, []
    cnt = dict(hits=0, misses=0, evictions=0, prefetched=0, prefetch_used=0, prefetch_wasted=0)
    for kind, layer, what in seq:
        if kind == "demand":
            want = list(dict.fromkeys(what))
            if layer == 0 and len(want) <= top_k:
                cache.note_token()
            res = cache.plan_each([layer * E + e for e in want], pinned_slots=pinned, touch_hits=True)
            pinned = tuple(r.slot for r in res if r.placed)
        else:
            idx, w = what
            want = list(dict.fromkeys(_lookahead_experts(idx.reshape(-1), w.reshape(-1).view(np.int32), top_k,
                                                         take_k)))
            res = cache.plan_each([layer * E + e for e in want], pinned_slots=pinned, touch_hits=False)
        for r in res:
            if r.evicted_key >= 0:
                cnt["evictions"] += 1
                if flag.get(r.slot):
                    cnt["prefetch_wasted"] += 1
            if kind == "demand":
                if r.hit:
                    cnt["hits"] += 1
                    if flag.get(r.slot):
                        cnt["prefetch_used"] += 1
                else:
                    cnt["misses"] += 1
                if r.placed:
                    flag[r.slot] = 0
            elif r.placed and not r.hit:
                cnt["prefetched"] += 1
                flag[r.slot] = 1
        out.append(res)
    cache.close()
    return out, cnt


@pytest.mark.parametrize("policy,slots,pcap,take_k,fused", [
    ("slru", 40, 12, 1, False),
    ("slru", 40, 12, 2, True),
    ("slru", 48, 0, 0, False),
    ("lfu-decay", 40, 0, 1, True),
    ("lfu-decay", 48, 0, 6, False),
])
def test_device_prefetch_matches_host_prefetch(policy, slots, pcap, take_k, fused):
    """locali_dplan_prefetch beside demand calls against the host store's
    convention: per-key results of every call (the take_k highest weights
    per row with ties in row order, the pins of the last demand call, hits
    untouched, unplaceable keys dropped), demand route slots, and the
    counters including prefetched / used / wasted. Fused: the launch also
    copies the placed misses, and each lands in its slot byte for byte."""
    layers, E, top_k, n_calls = 4, 48, 6, 150
    rng = np.random.default_rng(slots + pcap + 10 * take_k + fused)
    seq = prefetch_calls(rng, n_calls, layers, E, top_k)
    expect, cnt = host_prefetch_run(seq, layers, E, slots, pcap, policy, top_k, take_k)
    dp = DevicePlanner(layers * E, slots, pcap, n_experts=E, policy=policy, max_routes=64, device=DEV)
    sizes = [2048, 256]
    payload = torch.randint(0, 256, (layers * E, sum(sizes)), dtype=torch.uint8).pin_memory()
    arrays = [torch.zeros(slots, sz, dtype=torch.uint8, device=DEV) for sz in sizes]
    table = ([a.data_ptr() for a in arrays], sizes)
    host_src = torch.tensor(DevicePlanner.host_view([payload[k].data_ptr() for k in range(layers * E)]),
                            dtype=torch.uint64, device=DEV)
    for c, ((kind, layer, what), want_res) in enumerate(zip(seq, expect)):
        if kind == "demand":
            idx = torch.tensor(what, dtype=torch.int32, device=DEV)
            rs = dp.plan_fill(idx, layer, top_k, table, host_src) if fused else dp.plan(idx, layer, top_k)
            slot_of = {r.key - layer * E: r.slot for r in want_res}
            assert rs.cpu().tolist() == [slot_of[e] for e in what], f"route slots of call {c}"
        else:
            idx, w = (torch.from_numpy(a).to(DEV) for a in what)
            if fused:
                dp.prefetch(idx, w, layer, top_k, take_k, table, host_src)
            else:
                dp.prefetch(idx, w, layer, top_k, take_k)
        counters, got = dp.read(max_results=len(want_res))
        assert counters["error"] == 0, (c, counters)
        assert [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in got] == \
               [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in want_res], f"{kind} call {c} layer {layer}"
        if fused:
            for r in want_res:
                if r.placed and not r.hit:
                    landed = torch.cat([a[r.slot].cpu() for a in arrays])
                    assert torch.equal(landed, payload[r.key]), f"{kind} call {c}: key {r.key} in slot {r.slot}"
    counters, _ = dp.read()
    assert {k: counters[k] for k in cnt} == cnt
    assert counters["calls"] == len(seq)
    assert cnt["prefetched"] > 20 and cnt["prefetch_used"] > 10 and cnt["evictions"] > 20, cnt
