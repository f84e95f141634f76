"""The arena store (locali_amd.arena / dsv4_arena) on the CPU: slot geometry
and the zero slot, fills that land the exact expert bytes from either file
layout, the planner driven the way the reference drives it
(dsv4_arena.py:68-127; arena.py:212-354) against the oracle planner,
prefetch and capacity semantics, and the stats surface (arena.py:437-451)."""

from __future__ import annotations

import random

import numpy as np

import pytest
import torch

from checkpoint_fixture import expert_bytes, make_index, make_snapshot
from locali_amd.arena import ArenaStore
from locali_amd.dsv4_arena import PROJS, V4ArenaStore
from oracle.scheduler import LFU_DECAY, SLRU, OraclePlanner

LAYERS, EXPERTS, TOP_K = 3, 8, 2


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = tmp_path_factory.mktemp("ckpt")
    truth = make_snapshot(root, layers=LAYERS, experts=EXPERTS, top_k=TOP_K, d=128, dff=64)
    return root, truth, make_index(root), make_index(root, packed=True)


def _store(index, slots, cls=V4ArenaStore, **kw):
    per = ArenaStore.__new__(ArenaStore)  # item size from the index, without allocating
    import json
    meta = next(iter(json.loads(open(index).read())["experts"].values()))
    per = sum(meta[p][k][3] for p in PROJS for k in ("weight", "scales", "biases"))
    return cls(index, ceiling_gb=(slots * per + 1) / 1e9, threads=2, device="cpu", **kw)


def _slot_bytes(store, t, slot) -> bytes:
    out = b""
    for p in PROJS:
        for k in ("weight", "scales", "biases"):
            out += store.arena[(t, p, k)][slot].contiguous().view(torch.uint8).numpy().tobytes()
    return out


def test_geometry_zero_slot_and_ceiling(ckpt):
    _, _, index, _ = ckpt
    st = _store(index, 5)
    try:
        assert st.tiers == ["cold"] and st.slots["cold"] == 5
        assert st.resident == 5 * st.item["cold"] <= st.ceiling
        assert st.arena[("cold", "gate_proj", "weight")].shape[0] == 5
        assert not any(_slot_bytes(st, "cold", 0))
        assert st.quant("cold", "bits") == 2 and st.quant("cold", "group_size") == 64
        assert st.use_f16_moe == {"cold": False}
    finally:
        st.close()
    with pytest.raises(ValueError, match="no usable expert slot"):
        _store(index, 1)


@pytest.mark.parametrize("packed", [False, True])
def test_fills_land_the_experts_bytes(ckpt, packed):
    _, truth, index, pindex = ckpt
    st = _store(pindex if packed else index, 6)
    try:
        assert st.tier_overlap == packed
        placed = st.slots_for(1, [3, 5, 3])
        assert set(placed) == {3, 5}
        for e, (t, s) in placed.items():
            assert _slot_bytes(st, t, s) == expert_bytes(truth, 1, e)
        assert not any(_slot_bytes(st, "cold", 0))
        assert st.bytes_read == 2 * st.item["cold"]
        ea = st.expert_arena("cold")
        assert (ea.gate.bits, ea.down.bits, ea.gate.group_size) == (2, 2, 64)
        assert (ea.d_model, ea.d_ff, ea.n_slots) == (128, 64, 6)
    finally:
        st.close()


def test_host_source_fills_land_the_experts_bytes(ckpt, tmp_path):
    """A host-memory arena copies misses from host_source, never the files:
    the index's files are gone and the slots still hold the exact bytes."""
    import numpy as np
    _, truth, index, _ = ckpt
    moved = tmp_path / "v4.idx"
    moved.write_text(index.read_text().replace(str(index.parent), str(tmp_path / "absent")))
    calls = []

    def src(layer, expert):
        calls.append((layer, expert))
        return torch.from_numpy(np.frombuffer(expert_bytes(truth, layer, expert), np.uint8).copy())

    st = _store(moved, 5, host_source=src)
    try:
        for layer, experts in ((0, [1, 2]), (2, [7, 1]), (0, [2, 4])):
            placed = st.slots_for(layer, experts)
            for e, (t, s) in placed.items():
                assert _slot_bytes(st, t, s) == expert_bytes(truth, layer, e)
        assert calls == [(0, 1), (0, 2), (2, 7), (2, 1), (0, 4)]
        assert st.bytes_read == 5 * st.item["cold"] and st.stats()["evictions"] == 1
    finally:
        st.close()
    bad = _store(moved, 4, host_source=lambda layer, e: torch.zeros(3, dtype=torch.uint8))
    try:
        with pytest.raises(ValueError, match="host bytes"):
            bad.slots_for(0, [1])
    finally:
        bad.close()


@pytest.mark.parametrize("policy,slots", [("lru", 5), ("lru", 9), ("slru-all", 9), ("slru-all", 13),
                                          ("lfu-decay", 5), ("lfu-decay", 8)])
def test_native_planner_matches_the_oracle_driven_the_same_way(ckpt, policy, slots):
    _, _, index, _ = ckpt
    st = _store(index, slots, cache_policy=policy)
    prot = (slots - 1) // 2 if policy == "slru-all" else 0
    ref = OraclePlanner(LAYERS * EXPERTS, slots, prot, LFU_DECAY if policy == "lfu-decay" else SLRU)
    rng = random.Random(5)
    pinned: dict = {}
    hits = misses = evictions = 0
    try:
        for tok in range(12):
            for layer in range(LAYERS):
                want = list(dict.fromkeys(rng.randrange(EXPERTS) for _ in range(TOP_K)))
                if layer == 0 and len(want) <= TOP_K:
                    ref.note_token()
                res, pins = [], set(pinned)
                for e in want:                        # one key at a time, growing pins
                    rc, (r,) = ref.plan([layer * EXPERTS + e], pinned_slots=pins, touch_hits=True)
                    assert rc == 0
                    res.append(r)
                    pins.add(r.slot)
                want_slots = {e: r.slot for e, r in zip(want, res)}
                hits += sum(r.hit for r in res)
                misses += sum(not r.hit for r in res)
                evictions += sum(r.evicted_key >= 0 for r in res)
                pinned = set(want_slots.values())
                placed = st.slots_for(layer, want)
                assert {e: s for e, (_, s) in placed.items()} == want_slots
        s = st.stats()
        assert (s["hits"], s["misses"], s["evictions"]) == (hits, misses, evictions)
        assert s["protected"]["cold"] == ref.protected_size
        assert s["scheduler"] == "c"
    finally:
        st.close()


def test_one_multi_key_call_could_put_two_experts_on_one_slot():
    """Why the store plans key by key: with the previous call's two slots
    pinned and three usable slots, a single two-key call evicts its own first
    claim for its second miss."""
    ref = OraclePlanner(16, 4, 0, SLRU)
    _, first = ref.plan([0, 1], pinned_slots=(), touch_hits=True)
    _, res = ref.plan([2, 3], pinned_slots={r.slot for r in first}, touch_hits=True)
    assert res[0].slot == res[1].slot and res[1].evicted_key == 2


def test_python_planner_is_lru_with_pins(ckpt):
    _, truth, index, _ = ckpt
    st = _store(index, 3, native_scheduler=False, cache_policy="lru")
    try:
        a = st.slots_for(0, [1, 2])
        assert sorted(s for _, s in a.values()) == [1, 2]
        st.slots_for(0, [1])                          # 1 becomes most recent
        b = st.slots_for(0, [4])                      # evicts 2 (least recent, not pinned)
        assert b[4][1] == a[2][1]
        assert _slot_bytes(st, "cold", b[4][1]) == expert_bytes(truth, 0, 4)
        s = st.stats()
        assert (s["hits"], s["misses"], s["evictions"]) == (1, 3, 1)
        assert s["scheduler"] == "python"
    finally:
        st.close()
    with pytest.raises(RuntimeError, match="lfu-decay"):
        _store(index, 3, native_scheduler=False, cache_policy="lfu-decay")


@pytest.mark.parametrize("policy,slots", [("lru", 4), ("lru", 9), ("slru-all", 9), ("slru-all", 14),
                                          ("slru-cold", 11)])
def test_python_planner_matches_the_oracle_hits_first(ckpt, policy, slots):
    """native_scheduler=False follows the reference's fallback planner
    (arena.py:305-354): a call's resident experts resolve first (a demand
    hit refreshes its entry, a prefetch hit does not), then its misses in
    call order, each miss pinning the previous demand call's slots and every
    slot this call holds. That is the oracle planner driven one key at a
    time in that order; slots, evictions and segment sizes must agree."""
    _, _, index, _ = ckpt
    st = _store(index, slots, native_scheduler=False, cache_policy=policy)
    prot = (slots - 1) // 2 if policy in ("slru-all", "slru-cold") else 0
    ref = OraclePlanner(LAYERS * EXPERTS, slots, prot, SLRU)
    rng = random.Random(11 + slots)
    pinned: set = set()
    evictions = 0
    try:
        for step in range(60):
            layer = rng.randrange(LAYERS)
            prefetch = step % 5 == 4
            want = list(dict.fromkeys(rng.randrange(EXPERTS) for _ in range(rng.randint(1, 3))))
            keys = {e: layer * EXPERTS + e for e in want}
            hits = [e for e in want if ref.peek(keys[e]) >= 0]
            miss = [e for e in want if ref.peek(keys[e]) < 0]
            expect, held = {}, set()
            for e in hits:
                _, (r,) = ref.plan([keys[e]], pinned_slots=(), touch_hits=not prefetch)
                expect[e] = r.slot
                held.add(r.slot)
            for e in miss:
                _, (r,) = ref.plan([keys[e]], pinned_slots=pinned | held, touch_hits=not prefetch)
                if r.placed:
                    expect[e] = r.slot
                    held.add(r.slot)
                    evictions += r.evicted_key >= 0
            if prefetch:
                out, plan = st.submit(layer, want, prefetch=True)
                st.wait([f for fs in plan.values() for f in fs])
            else:
                out = st.slots_for(layer, want)
                pinned = held
            assert {e: s for e, (_, s) in out.items()} == expect, f"step {step}"
            assert st.stats()["protected"]["cold"] == ref.protected_size
            assert st.ledger["cold"].size[st.ledger["cold"].PROBATION] == ref.probation_size
        assert st.stats()["evictions"] == evictions and st.stats()["scheduler"] == "python"
    finally:
        st.close()


def test_tier_geometry_splits_the_ceiling():
    """Slot counts per tier from the byte ceiling (reference arena.py:100-165):
    hot and cold take hot_share and the rest in whole experts (zero slot
    counted in); slru-cold protects half of the cold tier's usable slots only;
    the first expert listed for a tier fixes its arrays."""
    from locali_amd.arena import tier_geometry

    def expert(tier, rows):
        recs = {k: ["/r", "s", 0, rows * w, [rows, w], dt]
                for k, w, dt in (("weight", 8, "U32"), ("scales", 1, "BF16"), ("biases", 1, "BF16"))}
        return {"tier": tier, **{p: dict(recs) for p in PROJS}}

    meta = {"L0.E0": expert("cold", 10), "L0.E1": expert("hot", 20), "L0.E2": expert("hot", 99)}
    per_cold, per_hot = 3 * 10 * 10, 3 * 20 * 10
    g = tier_geometry(meta, 100_000, 0.33, "slru-cold")
    assert sorted(g) == ["cold", "hot"]
    assert (g["cold"].expert_bytes, g["hot"].expert_bytes) == (per_cold, per_hot)
    assert g["hot"].slots == int(100_000 * 0.33 / per_hot) == 55
    assert g["cold"].slots == int(100_000 * 0.67 / per_cold) == 223
    assert (g["cold"].protected, g["hot"].protected) == (111, 0)
    assert g["hot"].arrays[("up_proj", "weight")][1] == (20, 8)
    one = tier_geometry({"L0.E0": expert("cold", 10)}, 10_000, 0.33, "slru-all")["cold"]
    assert (one.slots, one.protected) == (33, 16)
    assert tier_geometry(meta, 100_000, 0.33, "lru")["cold"].protected == 0


def test_prefetch_is_best_effort_and_accounted(ckpt):
    _, truth, index, _ = ckpt
    st = _store(index, 5)
    try:
        st.slots_for(0, [0, 1])
        out, plan = st.submit(1, [2, 6], prefetch=True)
        st.wait([f for fs in plan.values() for f in fs])
        s = st.stats()
        assert (s["hits"], s["misses"], s["prefetched"]) == (0, 2, 2)
        placed = st.slots_for(1, [6])                 # a demand hit on a prefetched expert
        assert placed[6] == out[6]
        assert _slot_bytes(st, "cold", out[6][1]) == expert_bytes(truth, 1, 6)
        s = st.stats()
        assert (s["hits"], s["prefetch_used"]) == (1, 1)
        st.slots_for(2, [3, 4])                       # evicts L0.E0 and L0.E1
        st.slots_for(2, [5, 7])                       # evicts the never-used prefetch L1.E2
        s = st.stats()
        assert s["prefetch_wasted"] == 1 and s["evictions"] == 4
    finally:
        st.close()


def test_a_prefetch_never_fills_a_slot_it_gave_away(ckpt):
    _, truth, index, _ = ckpt
    st = _store(index, 4)                              # three usable slots
    try:
        st.slots_for(0, [0, 1])                       # pins two of them
        out, plan = st.submit(1, [2, 6], prefetch=True)
        st.wait([f for fs in plan.values() for f in fs])
        slots = [s for _, s in out.values()]
        assert len(slots) == len(set(slots))          # no expert shares a slot
        for e, (t, s) in out.items():
            assert _slot_bytes(st, t, s) == expert_bytes(truth, 1, e)
    finally:
        st.close()


def test_capacity_is_enforced_for_demand_only(ckpt):
    _, _, index, _ = ckpt
    st = _store(index, 3)
    try:
        with pytest.raises(ValueError, match="arena has 2"):
            st.slots_for(0, [0, 1, 2])
        out, _ = st.submit(1, [0, 1, 2, 3], prefetch=True)   # best effort, no raise
        assert len(out) <= 2
    finally:
        st.close()


def test_stats_surface(ckpt):
    _, _, index, _ = ckpt
    st = _store(index, 3)
    try:
        keys = {"hits", "misses", "hit_rate", "evictions", "bytes_read", "resident", "peak", "slots",
                "t_stall", "t_convert", "t_eval", "prefetched", "prefetch_used",
                "prefetch_wasted", "cache_policy", "protected", "scheduler"}
        assert set(st.stats()) == keys
        st.slots_for(0, [1])
        st.slots_for(0, [1])
        assert st.stats()["hit_rate"] == 0.5
    finally:
        st.close()
    assert not st.arena and not st.fds


def test_lookahead_selection_matches_a_stable_weight_sort():
    """The prefetch's lookahead selection (reference arena.py:527-532): the k
    highest gate weights per row, ties kept in row order, through one host
    copy of indices and weight bits."""
    from locali_amd.arena import _host_ints, _lookahead_experts
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, 256, (5, 6), generator=g, dtype=torch.int32)
    w = torch.rand(5, 6, generator=g)
    w[1, 2] = w[1, 4] = w[1].max() + 1.0          # a tie at the top of row 1
    inds, ib, wb = _host_ints([idx, idx, w])
    assert np.array_equal(inds, idx.reshape(-1).numpy())
    for k in (1, 3, 5):
        order = torch.argsort(-w, dim=-1, stable=True)[:, :k]
        want = torch.gather(idx, 1, order).reshape(-1).tolist()
        assert _lookahead_experts(ib, wb, 6, k) == want
    for k in (6, None):              # the whole routing, in the router's order
        assert _lookahead_experts(ib, wb, 6, k) == idx.reshape(-1).tolist()
    assert _lookahead_experts(ib, wb, 6, 2)[2:4] == [int(idx[1, 2]), int(idx[1, 4])]


class _FakeLanded:
    """A fill future that lands two submits after it was issued."""

    def __init__(self, clock):
        self.clock, self.born = clock, clock[0]

    def done(self):
        return self.clock[0] >= self.born + 2


@pytest.mark.parametrize("policy,slots", [("slru-all", 14), ("lfu-decay", 9), ("lru", 10)])
def test_fast_submit_equals_the_general_path(ckpt, policy, slots):
    """V4ArenaStore.submit's host-fill path (one planner call, fills queued
    before the bookkeeping) gives the general ArenaStore.submit's placements,
    fills, futures, pending experts, pins and counters on the same calls,
    demand and prefetch mixed, with fills that land late."""
    _, _, index, _ = ckpt
    stores, logs, clocks = [], [], []
    for _ in range(2):
        st = _store(index, slots, cache_policy=policy)
        log, clock = [], [0]
        st.host_source = lambda layer, e: None
        st.fill_stream = object()

        def fake(jobs, on_caller_stream=False, log=log, clock=clock):
            log.append(([(key, tt, s) for key, tt, s, _ in jobs], on_caller_stream))
            return _FakeLanded(clock)
        st._fill_from_host = fake
        st._mark_demand = lambda: None
        stores.append(st)
        logs.append(log)
        clocks.append(clock)
    fast, general = stores
    rng = random.Random(17 + slots)
    try:
        for step in range(90):
            layer = rng.randrange(LAYERS)
            prefetch = step % 4 == 3
            want = [rng.randrange(EXPERTS) for _ in range(rng.randint(1, 3))]
            got = []
            for st, clock in ((fast, clocks[0]), (general, clocks[1])):
                clock[0] = step
                if st is fast:
                    out, plan = st.submit(layer, want, prefetch=prefetch)
                else:
                    out, plan = ArenaStore.submit(st, layer, want, prefetch=prefetch)
                got.append((out, {t: len(f) for t, f in plan.items()}, plan.pending_experts,
                            {k: len(v) for k, v in st.inflight.items()}, dict(st.pinned)))
            assert got[0] == got[1], f"step {step}"
            assert logs[0] == logs[1]
        keys = ("hits", "misses", "evictions", "bytes_read", "prefetched", "prefetch_used",
                "prefetch_wasted", "protected")
        assert {k: fast.stats()[k] for k in keys} == {k: general.stats()[k] for k in keys}
        assert fast.stats()["misses"] > 0 and fast.stats()["prefetched"] > 0
    finally:
        for st in stores:
            st.fill_stream = None
            st.close()


def test_a_truncated_shard_is_a_short_read(tmp_path):
    """A record past the end of its shard raises IOError from the fill (the
    reference's short-read check, arena.py:183-184, 199-200); the arena's
    other slots are untouched."""
    root = tmp_path / "ckpt"
    root.mkdir()
    make_snapshot(root, layers=LAYERS, experts=EXPERTS, top_k=TOP_K, d=128, dff=64)
    index = make_index(root)
    shard = root / "model-00002-of-00003.safetensors"
    shard.write_bytes(shard.read_bytes()[: shard.stat().st_size // 2])
    st = _store(index, 6)
    try:
        st.slots_for(0, [1])                         # layer 0's shard is whole
        with pytest.raises(IOError, match="short read"):
            st.slots_for(1, [EXPERTS - 1])
    finally:
        st.close()


def test_device_planner_refuses_what_it_does_not_cover(ckpt):
    """device_planner=True needs the compiled planner and host-memory fills
    of one tier; the store says so before it touches a GPU."""
    _, truth, index, _ = ckpt
    with pytest.raises(ValueError, match="host_source"):
        _store(index, 5, device_planner=True)
    src = lambda layer, e: torch.from_numpy(np.frombuffer(expert_bytes(truth, layer, e), np.uint8).copy())
    with pytest.raises(ValueError, match="native_scheduler"):
        _store(index, 5, device_planner=True, native_scheduler=False, host_source=src)
