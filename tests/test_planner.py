"""Slot planner parity (CPU): liblocali_amd.so's locali_cache_* vs the
reference planner.

Pins, in order of strength:
  * golden traces recorded from the reference's own native/locali_core.c
    (compiled unchanged by oracle/Makefile, tests/golden/planner_traces.json);
  * the reference KATs native/test_locali_core.c:14-74 restated as tests;
  * the reference differential test tests/test_locali_native.py:81-122 (the
    Python ReferenceCache spec, restated by oracle.scheduler);
  * the live reference library in oracle/_ref when it has been built here.
"""

from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np
import pytest

import planner_traces as pt
from locali_amd import native
from locali_amd.native import NativeCache
from oracle.scheduler import LFU_DECAY, SLRU, OraclePlanner

ROOT = Path(__file__).resolve().parents[1]
TRACES = json.loads((ROOT / "tests" / "golden" / "planner_traces.json").read_text())
REF_LIB = ROOT / "oracle" / "_ref" / "liblocali_core_ref.so"


class _Ours:
    """NativeCache adapter exposing the trace-runner protocol."""

    def __init__(self, cap, slots, prot, policy):
        self.c = NativeCache(cap, slots, prot, policy="lfu-decay" if policy else "slru")

    def plan(self, keys, pins, touch):
        return self.c.plan_raw(keys, pins, touch)

    def note_token(self):
        self.c.note_token()

    def peek(self, k):
        return self.c.peek(k)

    @property
    def probation_size(self):
        return self.c.probation_size

    @property
    def protected_size(self):
        return self.c.protected_size


class _Oracle:
    def __init__(self, cap, slots, prot, policy):
        self.o = OraclePlanner(cap, slots, prot, LFU_DECAY if policy else SLRU)

    def plan(self, keys, pins, touch):
        rc, res = self.o.plan(keys, pins, touch)
        return rc, [(r.key, r.slot, r.evicted_key, int(r.hit), int(r.placed)) for r in res]

    def note_token(self):
        self.o.note_token()

    def peek(self, k):
        return self.o.peek(k)

    @property
    def probation_size(self):
        return self.o.probation_size

    @property
    def protected_size(self):
        return self.o.protected_size


CASES = {name: (cap, slots, prot, pol, ops, keep)
         for name, cap, slots, prot, pol, ops, keep in pt.all_cases()}


@pytest.mark.parametrize("case", TRACES["cases"], ids=lambda c: c["name"])
@pytest.mark.parametrize("impl", [_Ours, _Oracle], ids=["liblocali_amd", "oracle"])
def test_golden_planner_traces(case, impl):
    cap, slots, prot, pol, ops, _ = CASES[case["name"]]
    assert (cap, slots, prot, pol) == (case["key_capacity"], case["slots"], case["protected"],
                                      case["policy"])
    assert len(ops) == case["n_ops"]
    records = pt.resolve_and_run(impl(cap, slots, prot, pol), ops, TRACES["probe"], cap)
    if "records" in case:
        for i, (got, want) in enumerate(zip(records, case["records"])):
            assert got == want, f"op {i}: {ops[i]}"
    assert pt.digest(records) == case["digest"]


def _one(c, key, touch=True):
    return c.plan([key], touch_hits=touch)[0]


def test_kat_lru():                       # native/test_locali_core.c:14-26
    c = NativeCache(16, 4, 0)
    assert _one(c, 1).slot == 3
    assert _one(c, 2).slot == 2
    assert _one(c, 3).slot == 1
    assert _one(c, 1).hit
    r = _one(c, 4)
    assert not r.hit and r.evicted_key == 2 and r.slot == 2
    assert c.peek(1) == 3 and c.peek(2) == -1


def test_kat_slru_reservation_and_promotion():   # native/test_locali_core.c:28-43
    c = NativeCache(16, 5, 2)
    assert _one(c, 0).slot == 4
    assert _one(c, 1).slot == 3
    r = _one(c, 2)
    assert r.evicted_key == 0 and r.slot == 4
    assert c.probation_size == 2
    assert _one(c, 1).hit
    assert c.probation_size == 1 and c.protected_size == 1
    assert _one(c, 3).slot == 2
    assert _one(c, 2).hit
    assert c.protected_size == 2


def test_kat_pinned_slots_are_not_reused():      # native/test_locali_core.c:45-57
    c = NativeCache(8, 3, 0)
    first = c.plan([0, 1])
    r = c.plan([2], pinned_slots=[first[0].slot, first[1].slot])[0]
    assert not r.placed and r.slot == -1


def test_kat_lfu_decay():                        # native/test_locali_core.c:59-74
    c = NativeCache(16, 3, 0, policy="lfu-decay")
    assert not _one(c, 1).hit
    assert _one(c, 1).hit
    assert not _one(c, 2).hit
    assert _one(c, 3).evicted_key == 2
    for _ in range(16):
        c.note_token()
    assert _one(c, 4).evicted_key == 3
    assert c.peek(1) >= 0


@pytest.mark.parametrize("protected_capacity", [0, 3])
def test_differential_reference_sequence(protected_capacity):  # tests/test_locali_native.py:81-103
    ours = NativeCache(64, 8, protected_capacity)
    spec = OraclePlanner(64, 8, protected_capacity)
    sequence = [0, 1, 2, 3, 0, 4, 5, 1, 6, 7, 2, 8, 0, 9, 3, 10]
    for position, key in enumerate(sequence):
        resident = [s for s in range(1, 8) if s in set(spec.probation.values()) | set(spec.protected.values())]
        pinned = resident[:1] if position % 4 == 3 else []
        rc, want = spec.plan([key], pinned, True)
        got = ours.plan([key], pinned_slots=pinned, touch_hits=True)[0]
        w = want[0]
        assert (got.slot, got.hit, got.evicted_key, got.placed) == (w.slot, w.hit, w.evicted_key, w.placed)
        assert ours.probation_size == spec.probation_size
        assert ours.protected_size == spec.protected_size
        for cand in range(11):
            assert ours.peek(cand) == spec.peek(cand)


def test_invalid_key_returns_minus3_after_partial_results():
    c = NativeCache(10, 4, 0)
    rc, res = c.plan_raw([1, 2, 50, 3])
    assert rc == -3
    assert [r[1] for r in res[:2]] == [3, 2]
    assert c.peek(1) == 3 and c.peek(2) == 2 and c.peek(3) == -1
    with pytest.raises(ValueError):
        c.plan([99])


@pytest.mark.parametrize("args", [(0, 4, 0, 0), (8, 1, 0, 0), (8, 4, 4, 0), (8, 4, -1, 0),
                                  (8, 4, 0, 7)])
def test_create_rejects_bad_arguments(args):
    lib = native._lib.lib()
    assert not lib.locali_cache_create_policy(*args)


def test_lfu_forces_zero_protected():
    c = NativeCache(16, 5, 3, policy="lfu-decay")
    for k in range(6):
        c.plan([k])
        c.plan([k])
    assert c.protected_size == 0


@pytest.mark.skipif(not REF_LIB.exists(), reason="reference planner not built (make -C oracle ref)")
def test_live_reference_library_agrees_on_random_workloads():
    ref = pt.bind(ctypes.CDLL(str(REF_LIB)))
    for seed in range(6):
        slots, prot, pol = [(9, 4, 0), (12, 0, 1), (7, 0, 0)][seed % 3]
        ops = pt.workload_random(1000 + seed, 90, 200, 5, note_prob=0.15 if pol else 0.0)
        a = pt.resolve_and_run(pt.CPlanner(ref, 90, slots, prot, pol), ops, pt.PROBE, 90)
        b = pt.resolve_and_run(_Ours(90, slots, prot, pol), ops, pt.PROBE, 90)
        assert a == b


@pytest.mark.parametrize("policy,slots,prot", [("slru", 6, 0), ("slru", 9, 4), ("lfu-decay", 7, 0)])
def test_plan_each_equals_one_call_per_key_with_growing_pins(policy, slots, prot):
    """locali_cache_plan_each (include/locali_planner.h) against the oracle
    planner driven one key per call, each call pinning the caller's slots plus
    the slots the earlier keys resolved to -- slots, hits, evictions, segment
    sizes and the -3 state, on nearly full tiers where the pins matter."""
    import random
    rng = random.Random(slots * 7 + prot)
    ours = NativeCache(40, slots, prot, policy=policy)
    ref = OraclePlanner(40, slots, prot, LFU_DECAY if policy == "lfu-decay" else SLRU)
    pinned: set = set()
    for step in range(300):
        if step % 7 == 0:
            ours.note_token()
            ref.note_token()
        keys = list(dict.fromkeys(rng.randrange(40) for _ in range(rng.randint(1, slots - 1))))
        touch = step % 5 != 4
        got = ours.plan_each(keys, pinned_slots=tuple(pinned), touch_hits=touch)
        pins, want = set(pinned), []
        for k in keys:
            rc, (r,) = ref.plan([k], pinned_slots=pins, touch_hits=touch)
            assert rc == 0
            want.append((r.key, r.slot, r.evicted_key, bool(r.hit), bool(r.placed)))
            if r.placed:
                pins.add(r.slot)
        assert [(r.key, r.slot, r.evicted_key, r.hit, r.placed) for r in got] == want, f"step {step}"
        assert (ours.probation_size, ours.protected_size) == (ref.probation_size, ref.protected_size)
        if touch:
            pinned = {r.slot for r in got if r.placed}
    with pytest.raises(ValueError):
        ours.plan_each([1, 99, 2])


@pytest.mark.parametrize("policy", ["slru", "lfu-decay"])
def test_device_planner_placement_bound_is_sound(policy):
    """DevicePlanner.placement_certain, the host-side check that lets a
    device-planned demand call proceed, never admits a call that the
    compiled planner fails to place: random geometries and call sequences
    under the store's convention (plan_each, the previous call's slots
    pinned). The calls it refuses include every call that did fail, and
    some did fail, so the check is not vacuous."""
    from locali_amd.native import DevicePlanner
    rng = np.random.default_rng(11 if policy == "slru" else 12)
    failed = refused = 0
    for _ in range(300):
        slots = int(rng.integers(3, 24))
        pcap = int(rng.integers(0, slots - 1)) if policy == "slru" else 0
        n_keys = int(rng.integers(2, 40))
        probation = slots - 1 - pcap
        cache = NativeCache(n_keys, slots, pcap, policy=policy)
        pinned = []
        for _ in range(20):
            k = int(rng.integers(1, min(n_keys, slots + 2) + 1))
            keys = [int(v) for v in rng.choice(n_keys, size=k, replace=False)]
            ok = DevicePlanner.placement_certain(len(keys), len(pinned), probation)
            res = cache.plan_each(keys, pinned_slots=pinned)
            placed = all(r.placed for r in res)
            refused += not ok
            failed += not placed
            assert placed or not ok, (slots, pcap, keys, pinned)
            pinned = sorted({r.slot for r in res if r.placed})
        cache.close()
    assert failed > 0 and refused >= failed
