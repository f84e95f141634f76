"""Seeded planner workloads and a trace runner shared by the golden-trace
generator (make_planner_traces.py, which drives the reference planner compiled
into oracle/_ref) and the tests (which drive liblocali_amd.so and the Python
oracle through the same operations).

A workload is a list of operations:
  ["plan", keys, pinned_slots, touch_hits]   -> one locali_cache_plan call
  ["note"]                                   -> one locali_cache_note_token
The runner records, per operation, the return code, every result tuple
(key, slot, evicted_key, hit, placed), probation/protected sizes and a peek
of a fixed probe set of keys.
"""

from __future__ import annotations

import ctypes
import hashlib
import json
import random


class CResult(ctypes.Structure):
    _fields_ = [
        ("key", ctypes.c_int32),
        ("slot", ctypes.c_int32),
        ("evicted_key", ctypes.c_int32),
        ("hit", ctypes.c_uint8),
        ("placed", ctypes.c_uint8),
    ]


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    lib.locali_cache_create_policy.argtypes = [ctypes.c_int32] * 4
    lib.locali_cache_create_policy.restype = ctypes.c_void_p
    lib.locali_cache_destroy.argtypes = [ctypes.c_void_p]
    lib.locali_cache_note_token.argtypes = [ctypes.c_void_p]
    lib.locali_cache_plan.argtypes = [
        ctypes.c_void_p, ctypes.POINTER(ctypes.c_int32), ctypes.c_size_t,
        ctypes.POINTER(ctypes.c_int32), ctypes.c_size_t, ctypes.c_int,
        ctypes.POINTER(CResult)]
    lib.locali_cache_plan.restype = ctypes.c_int
    lib.locali_cache_peek.argtypes = [ctypes.c_void_p, ctypes.c_int32]
    lib.locali_cache_peek.restype = ctypes.c_int32
    lib.locali_cache_probation_size.argtypes = [ctypes.c_void_p]
    lib.locali_cache_probation_size.restype = ctypes.c_int32
    lib.locali_cache_protected_size.argtypes = [ctypes.c_void_p]
    lib.locali_cache_protected_size.restype = ctypes.c_int32
    return lib


class CPlanner:
    """Minimal driver over any library exporting the locali_cache_* ABI."""

    def __init__(self, lib, key_capacity, slots, protected_capacity, policy):
        self.lib = lib
        self.key_capacity = key_capacity
        self.h = lib.locali_cache_create_policy(key_capacity, slots,
                                                protected_capacity, policy)
        if not self.h:
            raise ValueError("create failed")

    def plan(self, keys, pinned_slots=(), touch_hits=True):
        n = len(keys)
        karr = (ctypes.c_int32 * max(n, 1))(*keys)
        parr = (ctypes.c_int32 * len(pinned_slots))(*pinned_slots) if pinned_slots else None
        res = (CResult * max(n, 1))()
        rc = self.lib.locali_cache_plan(self.h, karr, n, parr, len(pinned_slots),
                                        int(touch_hits), res)
        out = []
        for r in res[:n]:
            out.append((r.key, r.slot, r.evicted_key, int(r.hit), int(r.placed)))
        return rc, out

    def note_token(self):
        self.lib.locali_cache_note_token(self.h)

    def peek(self, key):
        return self.lib.locali_cache_peek(self.h, key)

    @property
    def probation_size(self):
        return self.lib.locali_cache_probation_size(self.h)

    @property
    def protected_size(self):
        return self.lib.locali_cache_protected_size(self.h)

    def close(self):
        if self.h:
            self.lib.locali_cache_destroy(self.h)
            self.h = None


def digest(records) -> str:
    return hashlib.sha256(json.dumps(records, separators=(",", ":")).encode()).hexdigest()


# --------------------------------------------------------------------------
# Seeded workloads
# --------------------------------------------------------------------------

def _zipf_pick(rng, n, k, s=1.1):
    weights = [1.0 / (r + 1) ** s for r in range(n)]
    perm = list(range(n))
    rng.shuffle(perm)
    chosen = []
    pool = list(range(n))
    w = weights[:]
    for _ in range(k):
        idx = rng.choices(range(len(pool)), weights=w)[0]
        chosen.append(perm[pool[idx]])
        del pool[idx]
        del w[idx]
    return chosen


def workload_layers(seed, layers, experts, top_k, steps, pin_previous=True,
                    prefetch_every=0, note_layer0=True):
    """Decode-shaped ops: per step and layer, the unique experts of one token
    in first-appearance order (reference arena.py:375), keys = layer*E + e
    (dsv4_arena.py:57-62), pinned = previous demand call's slots
    (dsv4_arena.py:86-90, 125-126). Slots are not known when the workload is
    built, so pins are resolved by the runner through "pin_prev"."""
    rng = random.Random(seed)
    ops = []
    for step in range(steps):
        for layer in range(layers):
            experts_l = _zipf_pick(rng, experts, top_k)
            if note_layer0 and layer == 0:
                ops.append(["note"])
            keys = [layer * experts + e for e in experts_l]
            ops.append(["plan", keys, "pin_prev" if pin_previous else [], True])
            if prefetch_every and (step * layers + layer) % prefetch_every == 0:
                nxt = (layer + 1) % layers
                pk = [nxt * experts + e for e in _zipf_pick(rng, experts, top_k)[:4]]
                ops.append(["plan", pk, "pin_prev", False])
    return ops


def resolve_and_run(planner, ops, probe, cap):
    """Apply ops to a planner and return JSON-able per-op records.

    "pin_prev" resolves to the slots returned by the previous demand
    (touch_hits=True) plan call. For a -3 return only the results the C
    planner is guaranteed to have written (before the invalid key) are kept."""
    records = []
    prev_slots: list[int] = []
    for op in ops:
        if op[0] == "note":
            planner.note_token()
            records.append(["note", planner.probation_size, planner.protected_size])
            continue
        _, keys, pinned, touch = op
        pins = prev_slots if pinned == "pin_prev" else list(pinned)
        rc, results = planner.plan(keys, pins, touch)
        if rc == -3:
            bad = next(i for i, k in enumerate(keys) if not 0 <= k < cap)
            results = results[:bad]
        results = [list(map(int, (r if isinstance(r, tuple) else
                                  (r.key, r.slot, r.evicted_key, r.hit, r.placed))))
                   for r in results]
        if touch and rc == 0:
            prev_slots = [r[1] for r in results if r[4]]
        records.append(["plan", rc, results, planner.probation_size,
                        planner.protected_size, [planner.peek(k) for k in probe]])
    return records


def workload_random(seed, key_capacity, steps, max_keys, pin_prob=0.3,
                    invalid_at=None, note_prob=0.0, touch_prob=0.85):
    rng = random.Random(seed)
    ops = []
    for i in range(steps):
        if note_prob and rng.random() < note_prob:
            ops.append(["note"])
        n = rng.randint(1, max_keys)
        keys = []
        while len(keys) < n:
            k = int(min(key_capacity - 1, rng.paretovariate(1.2) - 1))
            if k not in keys:
                keys.append(k)
        if invalid_at is not None and i == invalid_at:
            keys.insert(len(keys) // 2, key_capacity + 3)
        pinned = "pin_prev" if rng.random() < pin_prob else []
        ops.append(["plan", keys, pinned, rng.random() < touch_prob])
    return ops


def all_cases():
    """(name, key_capacity, slots, protected_capacity, policy, ops, keep_full)"""
    cases = []
    # Reference differential sequence (tests/test_locali_native.py:85) as one
    # key per call, protected 0 and 3, 64 keys, 8 slots.
    seq = [0, 1, 2, 3, 0, 4, 5, 1, 6, 7, 2, 8, 0, 9, 3, 10]
    for prot in (0, 3):
        cases.append((f"ref_sequence_p{prot}", 64, 8, prot, 0,
                      [["plan", [k], [], True] for k in seq], True))
    # Random multi-key workloads: SLRU with protected 0 and (n-1)//2, LFU.
    for seed, (slots, prot, pol) in enumerate([(9, 0, 0), (9, 4, 0), (17, 8, 0),
                                               (17, 0, 1), (33, 0, 1), (5, 2, 0)]):
        cases.append((f"random_s{slots}_p{prot}_pol{pol}", 200, slots, prot, pol,
                      workload_random(100 + seed, 200, 300, 6,
                                      note_prob=0.2 if pol else 0.0), True))
    # Invalid key mid-call -> -3 with earlier results kept.
    cases.append(("invalid_key", 50, 7, 3, 0,
                  workload_random(7, 50, 40, 5, invalid_at=20), True))
    # Decode-shaped per-layer pool: 4 layers x 32 experts, top-6, 13 slots.
    cases.append(("decode_small_slru", 4 * 32, 13, 6, 0,
                  workload_layers(11, 4, 32, 6, 24, prefetch_every=5), True))
    cases.append(("decode_small_lfu", 4 * 32, 13, 0, 1,
                  workload_layers(12, 4, 32, 6, 40), True))
    # Bounded-arena shape: one pool of 97 slots over 43x256 keys (96 usable
    # slots + zero slot), SLRU (protected (n-1)//2) and LFU; digest only.
    cases.append(("c5_pool_slru", 43 * 256, 97, 48, 0,
                  workload_layers(21, 43, 256, 6, 6), False))
    cases.append(("c5_pool_lfu", 43 * 256, 97, 0, 1,
                  workload_layers(22, 43, 256, 6, 6), False))
    return cases


PROBE = list(range(12))
