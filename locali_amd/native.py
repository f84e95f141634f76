"""Slot planner handle over liblocali_amd.so.

Mirrors the reference's ctypes wrapper ``locali_native.NativeCache``
(locali_native.py:58-167): same constructor arguments, policy names
``{"slru": 0, "lfu-decay": 1}`` (:101), ``plan`` returning CacheResult records
and raising ``ValueError`` on a non-zero planner code (:137-138), ``peek``,
``probation_size``, ``protected_size``, ``note_token`` and ``close``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

from . import _lib

POLICIES = {"slru": 0, "lfu-decay": 1}


@dataclass(frozen=True)
class CacheResult:
    key: int
    slot: int
    evicted_key: int
    hit: bool
    placed: bool


def available(path: Path | None = None) -> bool:
    return Path(path or _lib.LIB_PATH).is_file()


class NativeCache:
    def __init__(self, key_capacity: int, slots: int, protected_capacity: int, *,
                 policy: str = "slru"):
        self._cache = None
        self._lib = _lib.lib()
        if policy not in POLICIES:
            raise ValueError(f"unknown native cache policy: {policy}")
        self._cache = self._lib.locali_cache_create_policy(
            key_capacity, slots, protected_capacity, POLICIES[policy])
        if not self._cache:
            raise MemoryError("failed to create Locali native cache")
        self.key_capacity = key_capacity
        self.slots = slots

    def note_token(self) -> None:
        self._lib.locali_cache_note_token(self._cache)

    def plan(self, keys, *, pinned_slots=(), touch_hits: bool = True) -> list[CacheResult]:
        if not keys:
            return []
        n = len(keys)
        key_array = (ctypes.c_int32 * n)(*keys)
        pinned_array = ((ctypes.c_int32 * len(pinned_slots))(*pinned_slots)
                        if pinned_slots else None)
        results = (_lib.CacheResult * n)()
        rc = self._lib.locali_cache_plan(self._cache, key_array, n, pinned_array,
                                         len(pinned_slots), int(touch_hits), results)
        if rc:
            raise ValueError(f"native cache plan failed with error {rc}")
        return [CacheResult(r.key, r.slot, r.evicted_key, bool(r.hit), bool(r.placed))
                for r in results]

    def plan_each(self, keys, *, pinned_slots=(), touch_hits: bool = True) -> list[CacheResult]:
        """plan() one key at a time in a single call, each key also pinning
        the slots the keys before it resolved to (locali_cache_plan_each)."""
        if not keys:
            return []
        n = len(keys)
        key_array = (ctypes.c_int32 * n)(*keys)
        pinned_array = ((ctypes.c_int32 * len(pinned_slots))(*pinned_slots)
                        if pinned_slots else None)
        results = (_lib.CacheResult * n)()
        rc = self._lib.locali_cache_plan_each(self._cache, key_array, n, pinned_array,
                                              len(pinned_slots), int(touch_hits), results)
        if rc:
            raise ValueError(f"native cache plan failed with error {rc}")
        return [CacheResult(r.key, r.slot, r.evicted_key, bool(r.hit), bool(r.placed))
                for r in results]

    def plan_each_into(self, keys, pinned_slots=(), touch_hits: bool = True):
        """plan_each() returning the ctypes CacheResult array itself (fields
        key, slot, evicted_key, hit, placed), for per-layer hot loops."""
        n = len(keys)
        key_array = (ctypes.c_int32 * n)(*keys)
        pinned_array = ((ctypes.c_int32 * len(pinned_slots))(*pinned_slots)
                        if pinned_slots else None)
        results = (_lib.CacheResult * n)()
        rc = self._lib.locali_cache_plan_each(self._cache, key_array, n, pinned_array,
                                              len(pinned_slots), int(touch_hits), results)
        if rc:
            raise ValueError(f"native cache plan failed with error {rc}")
        return results

    def plan_raw(self, keys, pinned_slots=(), touch_hits: bool = True):
        """(rc, [(key, slot, evicted_key, hit, placed)]) without raising; the
        results of an rc=-3 call are the ones the planner wrote before the
        invalid key."""
        n = len(keys)
        key_array = (ctypes.c_int32 * max(n, 1))(*keys)
        pinned_array = ((ctypes.c_int32 * len(pinned_slots))(*pinned_slots)
                        if pinned_slots else None)
        results = (_lib.CacheResult * max(n, 1))()
        rc = self._lib.locali_cache_plan(self._cache, key_array, n, pinned_array,
                                         len(pinned_slots), int(touch_hits), results)
        return rc, [(r.key, r.slot, r.evicted_key, int(r.hit), int(r.placed)) for r in results[:n]]

    def peek(self, key: int) -> int:
        return int(self._lib.locali_cache_peek(self._cache, key))

    @property
    def probation_size(self) -> int:
        return int(self._lib.locali_cache_probation_size(self._cache))

    @property
    def protected_size(self) -> int:
        return int(self._lib.locali_cache_protected_size(self._cache))

    def close(self) -> None:
        if getattr(self, "_cache", None):
            self._lib.locali_cache_destroy(self._cache)
            self._cache = None

    def __del__(self):
        self.close()


class DevicePlanner:
    """The planner's placement rules on the GPU (locali_dplan_*, see
    include/locali_planner.h): the state lives in one device buffer and each
    layer call is one kernel on the caller's current stream, so routing,
    placement, fills and expert kernels queue without a host round trip.
    Decisions equal NativeCache.plan_each's with the previous demand call's
    slots pinned and the LFU token tick on layer-0 calls of at most top_k
    experts (V4ArenaStore._place_keys)."""

    LDS_LIMIT = 160 * 1024 - 4096   # the kernel's LDS less its static part

    def __init__(self, key_capacity: int, slots: int, protected_capacity: int, *, n_experts: int,
                 policy: str = "slru", max_routes: int = 16384, device=None):
        import torch
        from .ops import _stream
        if policy not in POLICIES:
            raise ValueError(f"unknown native cache policy: {policy}")
        self._lib = _lib.lib()
        self.key_capacity, self.slots, self.n_experts = key_capacity, slots, n_experts
        self.policy = POLICIES[policy]
        self.max_routes = max_routes
        # keys that probation holds when it is full (LFU-decay keeps every
        # key there); see demand_fits
        self.probation_capacity = slots - 1 - (protected_capacity if policy == "slru" else 0)
        lds = self._lib.locali_dplan_lds_bytes(slots, n_experts, self.policy)
        if lds > self.LDS_LIMIT:
            raise ValueError(f"device planner: {slots} slots x {n_experts} experts need {lds} bytes of LDS "
                             f"(at most {self.LDS_LIMIT}); use the host planner")
        nbytes = self._lib.locali_dplan_state_bytes(key_capacity, slots, max_routes)
        if not nbytes:
            raise ValueError("device planner: bad shape")
        self.state = torch.empty(nbytes, dtype=torch.uint8, device=device)
        if self.state.data_ptr() % 256:
            raise RuntimeError("device planner state is not 256-byte aligned")
        _lib.check(self._lib.locali_dplan_init(self.state.data_ptr(), nbytes, key_capacity, slots,
                                                 protected_capacity, self.policy, max_routes, _stream()),
                   "locali_dplan_init")
        self._table = None

    @staticmethod
    def placement_certain(keys: int, pinned: int, probation_capacity: int) -> bool:
        """True when a call of `keys` distinct keys, with `pinned` slots of
        the previous call pinned, places every key whatever the planner's
        state (native/locali_core.c:113-180). A key finds no slot only when
        every resident key is pinned and no free slot may be taken: under
        SLRU that needs a full probation segment or no free slot, under
        LFU-decay no free slot, and either way at least probation_capacity
        resident keys. At most pinned + keys - 1 slots are pinned when the
        call's last key is planned."""
        return keys + pinned <= probation_capacity

    def demand_fits(self, keys: int, pinned: int) -> bool:
        return self.placement_certain(keys, pinned, self.probation_capacity)

    def plan(self, expert_idx, layer: int, top_k: int, *, touch_hits: bool = True, out=None):
        """Slots of the routes in expert_idx (device int32, any shape) for
        `layer`; returns a device int32 tensor of the same shape."""
        import torch
        from .ops import _stream
        idx = expert_idx.reshape(-1)
        if idx.dtype != torch.int32 or not idx.is_cuda:
            raise ValueError("device planner: expert_idx must be a device int32 tensor")
        idx = idx.contiguous()
        if out is None:
            out = torch.empty(idx.numel(), dtype=torch.int32, device=idx.device)
        _lib.check(self._lib.locali_dplan_plan(self.state.data_ptr(), self.key_capacity, self.slots, self.policy,
                                                 self.max_routes, idx.data_ptr(), idx.numel(), layer,
                                                 self.n_experts, top_k, int(touch_hits), out.data_ptr(),
                                                 _stream()),
                   "locali_dplan_plan")
        return out.view(expert_idx.shape)

    def _records(self, table):
        if self._table is None or self._table[0] is not table:
            base, per = table[0], table[1]
            self._table = (table, (ctypes.c_void_p * len(base))(*base), (ctypes.c_size_t * len(per))(*per),
                           len(base))
        return self._table[1:]

    def fill(self, table, host_src, layer: int, max_misses: int) -> None:
        """Copy the last plan's misses into their slots. table: (bases,
        per-slot bytes) of the arena arrays in record order; host_src: device
        uint64 tensor of the key_capacity device-visible payload addresses."""
        from .ops import _stream
        bases, pers, n = self._records(table)
        _lib.check(self._lib.locali_dplan_fill(self.state.data_ptr(), bases, pers, n, host_src.data_ptr(), layer,
                                                 self.n_experts, max_misses, _stream()),
                   "locali_dplan_fill")

    def plan_fill(self, expert_idx, layer: int, top_k: int, table, host_src, *, touch_hits: bool = True,
                  out=None):
        """plan() then fill() in one launch: the misses' copies start while
        the planner decides the keys after them. Same results."""
        import torch
        from .ops import _stream
        idx = expert_idx.reshape(-1)
        if idx.dtype != torch.int32 or not idx.is_cuda:
            raise ValueError("device planner: expert_idx must be a device int32 tensor")
        idx = idx.contiguous()
        if out is None:
            out = torch.empty(idx.numel(), dtype=torch.int32, device=idx.device)
        bases, pers, n = self._records(table)
        _lib.check(self._lib.locali_dplan_plan_fill(self.state.data_ptr(), self.key_capacity, self.slots,
                                                      self.policy, self.max_routes, idx.data_ptr(), idx.numel(),
                                                      layer, self.n_experts, top_k, int(touch_hits),
                                                      out.data_ptr(), bases, pers, n, host_src.data_ptr(),
                                                      _stream()),
                   "locali_dplan_plan_fill")
        return out.view(expert_idx.shape)

    def prefetch(self, expert_idx, weights, layer: int, top_k: int, take_k: int = 0, table=None, host_src=None):
        """The cross-layer prefetch call (locali_dplan_prefetch): expert_idx
        (device int32) and weights (device fp32) are rows of top_k routes of
        a lookahead routing; each row's take_k highest weights (ties in row
        order; every route when take_k is 0 or >= top_k) are planned with
        hits left in place and the last demand call's slots pinned, and keys
        that find no slot are dropped. With table and host_src the same
        launch copies the placed misses (as plan_fill); otherwise fill()
        copies them afterwards."""
        import torch
        from .ops import _stream
        idx = expert_idx.reshape(-1, top_k)
        w = weights.reshape(-1, top_k)
        if idx.dtype != torch.int32 or not idx.is_cuda or w.dtype != torch.float32 or not w.is_cuda:
            raise ValueError("device planner: prefetch takes device int32 experts and float32 weights")
        if idx.shape != w.shape:
            raise ValueError("device planner: prefetch experts and weights differ in shape")
        idx, w = idx.contiguous(), w.contiguous()
        if table is not None:
            bases, pers, n = self._records(table)
            src = host_src.data_ptr()
        else:
            bases, pers, n, src = None, None, 0, None
        _lib.check(self._lib.locali_dplan_prefetch(self.state.data_ptr(), self.key_capacity, self.slots, self.policy,
                                                     self.max_routes, idx.data_ptr(), w.data_ptr(), idx.shape[0],
                                                     top_k, int(take_k or 0), layer, self.n_experts, bases, pers,
                                                     n, src, _stream()),
                   "locali_dplan_prefetch")

    @staticmethod
    def host_view(pointers) -> list[int]:
        """Device-visible addresses of pinned host payloads (raises for any
        that is not pinned and 16-byte aligned)."""
        n = len(pointers)
        src = (ctypes.c_void_p * max(n, 1))(*pointers)
        out = (ctypes.c_uint64 * max(n, 1))()
        _lib.check(_lib.lib().locali_dplan_host_view(src, n, out), "locali_dplan_host_view")
        return list(out[:n])

    def read(self, max_results: int = 0):
        """(counters dict, per-key results of the last call); waits for the
        current stream."""
        from .ops import _stream
        st = _lib.DPlanStats()
        res = (_lib.CacheResult * max(max_results, 1))()
        _lib.check(self._lib.locali_dplan_read(self.state.data_ptr(), ctypes.byref(st), res, max_results,
                                                 _stream()),
                   "locali_dplan_read")
        counters = {f: getattr(st, f) for f, _ in _lib.DPlanStats._fields_}
        n = min(max_results, st.last_keys)
        return counters, [CacheResult(r.key, r.slot, r.evicted_key, bool(r.hit), bool(r.placed))
                          for r in res[:n]]

    def peek(self, key: int) -> int:
        from .ops import _stream
        return int(self._lib.locali_dplan_peek(self.state.data_ptr(), key, _stream()))
