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
