"""Pure-Python slot planner -- TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Restates the reference planner one rule at a time:
  * SLRU claim / touch:   native/locali_core.c:79-141, mirrored by the
                          reference's own executable spec
                          tests/test_locali_native.py:11-62 (ReferenceCache)
  * LFU-decay:            native/locali_core.c:143-182 (victim), :250-257
                          (note_token halves hotness every 16th call),
                          :290-293 (hotness/clock bump on every planned key)
  * plan():               native/locali_core.c:259-313 (pin epoch, key order,
                          -3 on the first invalid key with earlier results kept)
Pinned by tests against the compiled reference (oracle/_ref) and its KATs
(native/test_locali_core.c:14-74).
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass

SLRU = 0
LFU_DECAY = 1


@dataclass(frozen=True)
class Result:
    key: int
    slot: int
    evicted_key: int
    hit: bool
    placed: bool


class OraclePlanner:
    def __init__(self, key_capacity: int, slots: int, protected_capacity: int,
                 policy: int = SLRU):
        if (key_capacity <= 0 or slots < 2 or protected_capacity < 0
                or protected_capacity >= slots or policy not in (SLRU, LFU_DECAY)):
            raise ValueError("invalid planner arguments")
        if policy == LFU_DECAY:
            protected_capacity = 0
        self.key_capacity = key_capacity
        self.slots = slots
        self.policy = policy
        self.protected_capacity = protected_capacity
        self.probation_capacity = slots - 1 - protected_capacity
        self.free = list(range(1, slots))          # popped from the end
        self.probation: OrderedDict[int, int] = OrderedDict()  # LRU first
        self.protected: OrderedDict[int, int] = OrderedDict()
        self.hotness = [0] * key_capacity
        self.last_used = [0] * key_capacity
        self.clock = 0
        self.tokens = 0

    # -- queries ---------------------------------------------------------
    def peek(self, key: int) -> int:
        if not 0 <= key < self.key_capacity:
            return -1
        if key in self.probation:
            return self.probation[key]
        return self.protected.get(key, -1)

    @property
    def probation_size(self) -> int:
        return len(self.probation)

    @property
    def protected_size(self) -> int:
        return len(self.protected)

    # -- mutation --------------------------------------------------------
    def note_token(self) -> None:
        if self.policy != LFU_DECAY:
            return
        self.tokens += 1
        if self.tokens % 16:
            return
        self.hotness = [h >> 1 for h in self.hotness]

    def _touch(self, key: int) -> None:
        if key in self.protected:
            self.protected.move_to_end(key)
            return
        if self.protected_capacity == 0:
            self.probation.move_to_end(key)
            return
        slot = self.probation.pop(key)
        self.protected[key] = slot
        if len(self.protected) > self.protected_capacity:
            old, old_slot = self.protected.popitem(last=False)
            self.probation[old] = old_slot

    def _claim_slru(self, key: int, pinned: set[int]):
        probation_full = len(self.probation) >= self.probation_capacity
        victim, source = None, None
        if probation_full or not self.free:
            victim = next((k for k, s in self.probation.items() if s not in pinned), None)
            source = self.probation
        if victim is None and not probation_full and self.free:
            slot, evicted = self.free.pop(), -1
        else:
            if victim is None:
                victim = next((k for k, s in self.protected.items() if s not in pinned), None)
                source = self.protected
            if victim is None:
                return -1, -1, False
            slot, evicted = source.pop(victim), victim
        self.probation[key] = slot
        return slot, evicted, True

    def _claim_lfu(self, key: int, pinned: set[int]):
        if self.free:
            slot, evicted = self.free.pop(), -1
        else:
            candidates = [k for k, s in self.probation.items() if s not in pinned]
            if not candidates:
                return -1, -1, False
            victim = min(candidates, key=lambda k: (self.hotness[k], self.last_used[k]))
            slot, evicted = self.probation.pop(victim), victim
        self.probation[key] = slot
        return slot, evicted, True

    def plan(self, keys, pinned_slots=(), touch_hits: bool = True):
        """Returns (rc, results). rc is 0 or -3 exactly like the C planner."""
        pinned = {s for s in pinned_slots if 0 < s < self.slots}
        out = []
        for key in keys:
            if not 0 <= key < self.key_capacity:
                return -3, out
            if self.policy == LFU_DECAY:
                self.hotness[key] = min(self.hotness[key] + 1, 2**32 - 1)
                self.clock += 1
                self.last_used[key] = self.clock
            slot = self.peek(key)
            if slot >= 0:
                if touch_hits and self.policy == SLRU:
                    self._touch(key)
                out.append(Result(key, slot, -1, True, True))
                continue
            if self.policy == LFU_DECAY:
                slot, evicted, placed = self._claim_lfu(key, pinned)
            else:
                slot, evicted, placed = self._claim_slru(key, pinned)
            out.append(Result(key, slot, evicted, False, placed))
        return 0, out
