"""The HBM expert arena: slot pools per tier, a slot planner, and bounded
asynchronous fills from the checkpoint files.

Mirrors the reference's ArenaStore / ArenaMoE (arena.py:64-681) for a GPU
with its own memory: the arena is a set of slot-major device tensors
[n_slots, *shape] per (tier, projection, array) -- exactly the layout the
expert kernels index by slot -- and a miss is a preadv of the expert's nine
records into pinned host staging followed by an asynchronous host -> HBM copy
on a dedicated fill stream (one copy-kernel launch for the nine records). With
host_source (the experts' records already in pinned host memory) a call's
misses are copied by one launch on the caller's stream (demand) or the fill
stream (prefetch). Slot 0 of every tier is reserved and all-zero: a
masked-out route reads it and contributes exactly 0.

Slots are claimed synchronously by the planner (so a later submit cannot
steal a slot an earlier one is still filling); only the reads and copies are
deferred to a thread pool, and a fill's future completes once its copy has
landed in HBM. `pinned` keeps the slots of the layer being computed out of the
victim search while a cross-layer prefetch claims slots; `inflight` maps a
resident key to the fills still writing it.

The planner is the compiled one (locali_amd.native, the reference C ABI) in
V4ArenaStore. For native_scheduler=False this base class plans with a slot
ledger of its own (_SlotLedger: per-slot holder, segment and recency stamp)
that follows the rules of the reference's Python fallback planner
(arena.py:212-354): a call's hits resolve before its misses.
"""

from __future__ import annotations

import json
import os
import threading
import time
from collections import Counter
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

PROJS = ("gate_proj", "up_proj", "down_proj")
ARRS = ("weight", "scales", "biases")
TORCH_DT = {"U32": torch.int32, "I32": torch.int32, "F16": torch.float16, "BF16": torch.bfloat16,
            "F32": torch.float32, "U8": torch.uint8}
POLICIES = ("lru", "slru-cold", "slru-all", "lfu-decay")


@dataclass(frozen=True)
class TierGeometry:
    """Shape of one tier's slot pool."""
    expert_bytes: int   # one expert's nine records
    slots: int          # slot 0 (the zero expert) included
    protected: int      # SLRU protected-segment capacity (0: plain LRU)
    arrays: dict        # (proj, array) -> (bytes per slot, shape, dtype name)


def tier_geometry(meta, ceiling: int, hot_share: float, cache_policy: str) -> dict:
    """{tier: TierGeometry} for an index's experts under a byte ceiling
    (reference arena.py:100-165).

    Every expert of a tier has the same nine arrays, so the first expert the
    index lists for a tier fixes its shapes; the search stops once two tiers
    (hot and cold) are seen. A lone tier gets the whole ceiling; hot and cold
    get hot_share and the rest; each holds as many whole experts as its bytes
    allow, the reserved zero slot counted in. Under slru-all every tier, under
    slru-cold only the cold one, keeps (slots - 1) // 2 slots for protected
    entries."""
    first: dict = {}
    for m in meta.values():
        if m["tier"] not in first:
            first[m["tier"]] = m
            if len(first) == 2:
                break
    names = sorted(first)
    out = {}
    for t in names:
        if len(names) == 1:
            frac = 1.0
        else:
            frac = {"hot": hot_share, "cold": 1.0 - hot_share}.get(t, 0.5)
        arrays = {(p, k): (int(first[t][p][k][3]), tuple(first[t][p][k][4]), first[t][p][k][5])
                  for p in PROJS for k in ARRS}
        per = sum(nb for nb, _, _ in arrays.values())
        n = int(ceiling * frac / per)
        slru = cache_policy == "slru-all" or (cache_policy == "slru-cold" and t == "cold")
        out[t] = TierGeometry(per, n, (n - 1) // 2 if slru and n > 0 else 0, arrays)
    return out


class _SlotLedger:
    """The Python planner's record of one tier's slots: the key each slot
    holds, the SLRU segment it sits in and a recency stamp.

    New keys enter probation. A demand hit on a probation entry moves it to
    the protected segment (when the tier has one); once that segment is over
    capacity its least recently used entry drops back to probation. A
    segment's least recently used entry is its smallest stamp (a counter
    bumped on every entry and refresh). Slots never used yet are handed out
    from the highest number down, and only while probation has room; slot 0
    is the reserved zero expert and is never handed out."""

    PROBATION, PROTECTED = 1, 2

    def __init__(self, n_slots: int, protected_cap: int):
        self.protected_cap = protected_cap
        self.probation_cap = n_slots - 1 - protected_cap
        self.holder: list = [None] * n_slots
        self.segment = np.zeros(n_slots, dtype=np.int8)     # 0: never used
        self.stamp = np.zeros(n_slots, dtype=np.int64)
        self.slot_of: dict = {}
        self.unused = n_slots - 1
        self.size = {self.PROBATION: 0, self.PROTECTED: 0}
        self.clock = 0

    def lookup(self, key):
        return self.slot_of.get(key)

    def _enter(self, slot: int, segment: int) -> None:
        if self.segment[slot]:
            self.size[int(self.segment[slot])] -= 1
        self.segment[slot] = segment
        self.size[segment] += 1
        self.clock += 1
        self.stamp[slot] = self.clock

    def _oldest(self, segment: int, held=()):
        cand = np.flatnonzero(self.segment == segment)
        if held:
            cand = cand[~np.isin(cand, np.fromiter(held, dtype=np.int64))]
        return int(cand[np.argmin(self.stamp[cand])]) if cand.size else None

    def refresh(self, key) -> None:
        """A demand hit: the entry becomes the most recent of its segment, or
        moves from probation to the protected segment."""
        slot = self.slot_of[key]
        if self.segment[slot] == self.PROTECTED or self.protected_cap == 0:
            self._enter(slot, int(self.segment[slot]))
            return
        self._enter(slot, self.PROTECTED)
        if self.size[self.PROTECTED] > self.protected_cap:
            self._enter(self._oldest(self.PROTECTED), self.PROBATION)

    def claim(self, key, held):
        """(slot, evicted key or None) for a key not resident, never taking a
        slot in `held`; (None, None) when every candidate is held."""
        if self.unused and self.size[self.PROBATION] < self.probation_cap:
            slot, evicted = self.unused, None
            self.unused -= 1
        else:
            slot = self._oldest(self.PROBATION, held)
            if slot is None:
                slot = self._oldest(self.PROTECTED, held)
            if slot is None:
                return None, None
            evicted = self.holder[slot]
            del self.slot_of[evicted]
        self.holder[slot] = key
        self.slot_of[key] = slot
        self._enter(slot, self.PROBATION)
        return slot, evicted

    @property
    def protected_size(self) -> int:
        return self.size[self.PROTECTED]


class ReadPlan(dict):
    """Per-tier futures plus the experts whose slots are not filled yet
    (reference arena.py:55-61)."""

    def __init__(self, *args, pending_experts=(), **kwargs):
        super().__init__(*args, **kwargs)
        self.pending_experts = frozenset(pending_experts)


class _Landed:
    """Future of a fill copied from pinned host memory: an event recorded on
    the stream that ran the experts' copies (`stream`, its raw handle). It
    holds the source tensors until the event has passed (the copy kernel
    reads them asynchronously), so a host_source that hands out fresh pinned
    tensors stays correct."""

    def __init__(self, event, sources=(), stream=None):
        self.event = event
        self.sources = list(sources)
        self.stream = stream

    def done(self) -> bool:
        if self.event.query():
            self.sources.clear()
            return True
        return False

    def result(self, timeout=None):
        self.event.synchronize()
        self.sources.clear()


class _SlotFills:
    """The latest host fill queued into each (tier, slot): a copy into a slot
    on one stream first waits for the previous copy into it when that one
    ran on the other stream and may still be pending."""

    def __init__(self):
        self.by_slot: dict = {}

    def pop_slots(self, t, slots):
        out = []
        for s in slots:
            f = self.by_slot.pop((t, s), None)
            if f is not None:
                out.append(f)
        return out

    def note(self, t, slots, landed):
        for s in slots:
            self.by_slot[(t, s)] = landed


class _Staging:
    """A small pool of pinned host buffers, one expert each."""

    def __init__(self, nbytes: int, count: int, pinned: bool):
        self.free = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=pinned) for _ in range(count)]
        self.cv = threading.Condition()

    def take(self) -> torch.Tensor:
        with self.cv:
            while not self.free:
                self.cv.wait()
            return self.free.pop()

    def give(self, buf: torch.Tensor) -> None:
        with self.cv:
            self.free.append(buf)
            self.cv.notify()


class ArenaStore:
    def __init__(self, index_path, ceiling_gb=8.0, hot_share=0.33, threads=8, nocache=True,
                 cache_policy="lru", device=None, host_source=None):
        idx = json.loads(Path(index_path).read_text())
        # host_source(layer, expert) -> pinned uint8 host tensor holding the
        # expert's nine records back to back in (gate, up, down) x (weight,
        # scales, biases) order: misses then copy straight from host memory
        # (a host tier for hosts whose RAM holds the experts) instead of
        # reading the checkpoint files. The tensor must stay alive until the
        # fill's future is done (the copy reads it asynchronously).
        self.host_source = host_source
        if cache_policy not in POLICIES:
            raise ValueError(f"cache_policy must be one of {POLICIES}")
        self.meta = idx["experts"]
        self.layers, self.E = int(idx["layers"]), int(idx["num_experts"])
        self.top_k = int(idx["top_k"])
        self.cache_policy = cache_policy
        self.ceiling = int(ceiling_gb * 1e9)
        self.tier_overlap = bool(idx.get("pack"))
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self._nocache = nocache
        self.fds: dict = {}
        self._fd_lock = threading.Lock()
        self.pool = ThreadPoolExecutor(max_workers=threads)
        self.hits = self.misses = self.evictions = self.bytes_read = 0
        self.t_stall = 0.0
        self.pinned: dict = {}
        self.inflight: dict = {}
        self.pf_keys: set = set()
        self.prefetched = self.prefetch_used = self.prefetch_wasted = 0

        geometry = tier_geometry(self.meta, self.ceiling, hot_share, cache_policy)
        self.tiers = sorted(geometry)
        self.arena, self.item, self.slots, self.protected_cap = {}, {}, {}, {}
        self.ledger = {}   # tier -> _SlotLedger (the Python planner's state)
        self.layout = {}   # (tier, proj, array) -> (nbytes per slot, shape, dtype name)
        for t in self.tiers:
            g = geometry[t]
            if g.slots < 2:
                raise ValueError(f"{ceiling_gb:.3f} GB gives tier {t} no usable expert slot after "
                                 "its reserved zero slot; raise ceiling_gb or adjust hot_share")
            n = self.slots[t] = g.slots
            self.item[t] = g.expert_bytes
            self.protected_cap[t] = g.protected
            self.ledger[t] = _SlotLedger(n, g.protected)
            for (p, k), (nb, shape, dt) in g.arrays.items():
                if dt not in TORCH_DT:
                    raise ValueError(f"tier {t} {p}.{k}: unsupported dtype {dt}")
                self.layout[(t, p, k)] = (nb, shape, dt)
                # zero-filled: slot 0 stays the all-zero expert
                self.arena[(t, p, k)] = torch.zeros((n, *shape), dtype=TORCH_DT[dt],
                                                    device=self.device)
        self.resident = sum(self.slots[t] * self.item[t] for t in self.tiers)
        if self.resident > self.ceiling:
            raise AssertionError(f"arena allocated {self.resident} bytes against {self.ceiling}")
        gpu = self.device.type == "cuda"
        self.fill_stream = torch.cuda.Stream(device=self.device) if gpu else None
        self._slot_fills = _SlotFills()
        self.staging = _Staging(max(self.item.values()), max(2, threads), pinned=gpu)

    # ---- kernel views ----------------------------------------------------
    def group_size(self, t) -> int:
        """Quantisation group of tier t (the index's, else the reference
        arena's fixed 64, arena.py:51)."""
        return 64

    def expert_arena(self, t):
        """The tier's slot arrays as the expert kernels take them; bits per
        projection follow from the packed and metadata widths."""
        from .ops import ExpertArenaT, ProjArena
        cache = self.__dict__.setdefault("_expert_arena", {})
        if t not in cache:
            g = self.group_size(t)
            projs = []
            for p in PROJS:
                w = self.arena[(t, p, "weight")]
                sc = self.arena[(t, p, "scales")]
                cols = sc.shape[-1] * g
                if (w.shape[-1] * 32) % cols:
                    raise ValueError(f"tier {t} {p}: packed width {w.shape[-1]} does not fit "
                                     f"{cols} inputs")
                projs.append(ProjArena(w, sc, self.arena[(t, p, "biases")],
                                       w.shape[-1] * 32 // cols, g))
            cache[t] = ExpertArenaT(*projs)
        return cache[t]

    def use_f16(self, t) -> bool:
        """Tier t keeps fp16 scales/biases: bf16 activations are cast to fp16
        before its experts (reference dsv4_arena.py:30-40, 172-173)."""
        return all(self.layout[(t, p, k)][2] == "F16" for p in PROJS for k in ("scales", "biases"))

    def slot_identity(self, t) -> torch.Tensor:
        cache = self.__dict__.setdefault("_slot_ident", {})
        if t not in cache:
            cache[t] = torch.arange(self.slots[t], dtype=torch.int32, device=self.device)
        return cache[t]

    # ---- files ---------------------------------------------------------
    def _fd(self, root, shard):
        key = (root, shard)
        with self._fd_lock:
            if key not in self.fds:
                self.fds[key] = os.open(os.path.join(root, shard), os.O_RDONLY)
            return self.fds[key]

    def tier(self, layer, expert):
        return self.meta[f"L{layer}.E{expert}"]["tier"]

    def _records(self, layer, expert, t):
        m = self.meta[f"L{layer}.E{expert}"]
        recs = [m[p][k] for p in PROJS for k in ARRS]
        for (p, k), rec in zip(((p, k) for p in PROJS for k in ARRS), recs):
            if rec[3] != self.layout[(t, p, k)][0]:
                raise ValueError(f"L{layer}.E{expert} {p}.{k}: {rec[3]} bytes, slot holds "
                                 f"{self.layout[(t, p, k)][0]}")
        return recs

    @staticmethod
    def _contiguous(recs):
        root, shard, end = recs[0][0], recs[0][1], recs[0][2]
        for r in recs:
            if (r[0], r[1], r[2]) != (root, shard, end):
                return False
            end += r[3]
        return True

    def _read(self, recs, host: np.ndarray) -> None:
        """preadv the nine records into consecutive ranges of `host`: one call
        for an expert-major packed expert, one per record otherwise."""
        views, off = [], 0
        for r in recs:
            views.append(memoryview(host[off:off + r[3]]))
            off += r[3]
        groups = [list(range(len(recs)))] if self._contiguous(recs) else [[i] for i in range(len(recs))]
        for g in groups:
            r0 = recs[g[0]]
            fd = self._fd(r0[0], r0[1])
            want = sum(recs[i][3] for i in g)
            got = os.preadv(fd, [views[i] for i in g], r0[2])
            if got != want:
                raise IOError(f"short read {got}/{want} at {r0[1]}+{r0[2]}")
            if self._nocache and hasattr(os, "posix_fadvise"):
                os.posix_fadvise(fd, r0[2], want, os.POSIX_FADV_DONTNEED)

    def _fill(self, t, slot, recs, key=None) -> None:
        """Worker: file -> pinned staging -> HBM slot; returns once the bytes
        are in device memory. A host-memory arena copies from host_source."""
        if self.host_source is not None:
            src, off = self._host_bytes(key, t), 0
            for (p, k), r in zip(((p, k) for p in PROJS for k in ARRS), recs):
                self.arena[(t, p, k)][slot].view(torch.uint8).reshape(-1).copy_(src[off:off + r[3]])
                off += r[3]
            return
        buf = self.staging.take()
        try:
            host = buf.numpy()
            self._read(recs, host)
            off = 0
            if self.fill_stream is not None:
                from .ops import arena_fill_slots
                with torch.cuda.device(self.device):
                    arena_fill_slots(self._slot_table(t), [slot], [buf.data_ptr()], self.fill_stream)
                    ev = torch.cuda.Event()
                    ev.record(self.fill_stream)
                ev.synchronize()
            else:
                for (p, k), r in zip(((p, k) for p in PROJS for k in ARRS), recs):
                    dst = self.arena[(t, p, k)][slot].view(torch.uint8).reshape(-1)
                    dst.copy_(buf[off:off + r[3]])
                    off += r[3]
        finally:
            self.staging.give(buf)

    def _mark_demand(self):
        """Record, on the caller's stream, the point before a demand call's
        fills and gather (see _fill_from_host)."""
        from .ops import current_stream
        mark = self.__dict__.get("_demand_mark")
        if mark is None:
            mark = self._demand_mark = torch.cuda.Event()
        cur = current_stream(self.device)
        mark.record(cur)
        self._demand_stream = cur.cuda_stream

    def _slot_table(self, t):
        """Tier t's nine slot-major arrays in record order (gate, up, down) x
        (weight, scales, biases), as ops.arena_fill_slots takes them."""
        from .ops import slot_table
        cache = self.__dict__.setdefault("_slot_tables", {})
        if t not in cache:
            cache[t] = slot_table([self.arena[(t, p, k)] for p in PROJS for k in ARRS])
        return cache[t]

    def _host_bytes(self, key, t) -> torch.Tensor:
        src = self.host_source(*key)
        if (src.is_cuda or src.dtype != torch.uint8 or src.numel() != self.item[t]
                or not src.is_contiguous()):
            raise ValueError(f"host_source{key}: expected {self.item[t]} contiguous host bytes (uint8)")
        return src

    def _fill_from_host(self, jobs, on_caller_stream=False) -> _Landed:
        """Queue the host -> HBM copies of several experts' records from
        host_source as one batch and return the future of their event.
        jobs: (key, tier, slot, recs), one tier.

        on_caller_stream: the copies run on the caller's current stream, in
        order with the work around them (a demand call's fills, which its own
        gather needs next). Otherwise they run on the fill stream, behind the
        caller's work that may still read a slot they overwrite: everything
        queued before the latest demand call (its mark). What that call queued
        after its mark -- its own fills and gather -- touches only its own
        slots, which stay pinned until the next demand call, so a copy on the
        fill stream never takes one of them. Without a demand mark on the
        caller's current stream the copies wait for everything queued on that
        stream. Either way a copy
        into a slot waits for the pending fill of that slot's previous owner
        when it ran on the other stream."""
        from .ops import arena_fill_slots, current_stream
        if self.device.index is not None and torch.cuda.current_device() != self.device.index:
            with torch.cuda.device(self.device):
                return self._fill_from_host(jobs, on_caller_stream)
        t = jobs[0][1]                   # the caller batches one tier at a time
        sources = [self._host_bytes(key, t) for key, _, _, _ in jobs]
        cur = current_stream(self.device)
        stream = cur if on_caller_stream else self.fill_stream
        for f in self._slot_fills.pop_slots(t, [slot for _, _, slot, _ in jobs]):
            if f.stream != stream.cuda_stream and not f.done():
                stream.wait_event(f.event)
        if not on_caller_stream:
            mark = self.__dict__.get("_demand_mark")
            if mark is not None and self._demand_stream == cur.cuda_stream:
                if not mark.query():
                    self.fill_stream.wait_event(mark)
            elif not cur.query():
                # one reused event (a wait takes the event's state when it is
                # queued); a stream with nothing left to run needs no wait
                order = self.__dict__.get("_order_event")
                if order is None:
                    order = self._order_event = torch.cuda.Event()
                order.record(cur)
                self.fill_stream.wait_event(order)
        arena_fill_slots(self._slot_table(t), [slot for _, _, slot, _ in jobs],
                         [src.data_ptr() for src in sources], stream)
        ev = torch.cuda.Event()
        ev.record(stream)
        landed = _Landed(ev, sources, stream.cuda_stream)
        self._slot_fills.note(t, [slot for _, _, slot, _ in jobs], landed)
        return landed

    # ---- Python planner (native_scheduler=False) ----------------------------
    def _evicted(self, victim):
        self.inflight.pop(victim, None)
        if victim in self.pf_keys:
            self.pf_keys.discard(victim)
            self.prefetch_wasted += 1
        self.evictions += 1

    def _protected_size(self, t):
        return self.ledger[t].protected_size

    def _hit(self, key, t, prefetch, waits):
        if not prefetch:
            self.hits += 1
            if key in self.pf_keys:
                self.pf_keys.discard(key)
                self.prefetch_used += 1
        futs = self.inflight.get(key)
        if futs:
            if all(f.done() for f in futs):
                del self.inflight[key]
            elif not prefetch:
                waits[t].extend(futs)

    def _place_keys(self, layer, want, prefetch):
        """The Python planner's placement of a layer's unique experts
        (the reference's fallback planner, arena.py:212-354): the resident
        ones are resolved first (a demand hit refreshes its entry), then the
        misses take slots in call order; no miss takes a slot that the
        previous demand call or this call already holds. Returns (placed,
        issued fills, fills to wait for)."""
        out, issued, misses = {}, [], []
        waits = {t: [] for t in self.tiers}
        held = {t: set() for t in self.tiers}
        for e in want:
            key, t = (layer, e), self.tier(layer, e)
            slot = self.ledger[t].lookup(key)
            if slot is None:
                misses.append((e, t))
                continue
            out[e] = (t, slot)
            held[t].add(slot)
            if not prefetch:
                self.ledger[t].refresh(key)
            self._hit(key, t, prefetch, waits)
        if not prefetch:
            self.misses += len(misses)
            for t, n in Counter(t for _, t in misses).items():
                if n > self.slots[t] - 1:
                    raise ValueError(f"layer {layer} needs {n} {t} experts but the arena has "
                                     f"{self.slots[t] - 1}; raise ceiling_gb or hot_share")
        for e, t in misses:
            slot, evicted = self.ledger[t].claim((layer, e), held[t] | set(self.pinned.get(t, ())))
            if slot is None:
                continue
            if evicted is not None:
                self._evicted(evicted)
            out[e] = (t, slot)
            held[t].add(slot)
            issued.append((e, t, slot))
        if not prefetch:
            self.pinned = held
        return out, issued, waits

    # ---- public surface (reference arena.py:291-457) ---------------------
    def submit(self, layer, experts, prefetch=False, fills_on_caller_stream=None):
        """Claim slots now; queue the fills; return ({expert: (tier, slot)},
        ReadPlan). prefetch=True is best effort: it never evicts a pinned slot,
        never raises on a full arena and leaves hit/miss accounting alone.

        Copies from host memory run on the caller's current stream for a
        demand call and on the fill stream for a prefetch, unless
        fills_on_caller_stream says otherwise (a call that overlaps its hits
        with its misses wants its fills beside its own stream)."""
        if fills_on_caller_stream is None:
            fills_on_caller_stream = not prefetch
        want = list(dict.fromkeys(int(e) for e in experts))
        out, issued, waits = self._place_keys(layer, want, prefetch)
        # A later miss of the same call may have taken an earlier one's slot
        # (only when the tier is nearly all pinned): that earlier claim is
        # stale and must not be filled or used.
        owner = {}
        for e, t, s in issued:
            owner[(t, s)] = e
        stale = [e for e, t, s in issued if owner[(t, s)] != e]
        if stale:
            if not prefetch:
                raise RuntimeError(f"layer {layer}: the arena cannot hold this call's experts "
                                   "next to the previous call's pinned slots; raise ceiling_gb")
            issued = [(e, t, s) for e, t, s in issued if owner[(t, s)] == e]
            for e in stale:
                out.pop(e, None)
        plan = ReadPlan()
        jobs = {t: [] for t in self.tiers}
        from_host = self.host_source is not None and self.fill_stream is not None
        if from_host and not prefetch:
            self._mark_demand()
        for e, t, s in issued:
            # a copy from host memory moves the whole expert; a file read
            # follows its records
            jobs[t].append(((layer, e), t, s, None if from_host else self._records(layer, e, t)))
            self.bytes_read += self.item[t]
        for t in self.tiers:   # a whole tier before the next
            futs = []
            batch = (self._fill_from_host(jobs[t], fills_on_caller_stream)
                     if jobs[t] and from_host else None)
            for key, tt, s, recs in jobs[t]:
                f = batch if batch is not None else self.pool.submit(self._fill, tt, s, recs, key)
                self.inflight.setdefault(key, []).append(f)
                futs.append(f)
            plan[t] = futs + waits[t]
        plan.pending_experts = frozenset(
            e for e in want if any(not f.done() for f in self.inflight.get((layer, e), ())))
        if prefetch:
            self.prefetched += len(issued)
            self.pf_keys.update((layer, e) for e, _, _ in issued)
        return out, plan

    def slots_for(self, layer, experts):
        """{expert: (tier, slot)}, every one resident in HBM on return."""
        placed, plan = self.submit(layer, experts)
        self.wait([f for futs in plan.values() for f in futs])
        return placed

    def wait(self, futs):
        """Every fill in futs has landed before work queued afterwards on the
        caller's current stream reads it. Copies from host memory are ordered
        on the device (copies queued on this stream already are; for others
        the stream waits for their event) and the host goes on; file reads
        block the host until their copies have landed."""
        if not futs:
            return
        from .ops import current_stream
        t0 = time.perf_counter()
        seen, cur = set(), None
        for f in futs:
            if isinstance(f, _Landed):
                if id(f) not in seen:
                    seen.add(id(f))
                    cur = cur or current_stream(self.device)
                    # copies queued on this very stream are already in order
                    if f.stream != cur.cuda_stream and not f.done():
                        cur.wait_event(f.event)
            else:
                f.result()
        self.t_stall += time.perf_counter() - t0

    def reset_stats(self):
        """Zero the hit, miss, eviction, byte, stall and prefetch counters."""
        self.hits = self.misses = self.evictions = self.bytes_read = 0
        self.prefetched = self.prefetch_used = self.prefetch_wasted = 0
        self.t_stall = 0.0

    def stats(self):
        n = self.hits + self.misses
        return {"hits": self.hits, "misses": self.misses, "hit_rate": self.hits / n if n else 0.0,
                "evictions": self.evictions, "bytes_read": self.bytes_read,
                "resident": self.resident, "peak": self.resident,
                "slots": {t: self.slots[t] for t in self.tiers},
                "t_stall": self.t_stall, "t_convert": 0.0, "t_eval": 0.0,
                "prefetched": self.prefetched, "prefetch_used": self.prefetch_used,
                "prefetch_wasted": self.prefetch_wasted, "cache_policy": self.cache_policy,
                "protected": {t: self._protected_size(t) for t in self.tiers}}

    def close(self):
        """Drain the fills, close the files and release the arena's memory."""
        self.pool.shutdown(wait=True)
        if self.fill_stream is not None:
            # fills from host memory are queued on the device only (the fill
            # stream's and the callers' streams): they must have landed before
            # the arena's memory goes back to the allocator
            torch.cuda.synchronize(self.device)
        self._slot_fills.by_slot.clear()
        for fd in self.fds.values():
            os.close(fd)
        self.fds.clear()
        self.arena.clear()
        self.__dict__.pop("_expert_arena", None)
        self.__dict__.pop("_slot_tables", None)
        self.staging.free.clear()


def _host_ints(tensors):
    """Host numpy int32 copies of 32-bit tensors, through one device-to-host
    copy (fp32 values travel as their bits)."""
    flat = [t.reshape(-1).to(torch.float32 if t.is_floating_point() else torch.int32).view(torch.int32)
            for t in tensors]
    host = torch.cat(flat).cpu().numpy()
    out, off = [], 0
    for t in flat:
        out.append(host[off:off + t.numel()])
        off += t.numel()
    return out


def _lookahead_experts(idx, weight_bits, top_k, k=None):
    """The experts a prefetch asks for: per row of the lookahead routing,
    the k highest gate weights (all top_k when k is unset or not smaller),
    ties in row order (reference arena.py:527-532). idx and weight_bits are
    the host int32 arrays of _host_ints (weights as fp32 bits)."""
    pi = idx.reshape(-1, top_k)
    if k and k < top_k:
        pg = weight_bits.view(np.float32).reshape(-1, top_k)
        order = np.argsort(-pg, axis=-1, kind="stable")
        pi = np.take_along_axis(pi, order[:, :k], axis=-1)
    return pi.reshape(-1).tolist()


class ArenaMoE:
    """Locali's own MoE module over the arena (reference arena.py:460-547):
    sigmoid router with a selection-only bias, top-k renormalised, weights in
    x.dtype. Subclasses replace route() (the V4 gate) and keep __call__."""

    def __init__(self, store: ArenaStore, layer: int, gate, bias, top_k: int):
        self.store, self.layer, self.gate, self.bias, self.top_k = store, layer, gate, bias, top_k
        self.scores_follow_output = False
        self.nxt = None          # next layer's module, for cross-layer prefetch
        self.nxt2 = None         # depth-2 lookahead
        self.prefetch_k = None   # prefetch only the highest-gate candidates
        self.prefetch_k2 = None
        self.overlap_hits = False
        self.swiglu_limit = 0.0
        self.fp32_swiglu = False
        self.shared_expert = None
        self._spec = None

    def route(self, x, input_ids=None):
        """(indices int32 [T, k], scores fp32 [T, k]) from the sigmoid router."""
        from . import ops
        if self._spec is None:
            w = self.gate.weight if hasattr(self.gate, "weight") else self.gate
            bias = None if self.bias is None else self.bias.to(device=w.device, dtype=torch.float32)
            self._spec = ops.RouterSpec(w, self.top_k, score_func="sigmoid", norm_topk=True,
                                        routed_scale=1.0, score_bias=bias)
        idx, w, _ = ops.router(self._spec, x.reshape(-1, x.shape[-1]), self._workspace())
        return idx, w

    def _workspace(self):
        from . import ops
        ws = getattr(self.store, "workspace", None)
        if ws is None:
            ws = self.store.workspace = ops.Workspace(self.store.device)
        return ws

    def __call__(self, x, input_ids=None):
        shape = x.shape
        flat = x.reshape(-1, shape[-1])
        if flat.shape[0] == 0:        # no tokens: an empty output, nothing routed or placed
            return torch.zeros(shape, dtype=x.dtype, device=x.device)
        inds, gates = self.route(x, input_ids)
        # The lookahead routing of the cross-layer prefetch (reference
        # arena.py:518-541) is a function of x alone: it is launched with this
        # layer's and all of it reaches the host in one copy and one wait.
        ahead = [(blk, k) + blk.route(x, input_ids)
                 for blk, k in ((self.nxt, self.prefetch_k), (self.nxt2, self.prefetch_k2))
                 if blk is not None]
        if ahead:
            parts = _host_ints([inds] + [t for a in ahead for t in a[2:]])
            ii = parts[0].reshape(-1, self.top_k).tolist()
        else:
            ii = inds.reshape(-1, self.top_k).tolist()      # host sync, as the reference
        experts = [e for row in ii for e in row]
        # Planner calls in the reference's order: this layer's demand, then
        # the prefetch, nearest layer first. Without tier overlap the gather
        # waits for every demand fill (slots_for's order, reference
        # arena.py:513-516). When fills are copies from host memory the waits
        # are on the device, so the gather is queued before the prefetch is
        # planned (the prefetch never takes this call's slots: they are
        # pinned); file reads block the host in the wait, so their prefetch
        # is queued first, beside the demand reads, as in the reference.
        split = self.overlap_hits and self.store.tier_overlap   # hits run beside the fills
        placed, reads = self.store.submit(self.layer, experts, fills_on_caller_stream=not split)
        device_waits = self.store.host_source is not None and self.store.fill_stream is not None

        def prefetch():
            for n, (blk, k, _, _) in enumerate(ahead):
                self.store.submit(blk.layer, _lookahead_experts(parts[1 + 2 * n], parts[2 + 2 * n],
                                                                self.top_k, k), prefetch=True)
        if not device_waits:
            prefetch()
        if not self.store.tier_overlap:
            self.store.wait([f for futs in reads.values() for f in futs])
            reads = None
        out = self._apply(flat, ii, placed, gates.reshape(-1, self.top_k), x.dtype, reads)
        if device_waits:
            prefetch()
        return out.reshape(shape).to(x.dtype)

    def _apply(self, flat, ii, placed, gates, dtype, reads=None):
        from . import ops
        T = len(ii)
        if len(self.store.tiers) == 1:
            t = self.store.tiers[0]
        else:
            present = [t for t in self.store.tiers if any(placed[e][0] == t for row in ii for e in row)]
            if len(present) > 1:
                return self._apply_tiers(flat, ii, placed, gates, dtype, reads, present)
            t = present[0]
        pending = getattr(reads, "pending_experts", ()) if reads is not None else ()
        if self.overlap_hits and T == 1 and pending and len(pending) < self.top_k:
            return self._apply_overlap(flat, ii[0], placed, gates, dtype, reads, t, pending)
        if reads is not None:
            self.store.wait(reads[t])
        slots = self._device_slots([[placed[e][1] for e in row] for row in ii], flat.device)
        return self._run_experts(t, flat, slots, gates, dtype)

    def _gather(self, t, inputs, indices):
        """Unweighted expert outputs of tier t, the reference's gather hook
        (arena.py:674-681, dsv4_arena.py:168-235): inputs [n, 1, 1, d]
        activations and indices [n, k] device slots of tier t give
        [n, k, 1, d], entry (r, j) the expert of slot indices[r, j] applied
        to inputs[r], in the tier's activation dtype (bf16 activations become
        fp16 for a tier of fp16 metadata, as the reference casts them). Each
        route is one row of a one-route call with weight 1, so an entry is
        the expert's down output rounded once to that dtype.

        The module's own calls fuse this with the combine (_run_experts).
        When a subclass overrides _gather, every tier evaluation of __call__
        goes through the override instead, and the library's combine then
        takes its outputs in the order the fused kernels do."""
        n, k = indices.shape
        d = inputs.shape[-1]
        x_in = inputs.reshape(n, d)
        if x_in.dtype == torch.bfloat16 and self.store.use_f16(t):
            x_in = x_in.to(torch.float16)
        rows = x_in.repeat_interleave(k, dim=0).contiguous()
        slots = indices.reshape(n * k, 1).to(torch.int32).contiguous()
        y = self._routes(self.store.expert_arena(t), rows, slots, self._workspace())
        return y.view(n, k, 1, d)

    def _gather_overridden(self) -> bool:
        return type(self)._gather is not ArenaMoE._gather

    def _tier_routes(self, t, x_in, slots, ws):
        """One route per row of x_in through tier t ([n, 1] slots): _routes,
        or the subclass's _gather when it replaces the hook."""
        if self._gather_overridden():
            return self._gather(t, x_in[:, None, None, :], slots).reshape(x_in.shape[0], x_in.shape[-1])
        return self._routes(self.store.expert_arena(t), x_in, slots, ws)

    def _run_experts(self, t, flat, slots, gates, dtype):
        """Tier t's expert kernels over device route slots [T, k]: the decode
        kernels up to two tokens, the slot-grouped kernels beyond."""
        from . import ops
        if self._gather_overridden():
            return self._combine_gathered(t, flat, slots, gates, dtype)
        T = flat.shape[0]
        arena = self.store.expert_arena(t)
        x_in = flat.contiguous()
        if x_in.dtype == torch.bfloat16 and self.store.use_f16(t):
            x_in = x_in.to(torch.float16)
        w = gates.to(torch.float32).contiguous()
        ws = self._workspace()
        if T <= 2:
            y = ops.expert_decode(arena, self.shared_expert, x_in, slots, w, swiglu_limit=self.swiglu_limit,
                                  fp32_swiglu=self.fp32_swiglu, ws=ws)
        else:
            n = arena.n_slots
            ident = self.store.slot_identity(t)
            y = ops.expert_grouped(arena, self.shared_expert, x_in, slots, ident, w, ws, n_experts=n,
                                   swiglu_limit=self.swiglu_limit, fp32_swiglu=self.fp32_swiglu)
        return y.to(dtype)

    def _combine_gathered(self, t, flat, slots, gates, dtype):
        """The [T, k] routes through a subclass's _gather, then the single-tier
        combine the fused kernels apply (each product of y and the rounded
        weight rounded, summed in float32, one rounding), then the folded
        shared expert with one more rounding."""
        from . import ops
        T, k = slots.shape
        x_in = flat.contiguous()
        if x_in.dtype == torch.bfloat16 and self.store.use_f16(t):
            x_in = x_in.to(torch.float16)
        y = self._gather(t, x_in[:, None, None, :], slots).reshape(T * k, -1).to(x_in.dtype)
        route_pos = torch.arange(T * k, dtype=torch.int32, device=flat.device).view(T, k)
        shared_y = None
        if self.shared_expert is not None:
            zero = torch.zeros(T, 1, dtype=torch.int32, device=flat.device)
            shared_y = self._routes(self.shared_expert, x_in, zero, self._workspace())
        out = ops.combine_routes(y, route_pos, gates.to(torch.float32).contiguous(), x_in.dtype,
                                 shared_y=shared_y, mode=ops.COMBINE_ROUNDED)
        return out.to(dtype)

    def _device_slots(self, rows, device):
        """[T, k] int32 slots on the device by an asynchronous copy from a
        small ring of pinned host buffers (a copy from pageable memory would
        block the host behind everything queued on the stream, fills
        included). Each layer call syncs on its routing before it plans, so a
        buffer is reused only after the copies of earlier calls have run."""
        flat = [s for row in rows for s in row]
        if device.type != "cuda":
            return torch.tensor(rows, dtype=torch.int32, device=device)
        from .ops import current_stream
        ring = self.__dict__.setdefault("_slot_ring", [])
        if not ring or ring[0][0].numel() < len(flat):
            n = max(64, len(flat))
            ring[:] = [[torch.empty(n, dtype=torch.int32, pin_memory=True), None, None] for _ in range(4)]
            for entry in ring:
                entry[2] = entry[0].numpy()
            self._slot_next = 0
        entry = ring[self._slot_next]
        self._slot_next = (self._slot_next + 1) % len(ring)
        if entry[1] is not None:
            entry[1].synchronize()        # the buffer's previous copy has run
        entry[2][:len(flat)] = flat
        out = entry[0][:len(flat)].to(device, non_blocking=True).view(len(rows), -1)
        entry[1] = torch.cuda.Event()
        entry[1].record(current_stream(device))
        return out

    def _routes(self, arena, x_in, slots, ws):
        """Unweighted expert outputs, one route per row of x_in: a one-route
        call with weight 1 returns the route's down output rounded to x_in's
        dtype."""
        from . import ops
        n = x_in.shape[0]
        ones = torch.ones(n, 1, dtype=torch.float32, device=x_in.device)
        kw = dict(swiglu_limit=self.swiglu_limit, fp32_swiglu=self.fp32_swiglu)
        if n <= 2:
            return ops.expert_decode(arena, None, x_in, slots, ones, ws=ws, **kw)
        ident = torch.arange(arena.n_slots, dtype=torch.int32, device=x_in.device)
        return ops.expert_grouped(arena, None, x_in, slots, ident, ones, ws, n_experts=arena.n_slots, **kw)

    def _apply_overlap(self, flat, row, placed, gates, dtype, reads, t, pending):
        """One token with some experts still filling (reference
        arena.py:575-618): the routes whose slots are resident are launched
        before the host blocks on the pending fills, the others after. The
        per-route outputs then meet in the library's combine in k order with
        the kernels' single-tier rounding (products of y and the rounded
        weight rounded, summed in float32, one rounding, then the folded
        shared expert with one more), so the result is bit-identical to the
        unsplit call."""
        from . import ops
        dev = flat.device
        ready = [j for j, e in enumerate(row) if e not in pending]
        late = [j for j, e in enumerate(row) if e in pending]
        x_in = flat.contiguous()
        if self.store.use_f16(t) and x_in.dtype == torch.bfloat16:
            x_in = x_in.to(torch.float16)
        ws = self._workspace()

        def run(pos):
            slots = self._device_slots([[placed[row[j]][1]] for j in pos], dev)
            return self._tier_routes(t, x_in.expand(len(pos), -1).contiguous(), slots, ws)

        y_ready = run(ready)
        self.store.wait(reads[t])
        y = torch.cat([y_ready, run(late)])            # rows: the ready routes, then the late ones
        where = {j: i for i, j in enumerate(ready + late)}
        route_pos = self._device_slots([[where[j] for j in range(len(row))]], dev)
        ys = None
        if self.shared_expert is not None:
            zero = torch.zeros(1, 1, dtype=torch.int32, device=dev)
            ys = self._routes(self.shared_expert, x_in, zero, ws)
        out = ops.combine_routes(y, route_pos, gates.reshape(-1)[:len(row)].reshape(1, -1).to(torch.float32),
                                 x_in.dtype, shared_y=ys, mode=ops.COMBINE_ROUNDED)
        return out.to(dtype)

    def _apply_tiers(self, flat, ii, placed, gates, dtype, reads, present):
        """Routes spanning tiers (reference arena.py:626-672). Each tier's
        own (token, k) entries run through that tier's experts, one route per
        entry; the library's combine then takes each token's routes tier by
        tier in the store's tier order and, within a tier, in k order -- the
        reference's row-major entry order of its per-tier scatter-adds --
        with float32 products of y and the score rounded to the activation
        dtype, a float32 sum and one rounding, then the shared expert (when
        folded) with one more."""
        from . import ops
        k = self.top_k
        dev = flat.device
        ws = self._workspace()
        rank = {t: i for i, t in enumerate(present)}
        entry, ys, base = {}, [], 0
        for t in present:
            if reads is not None:
                self.store.wait(reads[t])
            ent = [(r, j) for r, row in enumerate(ii) for j, e in enumerate(row) if placed[e][0] == t]
            rows = self._device_slots([[r for r, _ in ent]], dev).reshape(-1).to(torch.long)
            slots = self._device_slots([[placed[ii[r][j]][1]] for r, j in ent], dev)
            x_in = flat.index_select(0, rows).contiguous()
            if self.store.use_f16(t) and x_in.dtype == torch.bfloat16:
                x_in = x_in.to(torch.float16)
            ys.append(self._tier_routes(t, x_in, slots, ws))
            for i, rj in enumerate(ent):
                entry[rj] = base + i
            base += len(ent)
        order = [sorted(range(k), key=lambda j: (rank[placed[row[j]][0]], j)) for row in ii]
        route_pos = self._device_slots([[entry[(r, j)] for j in order[r]] for r in range(len(ii))], dev)
        perm = self._device_slots(order, dev).to(torch.long)
        w = torch.gather(gates.to(torch.float32), 1, perm).contiguous()
        y = torch.cat(ys) if len({v.dtype for v in ys}) == 1 else torch.cat([v.float() for v in ys])
        shared_y = None
        if self.shared_expert is not None:
            x_s = flat.contiguous()
            if x_s.dtype != self.shared_expert.gate.scales.dtype and x_s.dtype == torch.bfloat16:
                x_s = x_s.to(torch.float16)
            zero = torch.zeros(flat.shape[0], 1, dtype=torch.int32, device=dev)
            shared_y = self._routes(self.shared_expert, x_s, zero, ws).to(dtype)
        return ops.combine_routes(y, route_pos, w, dtype, shared_y=shared_y, mode=ops.COMBINE_FP32)
