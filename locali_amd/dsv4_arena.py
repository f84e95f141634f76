"""DeepSeek-V4 routed experts over the HBM expert arena: the drop-in for the
reference's V4ArenaStore / V4ArenaMoE (dsv4_arena.py:17-235).

The engine seam is unchanged (reference dsv4_engine.py:188-210, 253-261):

    store = V4ArenaStore(index_path, ceiling_gb=..., hot_share=..., threads=...,
                         nocache=..., cache_policy=..., native_scheduler=True)
    moe = V4ArenaMoE(store, layer, gate, top_k, swiglu_limit,
                     fused_decode=..., overlap_hits=...)
    routed = moe(x, input_ids)            # x's shape and dtype
    out = routed + shared_expert(x)       # the caller adds the shared expert

`gate(x, input_ids) -> (indices [..., k], scores [..., k])` is the gate
protocol; V4Gate implements it on the router kernel from the gate's own
tensors (weight, e_score_correction_bias, tid2eid). Expert arithmetic is the
HIP expert kernels (decode GEMV path up to two tokens, slot-grouped path
beyond), with the reference's contract: fp32 accumulation, projections
rounded to the activation dtype, up clipped to +-limit and gate capped at
limit, SiLU(gate) * up op by op in the activation dtype (fp32 with one final
rounding when fp32_swiglu), weights cast to the expert output dtype, terms
rounded, summed in fp32 and rounded.
"""

from __future__ import annotations

import json
from pathlib import Path

import torch

from . import ops
from .arena import PROJS, ArenaMoE, ArenaStore, ReadPlan
from .native import DevicePlanner, NativeCache


class V4ArenaStore(ArenaStore):
    """The arena with V4 affine quantisation metadata validated and the
    compiled planner per tier over layers * E keys (key = layer * E + e)."""

    def __init__(self, index_path, native_scheduler=True, device_planner=False, **kwargs):
        """device_planner: plan on the GPU (native.DevicePlanner) with the
        compiled planner's rules and fill misses from host_source's pinned
        payloads in the same stream, so that V4ArenaMoE calls never wait for
        the host (one tier, host_source required; cross-layer prefetch runs
        on the fill stream; counters are read from the device by stats())."""
        config = json.loads(Path(index_path).read_text())
        self.expert_quant = config.get("quantization", {})
        for tier, q in self.expert_quant.items():
            if q.get("mode", "affine") != "affine":
                raise ValueError(f"DeepSeek V4 streaming requires affine MLX weights, got "
                                 f"{q.get('mode')!r} for tier {tier}")
        super().__init__(index_path, **kwargs)
        self.use_f16_moe = {t: self.use_f16(t) for t in self.tiers}
        self.native_caches = {}
        if native_scheduler:
            policy = "lfu-decay" if self.cache_policy == "lfu-decay" else "slru"
            for t in self.tiers:
                self.native_caches[t] = NativeCache(self.layers * self.E, self.slots[t],
                                                    self.protected_cap[t], policy=policy)
        elif self.cache_policy == "lfu-decay":
            raise RuntimeError("lfu-decay requires the compiled planner")
        self.dplan = None
        if device_planner:
            problem = ("the device planner follows the compiled planner (native_scheduler=True)"
                       if not native_scheduler else
                       "the device planner covers one expert tier filled from host_source"
                       if len(self.tiers) != 1 or self.host_source is None else None)
            if problem:
                self.close()
                raise ValueError(problem)
            t = self.tiers[0]
            self.dplan = DevicePlanner(self.layers * self.E, self.slots[t], self.protected_cap[t],
                                       n_experts=self.E, policy=policy, device=self.device)
            self._dplan_src = None
            self._dplan_base = None
            self._dplan_pinned = 0   # distinct slots of the previous demand call
            self._pf_event = None    # the fill stream's last prefetch call

    def _key_id(self, key):
        layer, expert = key
        return layer * self.E + expert

    def _decode_key(self, key_id):
        return divmod(key_id, self.E)

    def quant(self, tier, field):
        defaults = {"bits": 2, "group_size": 128, "mode": "affine"}
        return self.expert_quant.get(tier, {}).get(field, defaults[field])

    def group_size(self, t) -> int:
        return int(self.quant(t, "group_size"))

    def _place_keys(self, layer, want, prefetch):
        """Planner calls for one layer (reference dsv4_arena.py:68-127): the
        previous demand call's slots are pinned, hits are touched only on
        demand, and the per-token LFU tick happens on layer 0 decode calls."""
        if not self.native_caches:
            return super()._place_keys(layer, want, prefetch)
        if not want:
            return {}, [], {t: [] for t in self.tiers}
        tiers = {self.tier(layer, e) for e in want}
        if len(tiers) != 1:
            raise ValueError(f"layer {layer} spans multiple expert tiers: {tiers}")
        t = tiers.pop()
        cache = self.native_caches[t]
        if layer == 0 and not prefetch and len(want) <= self.top_k:
            for c in self.native_caches.values():
                c.note_token()
        if not prefetch and len(want) > self.slots[t] - 1:
            raise ValueError(f"layer {layer} needs {len(want)} {t} experts but the arena has "
                             f"{self.slots[t] - 1}; raise ceiling_gb")
        # Each key is planned with the previous demand call's slots pinned
        # plus every slot this call has resolved so far (locali_cache_plan_each,
        # one native call): a multi-key call could hand a slot claimed (or
        # hit) earlier in the same call to a later miss when the tier is
        # nearly full, leaving two experts on one slot. Whenever that cannot
        # happen the assignments equal one multi-key call's (same operations
        # in the same order).
        results = cache.plan_each([layer * self.E + e for e in want],
                                  pinned_slots=tuple(self.pinned.get(t, ())), touch_hits=not prefetch)
        out, issued = {}, []
        waits = {name: [] for name in self.tiers}
        for e, r in zip(want, results):
            key = (layer, e)
            if r.hit:
                self._hit(key, t, prefetch, waits)
            else:
                if not prefetch:
                    self.misses += 1
                if r.evicted_key >= 0:
                    self._evicted(self._decode_key(r.evicted_key))
                if r.placed:
                    issued.append((e, t, r.slot))
            if r.placed:
                out[e] = (t, r.slot)
            elif not prefetch:
                raise RuntimeError(f"native scheduler could not place demanded L{layer}.E{e}")
        if not prefetch:
            self.pinned = {t: {s for _, s in out.values()}}
        return out, issued, waits

    def _layer_tier(self, layer, want):
        """The one tier of a layer's experts (a V4 layer never spans two)."""
        cache = self.__dict__.setdefault("_tier_of_layer", {})
        tiers = cache.get(layer)
        if tiers is None:
            tiers = cache[layer] = {self.tier(layer, e) for e in range(self.E)}
        if len(tiers) != 1:
            tiers = {self.tier(layer, e) for e in want}
            if len(tiers) != 1:
                raise ValueError(f"layer {layer} spans multiple expert tiers: {tiers}")
        return next(iter(tiers))

    def submit(self, layer, experts, prefetch=False, fills_on_caller_stream=None):
        """ArenaStore.submit; with the compiled planner and fills from host
        memory, a layer's misses are queued straight after the one planner
        call and the bookkeeping follows. Planner calls, slots, counters,
        futures, pins and streams are the general path's."""
        if not self.native_caches or self.host_source is None or self.fill_stream is None:
            return super().submit(layer, experts, prefetch, fills_on_caller_stream)
        if fills_on_caller_stream is None:
            fills_on_caller_stream = not prefetch
        want = list(dict.fromkeys(int(e) for e in experts))
        if not want:
            return {}, ReadPlan({t: [] for t in self.tiers})
        t = self._layer_tier(layer, want)
        cache = self.native_caches[t]
        if layer == 0 and not prefetch and len(want) <= self.top_k:
            for c in self.native_caches.values():
                c.note_token()
        if not prefetch and len(want) > self.slots[t] - 1:
            raise ValueError(f"layer {layer} needs {len(want)} {t} experts but the arena has "
                             f"{self.slots[t] - 1}; raise ceiling_gb")
        base = layer * self.E
        res = cache.plan_each_into([base + e for e in want], tuple(self.pinned.get(t, ())),
                                   not prefetch)
        issued = [(e, r.slot) for e, r in zip(want, res) if r.placed and not r.hit]
        if not prefetch:
            self._mark_demand()
        landed = (self._fill_from_host([((layer, e), t, s, None) for e, s in issued],
                                       fills_on_caller_stream) if issued else None)
        out, waits = {}, {name: [] for name in self.tiers}
        for e, r in zip(want, res):
            if r.hit:
                self._hit((layer, e), t, prefetch, waits)
            else:
                if not prefetch:
                    self.misses += 1
                if r.evicted_key >= 0:
                    self._evicted(self._decode_key(r.evicted_key))
            if r.placed:
                out[e] = (t, r.slot)
            elif not prefetch:
                raise RuntimeError(f"native scheduler could not place demanded L{layer}.E{e}")
        if not prefetch:
            self.pinned = {t: {s for _, s in out.values()}}
        futs = []
        for e, _ in issued:
            self.bytes_read += self.item[t]
            self.inflight.setdefault((layer, e), []).append(landed)
            futs.append(landed)
        plan = ReadPlan({name: [] for name in self.tiers})
        plan[t] = futs + waits[t]
        plan.pending_experts = frozenset(
            e for e in want if any(not f.done() for f in self.inflight.get((layer, e), ())))
        if prefetch:
            self.prefetched += len(issued)
            self.pf_keys.update((layer, e) for e, _ in issued)
        return out, plan

    def _dplan_sources(self, t):
        """Device table of every key's pinned payload address (built once;
        the payloads are held for the store's life)."""
        if self._dplan_src is None:
            keep = [self._host_bytes((layer, e), t) for layer in range(self.layers) for e in range(self.E)]
            ptrs = DevicePlanner.host_view([src.data_ptr() for src in keep])
            self._dplan_keep = keep
            self._dplan_src = torch.tensor(ptrs, dtype=torch.int64, device=self.device)
        return self._dplan_src

    def device_plan(self, layer, expert_idx):
        """Route slots [T, k] of one demand call planned on the device; the
        call's misses are copied by the same launch, each starting as soon
        as the planner has placed it, on the current stream."""
        t = self.tiers[0]
        # The kernel cannot raise: a demanded key it could not place would
        # read the zero slot. Calls that might not place every key are
        # refused here, where the host planner would raise.
        keys = min(int(expert_idx.numel()), self.E)
        if not self.dplan.demand_fits(keys, self._dplan_pinned):
            raise RuntimeError(f"device planner: a call of {keys} experts with {self._dplan_pinned} slots of "
                               f"the previous call pinned may find no unpinned slot (probation holds "
                               f"{self.dplan.probation_capacity} keys); use a larger arena or the host planner")
        src = self._dplan_sources(t)
        self._after_prefetch()
        slots = self.dplan.plan_fill(expert_idx, layer, self.top_k, self._slot_table(t), src)
        self._dplan_pinned = keys
        return slots

    def _after_prefetch(self):
        """The current stream waits for the prefetch calls queued on the fill
        stream: the planner state is used by one call at a time, in the
        reference's order, and their copies have landed before a later
        demand call can use their slots."""
        if self._pf_event is not None:
            ops.current_stream(self.device).wait_event(self._pf_event)
            self._pf_event = None

    def device_lookahead(self, ahead, x, input_ids=None):
        """The lookahead routings of a cross-layer prefetch: [(layer,
        prefetch_k, indices, weights)] for each (module, prefetch_k) of
        `ahead`. When every module routes through its V4Gate they run on the
        fill stream beside this layer's router, each with the store's own
        router workspace (the gate's workspace belongs to its layer's demand
        call on the current stream); any other gate routes on the current
        stream, whose state only its own calls are known to keep in order."""
        plain = all(type(blk).route is V4ArenaMoE.route and isinstance(blk.gate, V4Gate) for blk, _ in ahead)
        if not plain:
            return [(blk.layer, k) + tuple(blk.route(x, input_ids)) for blk, k in ahead]
        fs, cur = self.fill_stream, ops.current_stream(self.device)
        fs.wait_stream(cur)          # x and the workspace's last use are behind
        for t in (x, input_ids):
            if isinstance(t, torch.Tensor) and t.is_cuda:
                t.record_stream(fs)
        ws = self.__dict__.get("_look_ws")
        if ws is None:
            ws = self._look_ws = ops.Workspace(self.device)
        with torch.cuda.stream(fs):
            return [(blk.layer, k) + tuple(blk.gate(x, input_ids, ws=ws)) for blk, k in ahead]

    def device_prefetch(self, looks):
        """Queue the prefetch calls of one layer call on the fill stream, after
        the demand call already queued on the current stream (the reference's
        order: demand, then the nearest layer first). Each plans and copies
        in one launch (locali_dplan_prefetch); the next demand call waits for
        them (_after_prefetch)."""
        t = self.tiers[0]
        fs, cur = self.fill_stream, ops.current_stream(self.device)
        fs.wait_stream(cur)
        src = self._dplan_sources(t)
        with torch.cuda.stream(fs):
            for layer, k, idx, w in looks:
                self.dplan.prefetch(idx.to(torch.int32), w.to(torch.float32), layer, self.top_k, k or 0,
                                    self._slot_table(t), src)
            ev = torch.cuda.Event()
            ev.record(fs)
        self._pf_event = ev

    def _dplan_counters(self):
        self._after_prefetch()
        c, _ = self.dplan.read()
        if c["error"]:
            what = {1: "a route's expert outside the layer", 2: "a demanded expert found no unpinned slot",
                    3: "plan arguments disagree with the planner state",
                    4: "a copy workgroup gave up waiting for the planner"}.get(c["error"], c["error"])
            raise RuntimeError(f"device planner: {what}")
        return c

    def reset_stats(self):
        super().reset_stats()
        if self.dplan is not None:
            self._dplan_base = self._dplan_counters()

    def stats(self):
        st = super().stats()
        st["scheduler"] = "c" if self.native_caches else "python"
        if self.dplan is not None:
            c = self._dplan_counters()
            base = self._dplan_base or {k: 0 for k in c}
            hits, misses = c["hits"] - base["hits"], c["misses"] - base["misses"]
            pf = c["prefetched"] - base["prefetched"]
            st.update(hits=hits, misses=misses, hit_rate=hits / (hits + misses) if hits + misses else 0.0,
                      evictions=c["evictions"] - base["evictions"],
                      bytes_read=(misses + pf) * self.item[self.tiers[0]], scheduler="device",
                      protected={self.tiers[0]: c["protected_"]}, prefetched=pf,
                      prefetch_used=c["prefetch_used"] - base["prefetch_used"],
                      prefetch_wasted=c["prefetch_wasted"] - base["prefetch_wasted"])
        return st

    def _protected_size(self, t):
        if t in self.native_caches:
            return self.native_caches[t].protected_size
        return super()._protected_size(t)

    def close(self):
        for c in self.native_caches.values():
            c.close()
        self.native_caches = {}
        super().close()


class V4Gate:
    """The V4 MoEGate on the router kernel: logits = x . W^T in fp32;
    sqrt(softplus) (or sigmoid / softmax) scores; top-k on score + the
    selection-only bias; weights = score / (sum + 1e-20) * routed_scaling;
    hash layers take idx = tid2eid[input_id] (reference dsv4_arena.py:147-153,
    165-166; restated formula tf:models/deepseek_v4/modeling_deepseek_v4.py:
    1024-1073). Returns (indices int32 [..., k], scores fp32 [..., k])."""

    def __init__(self, weight, top_k=6, e_score_correction_bias=None, tid2eid=None,
                 score_func="sqrtsoftplus", routed_scaling_factor=1.5, norm_topk_prob=True):
        bias = (None if e_score_correction_bias is None
                else e_score_correction_bias.to(device=weight.device, dtype=torch.float32).contiguous())
        t2e = None if tid2eid is None else tid2eid.to(device=weight.device, dtype=torch.int32).contiguous()
        self.spec = ops.RouterSpec(weight.contiguous(), top_k, score_func=score_func,
                                   norm_topk=norm_topk_prob, routed_scale=routed_scaling_factor,
                                   score_bias=bias, tid2eid=t2e)
        self.top_k = top_k
        self.ws = ops.Workspace(weight.device)

    @property
    def weight(self):
        return self.spec.weight

    def __call__(self, x, input_ids=None, ws=None):
        """ws: a router workspace to use instead of the gate's own (a caller
        routing on another stream than the gate's layer)."""
        lead = x.shape[:-1]
        if self.spec.tid2eid is not None and input_ids is None:
            raise ValueError("hash-routed gate needs input_ids")
        idx, w, _ = ops.router(self.spec, x.reshape(-1, x.shape[-1]), ws if ws is not None else self.ws,
                                  input_ids=input_ids)
        return idx.reshape(*lead, self.top_k), w.reshape(*lead, self.top_k)


class V4ArenaMoE(ArenaMoE):
    """V4 top-k routing and clamped SwiGLU over the arena's affine experts.
    Routing is the gate's (hash routing in the first layers, selection-only
    bias elsewhere); only the routed experts are replaced -- the shared
    expert is added by the model block (dsv4_engine.py:255-259:
    routed + shared_experts(x)).

    shared_expert (optional, an ops.ExpertArenaT whose slot 0 holds the
    block's shared expert, same quantisation as the routed tier) folds that
    addition into the same launches: the call then returns
    routed + shared_expert(x), each rounded to x's dtype before the sum."""

    def __init__(self, store: V4ArenaStore, layer: int, gate, top_k: int,
                 swiglu_limit: float = 10.0, fused_decode: bool = False,
                 overlap_hits: bool = False, fp32_swiglu: bool = False, shared_expert=None):
        super().__init__(store, layer, gate, bias=None, top_k=top_k)
        self.shared_expert = shared_expert
        self.swiglu_limit = swiglu_limit
        self.scores_follow_output = True
        # The decode path always fuses gate/up + SwiGLU; the flag is accepted
        # for interface parity.
        self.fused_decode = fused_decode
        # Results do not depend on it: hit and miss routes are computed by the
        # same kernels once every fill has landed.
        self.overlap_hits = overlap_hits
        self.fp32_swiglu = fp32_swiglu

    def route(self, x, input_ids=None):
        return self.gate(x, input_ids)

    def __call__(self, x, input_ids=None):
        """With the store's device planner the call queues router, planner,
        fills and experts on the current stream and returns without waiting
        for the device; otherwise ArenaMoE's host-planned call."""
        if self.store.dplan is None:
            return super().__call__(x, input_ids)
        shape = x.shape
        flat = x.reshape(-1, shape[-1])
        if flat.shape[0] == 0:
            return torch.zeros(shape, dtype=x.dtype, device=x.device)
        # Cross-layer prefetch (reference arena.py:518-541): the lookahead
        # gates run on the fill stream beside this layer's router, and their
        # planner calls follow this layer's demand call there, so that their
        # copies overlap this layer's experts.
        ahead = [(blk, k) for blk, k in ((self.nxt, self.prefetch_k), (self.nxt2, self.prefetch_k2))
                 if blk is not None]
        looks = self.store.device_lookahead(ahead, x, input_ids) if ahead else None
        inds, gates = self.route(x, input_ids)
        T = flat.shape[0]
        slots = self.store.device_plan(self.layer, inds.reshape(T, self.top_k))
        if looks:
            self.store.device_prefetch(looks)
        out = self._run_experts(self.store.tiers[0], flat, slots, gates.reshape(T, self.top_k), x.dtype)
        return out.reshape(shape).to(x.dtype)


__all__ = ["V4ArenaStore", "V4ArenaMoE", "V4Gate", "PROJS"]
