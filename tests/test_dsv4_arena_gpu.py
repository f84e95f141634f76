"""V4ArenaMoE / V4ArenaStore on the GPU, read like the reference's
tests/test_dsv4_arena.py: experts streamed from a checkpoint on disk into the
HBM arena must give exactly what the expert kernels give on the same weights
held resident (bit-exact: same kernels, same arithmetic), for prefill-sized
and decode-sized calls, through evictions in a bounded arena, and with fp16
expert metadata; and within tolerance of the C oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from checkpoint_fixture import expert_bytes, make_index, make_snapshot
from gpu_helpers import arena_numpy, assert_close_terms, banner
from locali_amd import ops, synth
from locali_amd.dsv4_arena import V4ArenaMoE, V4ArenaStore, V4Gate

pytestmark = pytest.mark.gpu

D, DFF, E, K, LAYERS = 512, 512, 6, 2, 2


class FixedGate:
    def __init__(self, indices, scores):
        self.indices, self.scores = indices, scores

    def __call__(self, x, input_ids=None):
        return self.indices, self.scores


def _gpu(arena):
    return ops.ExpertArenaT(*(ops.ProjArena(p.weight.cuda(), p.scales.cuda(), p.biases.cuda(),
                                            p.bits, p.group_size)
                              for p in (arena.gate, arena.up, arena.down)))


def _direct(truth_gpu, x, idx, scores):
    """The same routes through the expert kernels on the resident weights
    (slot e = expert e)."""
    T = x.shape[0]
    w = scores.float().contiguous()
    if T <= 2:
        return ops.expert_decode(truth_gpu, None, x, idx.int().contiguous(), w)
    soe = torch.arange(E, dtype=torch.int32, device="cuda")
    return ops.expert_grouped(truth_gpu, None, x, idx.int().contiguous(), soe, w, ops.Workspace(),
                              n_experts=E)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    root = tmp_path_factory.mktemp("v4")
    truth = make_snapshot(root, layers=LAYERS, experts=E, top_k=K, d=D, dff=DFF)
    return truth, make_index(root), make_index(root, packed=True)


def _item(index):
    import json
    m = next(iter(json.loads(open(index).read())["experts"].values()))
    return sum(m[p][a][3] for p in ("gate_proj", "up_proj", "down_proj")
               for a in ("weight", "scales", "biases"))


@pytest.mark.parametrize("packed", [False, True])
def test_streamed_v4_experts_match_resident_kernels(ckpt, packed):
    truth, index, pindex = ckpt
    idx_path = pindex if packed else index
    banner(f"v4 arena streamed vs resident packed={packed}")
    store = V4ArenaStore(idx_path, ceiling_gb=(E + 1) * _item(idx_path) / 1e9 + 1e-6, threads=2,
                         nocache=False, cache_policy="lru")
    try:
        g = torch.Generator().manual_seed(7)
        x = (torch.randn(3, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
        indices = torch.tensor([[0, 2], [0, 2], [2, 0]], dtype=torch.int32, device="cuda")
        scores = torch.tensor([[0.7, 0.3], [0.4, 0.6], [0.2, 0.8]], dtype=torch.float32, device="cuda")
        moe = V4ArenaMoE(store, 0, FixedGate(indices, scores), K, swiglu_limit=10.0)
        streamed = moe(x)
        expected = _direct(_gpu(truth[0]), x, indices, scores)
        assert streamed.dtype == x.dtype and streamed.shape == x.shape
        assert torch.equal(streamed, expected)

        # Decode-sized mixed hit/miss: expert 0 is resident, expert 3 is new.
        store.tier_overlap = True
        dx = x[:1]
        di = torch.tensor([[0, 3]], dtype=torch.int32, device="cuda")
        dsc = torch.tensor([[0.65, 0.35]], dtype=torch.float32, device="cuda")
        moe.gate = FixedGate(di, dsc)
        assert torch.equal(moe(dx), _direct(_gpu(truth[0]), dx, di, dsc))
        st = store.stats()
        assert (st["hits"], st["misses"]) == (1, 3)
    finally:
        store.close()


def test_bounded_arena_evicts_and_stays_exact(ckpt):
    truth, index, _ = ckpt
    banner("v4 arena bounded: 4 usable slots, 2 layers, 10 decode steps")
    store = V4ArenaStore(index, ceiling_gb=5 * _item(index) / 1e9 + 1e-6, threads=2,
                         cache_policy="lru")
    rng = np.random.default_rng(3)
    try:
        assert store.slots["cold"] == 5
        resident = [_gpu(t) for t in truth]
        gates = [FixedGate(None, None) for _ in range(LAYERS)]
        mods = [V4ArenaMoE(store, L, gates[L], K) for L in range(LAYERS)]
        distinct = 0
        for step in range(10):
            x = torch.from_numpy(rng.standard_normal((1, D)).astype(np.float32)).to(torch.bfloat16).cuda()
            for L in range(LAYERS):
                ids = rng.choice(E, size=K, replace=False)
                w = rng.random(K).astype(np.float32)
                gates[L].indices = torch.tensor(ids[None], dtype=torch.int32, device="cuda")
                gates[L].scores = torch.tensor((w / w.sum())[None], device="cuda")
                got = mods[L](x)
                assert torch.equal(got, _direct(resident[L], x, gates[L].indices, gates[L].scores)), \
                    f"step {step} layer {L}"
                distinct += K
                x = got
        st = store.stats()
        assert st["hits"] + st["misses"] == distinct and st["evictions"] > 0
        assert st["bytes_read"] == st["misses"] * store.item["cold"]
    finally:
        store.close()


def test_f16_metadata_casts_bf16_activations(tmp_path):
    banner("v4 arena fp16 metadata")
    truth = make_snapshot(tmp_path, layers=1, experts=E, top_k=K, d=D, dff=DFF,
                          meta_dtype=torch.float16, seed=5)
    index = make_index(tmp_path)
    store = V4ArenaStore(index, ceiling_gb=(E + 1) * _item(index) / 1e9 + 1e-6, threads=2)
    try:
        assert store.use_f16_moe == {"cold": True}
        x = (torch.randn(4, D, generator=torch.Generator().manual_seed(1)) * 0.5).to(torch.bfloat16).cuda()
        ind = torch.tensor([[1, 4], [4, 5], [0, 1], [5, 2]], dtype=torch.int32, device="cuda")
        sc = torch.full((4, K), 0.5, device="cuda")
        got = V4ArenaMoE(store, 0, FixedGate(ind, sc), K)(x)
        want = _direct(_gpu(truth[0]), x.to(torch.float16), ind, sc).to(torch.bfloat16)
        assert got.dtype == torch.bfloat16 and torch.equal(got, want)
    finally:
        store.close()


def test_v4_gate_protocol_and_oracle_parity(ckpt, oracle_lib):
    truth, index, _ = ckpt
    banner("v4 gate + arena vs C oracle")
    from oracle import cref
    wg, bias = synth.uniform_router(E, D, torch.bfloat16, seed=11, device="cuda", bias_std=0.01)
    gate = V4Gate(wg, top_k=K, e_score_correction_bias=bias, routed_scaling_factor=1.5)
    x = synth.activations(5, D, torch.bfloat16, seed=12, device="cuda")
    inds, scores = gate(x.reshape(5, 1, D))
    assert inds.shape == (5, 1, K) and scores.dtype == torch.float32
    ref_idx, ref_w, _ = ops.router(gate.spec, x, ops.Workspace())
    assert torch.equal(inds.reshape(5, K), ref_idx) and torch.equal(scores.reshape(5, K), ref_w)
    store = V4ArenaStore(index, ceiling_gb=(E + 1) * _item(index) / 1e9 + 1e-6, threads=2)
    try:
        got = V4ArenaMoE(store, 1, gate, K)(x.reshape(5, 1, D)).reshape(5, D)
        slots = inds.reshape(5, K).cpu().numpy().astype(np.int32)
        want, terms = cref.load().moe_layer(x.float().cpu().numpy(), slots,
                                            scores.reshape(5, K).cpu().numpy(),
                                            arena_numpy(truth[1], float_meta=False), "bf16",
                                            return_terms=True)
        assert_close_terms(got.float().cpu().numpy(), want, terms, "v4 arena vs oracle")
    finally:
        store.close()


def _host_source(truth):
    """Pinned host copies of every expert, nine records back to back."""
    cache = {}

    def src(layer, expert):
        if (layer, expert) not in cache:
            raw = np.frombuffer(expert_bytes(truth, layer, expert), dtype=np.uint8)
            cache[(layer, expert)] = torch.from_numpy(raw.copy()).pin_memory()
        return cache[(layer, expert)]
    return src


@pytest.mark.parametrize("policy", ["lru", "lfu-decay"])
def test_host_source_fills_evict_and_stay_exact(ckpt, policy):
    """Misses copied from pinned host memory on the fill stream (no file
    reads) through evictions in a 6-slot arena: every call equals the
    resident kernels bit for bit, and prefill-sized calls too."""
    truth, index, _ = ckpt
    banner(f"v4 arena host source: 6 usable slots, policy {policy}")
    store = V4ArenaStore(index, ceiling_gb=7 * _item(index) / 1e9 + 1e-6, threads=2,
                         cache_policy=policy, host_source=_host_source(truth))
    rng = np.random.default_rng(5)
    try:
        resident = [_gpu(t) for t in truth]
        gates = [FixedGate(None, None) for _ in range(LAYERS)]
        mods = [V4ArenaMoE(store, L, gates[L], K) for L in range(LAYERS)]
        for step in range(8):
            T = 1 if step % 3 else 3
            x = torch.from_numpy(rng.standard_normal((T, D)).astype(np.float32)).to(torch.bfloat16).cuda()
            for L in range(LAYERS):
                # 3 experts per call: this call's and the previous call's (pinned) fit 6 slots
                pool = rng.choice(E, size=3, replace=False)
                ids = np.stack([rng.choice(pool, size=K, replace=False) for _ in range(T)])
                w = rng.random((T, K)).astype(np.float32)
                gates[L].indices = torch.tensor(ids, dtype=torch.int32, device="cuda")
                gates[L].scores = torch.tensor(w / w.sum(1, keepdims=True), device="cuda")
                got = mods[L](x)
                assert torch.equal(got, _direct(resident[L], x, gates[L].indices, gates[L].scores)), \
                    f"step {step} layer {L}"
                x = got
        st = store.stats()
        assert st["evictions"] > 0 and st["misses"] > 0
        assert st["bytes_read"] == st["misses"] * store.item["cold"]
    finally:
        store.close()


@pytest.mark.parametrize("T", [1, 3])
def test_shared_expert_folds_into_the_call(ckpt, oracle_lib, T):
    """V4ArenaMoE(shared_expert=...) returns routed + shared_experts(x) as
    the engine block forms it (dsv4_engine.py:259): bit-exact against the
    expert kernels called with the same shared expert on resident weights,
    within tolerance of the oracle's routed-then-shared rounding, and for a
    decode call exactly the routed call's output plus the shared expert
    alone, summed in bf16."""
    from oracle import cref
    truth, index, _ = ckpt
    banner(f"v4 arena shared expert folded T={T}")
    shared_cpu = synth.expert_arena(1, D, DFF, bits_gate_up=2, group=64, dtype=torch.bfloat16,
                                    seed=41, zero_slot=False)
    shared = _gpu(shared_cpu)
    store = V4ArenaStore(index, ceiling_gb=(E + 1) * _item(index) / 1e9 + 1e-6, threads=2)
    try:
        g = torch.Generator().manual_seed(9)
        x = (torch.randn(T, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
        ind = torch.tensor([[1, 4], [4, 5], [0, 1]][:T], dtype=torch.int32, device="cuda")
        sc = torch.tensor([[0.6, 0.4], [0.3, 0.7], [0.5, 0.5]][:T], device="cuda")
        folded = V4ArenaMoE(store, 0, FixedGate(ind, sc), K, shared_expert=shared)(x)
        resident = _gpu(truth[0])
        if T <= 2:
            direct = ops.expert_decode(resident, shared, x, ind, sc)
            routed = V4ArenaMoE(store, 0, FixedGate(ind, sc), K)(x)
            alone = ops.expert_decode(shared, None, x, torch.zeros(T, 1, dtype=torch.int32, device="cuda"),
                                      torch.ones(T, 1, device="cuda"))
            assert torch.equal(folded, routed + alone)
        else:
            soe = torch.arange(E, dtype=torch.int32, device="cuda")
            direct = ops.expert_grouped(resident, shared, x, ind, soe, sc, ops.Workspace(), n_experts=E)
        assert torch.equal(folded, direct)
        want, terms = cref.load().moe_layer(x.float().cpu().numpy(), ind.cpu().numpy(),
                                            sc.cpu().numpy(), arena_numpy(truth[0], float_meta=False),
                                            "bf16", shared=arena_numpy(shared_cpu, float_meta=False),
                                            return_terms=True)
        assert_close_terms(folded.float().cpu().numpy(), want, terms, "folded shared vs oracle")
    finally:
        store.close()


class _TwoTiers:
    """The store surface ArenaMoE._apply reads, over two resident tiers."""
    tiers = ["cold", "hot"]

    def __init__(self, arenas):
        self.arenas, self.device, self.workspace = arenas, torch.device("cuda"), None

    def expert_arena(self, t):
        return self.arenas[t]

    def use_f16(self, t):
        return False

    def wait(self, reads):
        pass

    def slot_identity(self, t):
        return torch.arange(self.arenas[t].n_slots, dtype=torch.int32, device="cuda")


@pytest.mark.parametrize("T", [1, 2, 7])
def test_routes_spanning_two_tiers(T):
    """A call whose routes land in two tiers with different quantisation
    (2-bit cold, 4-bit hot) takes the reference's mixed path (arena.py:626-672):
    each tier's own entries through its experts, float32 products of y and the
    dtype-rounded scores summed tier by tier, one rounding. Within the term
    rounding bound of the oracle's restatement of that order; and a call with
    every route in one tier still takes the single-tier path unchanged."""
    from locali_amd.arena import ArenaMoE
    from oracle import moe as moe_oracle
    banner(f"two tiers T={T}")
    d, dff, k = 1024, 512, 4
    cold = synth.expert_arena(9, d, dff, bits_gate_up=2, dtype=torch.bfloat16, seed=51, device="cuda")
    hot = synth.expert_arena(5, d, dff, bits_gate_up=4, dtype=torch.bfloat16, seed=52, device="cuda")
    store = _TwoTiers({"cold": cold, "hot": hot})
    moe = ArenaMoE(store, 0, None, None, k)
    moe.swiglu_limit = 10.0
    # experts 0..7 in cold slots 1..8, experts 8..11 in hot slots 1..4
    placed = {e: ("cold", e + 1) for e in range(8)}
    placed.update({e: ("hot", e - 7) for e in range(8, 12)})
    g = torch.Generator().manual_seed(60 + T)
    ii = [torch.randperm(12, generator=g)[:k].tolist() for _ in range(T)]
    ii[0] = [9, 2, 11, 5]                  # both tiers, interleaved
    gates = torch.rand(T, k, generator=g)
    x = synth.activations(T, d, torch.bfloat16, seed=53, device="cuda")
    out = moe._apply(x, ii, placed, gates.cuda(), torch.bfloat16)
    torch.cuda.synchronize()
    tier_of = [[placed[e][0] for e in row] for row in ii]
    slot = np.array([[placed[e][1] for e in row] for row in ii])
    want, terms = moe_oracle.mixed_tiers(
        x.float().cpu().numpy(), tier_of, slot, gates.numpy(),
        {"cold": arena_numpy(cold), "hot": arena_numpy(hot)}, ["cold", "hot"], "bf16", limit=10.0)
    assert_close_terms(out.float().cpu().numpy(), want, terms, f"two tiers T={T}")
    # one tier only: the single-tier path (rounded products) is what runs
    one = [[e % 8 for e in row] for row in ii]
    got1 = moe._apply(x, one, placed, gates.cuda(), torch.bfloat16)
    slots1 = torch.tensor([[placed[e][1] for e in row] for row in one], dtype=torch.int32, device="cuda")
    w = gates.cuda().float()
    if T <= 2:
        ref1 = ops.expert_decode(cold, None, x, slots1, w, swiglu_limit=10.0)
    else:
        ref1 = ops.expert_grouped(cold, None, x, slots1, torch.arange(9, dtype=torch.int32, device="cuda"),
                                  w, ops.Workspace(), n_experts=9, swiglu_limit=10.0)
    assert torch.equal(got1, ref1)


def test_streamed_3bit_experts_match_resident_kernels(tmp_path):
    """A checkpoint of 3-bit experts (the DSpark/MTP tier's width, whose
    codes cross word boundaries) streams from disk through the store and
    gives exactly what the expert kernels give on the same weights held
    resident, for a prefill-sized and a decode-sized call."""
    banner("v4 arena streamed 3-bit")
    truth = make_snapshot(tmp_path, layers=1, experts=E, top_k=K, d=D, dff=DFF, bits=3, seed=5)
    index = make_index(tmp_path)
    store = V4ArenaStore(index, ceiling_gb=(E + 1) * _item(index) / 1e9 + 1e-6, threads=2,
                         nocache=False, cache_policy="lru")
    try:
        assert store.quant("cold", "bits") == 3
        assert store.expert_arena("cold").gate.bits == 3
        g = torch.Generator().manual_seed(8)
        x = (torch.randn(3, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
        indices = torch.tensor([[1, 4], [4, 5], [5, 1]], dtype=torch.int32, device="cuda")
        scores = torch.tensor([[0.6, 0.4], [0.3, 0.7], [0.5, 0.5]], dtype=torch.float32, device="cuda")
        moe = V4ArenaMoE(store, 0, FixedGate(indices, scores), K, swiglu_limit=10.0)
        assert torch.equal(moe(x), _direct(_gpu(truth[0]), x, indices, scores))
        dx, di = x[:1], torch.tensor([[5, 2]], dtype=torch.int32, device="cuda")
        moe.gate = FixedGate(di, scores[:1])
        assert torch.equal(moe(dx), _direct(_gpu(truth[0]), dx, di, scores[:1]))
    finally:
        store.close()


@pytest.mark.parametrize("with_shared", [False, True])
def test_overlap_hits_splits_a_decode_call_and_stays_exact(ckpt, with_shared):
    """overlap_hits with one token and some of its experts still filling
    (reference arena.py:575-618): the resident routes run before the host
    waits, the pending ones after, and the split call gives bit-for-bit what
    the unsplit call gives (with and without a folded shared expert). The
    split is forced with a read plan that names expert 4 as pending; a real
    streamed call with overlap_hits on must agree as well."""
    from locali_amd.arena import ReadPlan
    truth, index, _ = ckpt
    banner(f"overlap_hits shared={with_shared}")
    store = V4ArenaStore(index, ceiling_gb=(E + 1) * _item(index) / 1e9 + 1e-6, threads=2,
                         cache_policy="lru")
    try:
        sh = (synth.expert_arena(1, D, DFF, dtype=torch.bfloat16, seed=91, device="cuda", zero_slot=False)
              if with_shared else None)
        g = torch.Generator().manual_seed(12)
        x = (torch.randn(1, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
        di = torch.tensor([[1, 4]], dtype=torch.int32, device="cuda")
        sc = torch.tensor([[0.55, 0.45]], dtype=torch.float32, device="cuda")
        want = V4ArenaMoE(store, 0, FixedGate(di, sc), K, swiglu_limit=10.0, shared_expert=sh)(x)
        mo = V4ArenaMoE(store, 0, FixedGate(di, sc), K, swiglu_limit=10.0, overlap_hits=True,
                        shared_expert=sh)
        placed = store.slots_for(0, [1, 4])
        reads = ReadPlan({t: [] for t in store.tiers}, pending_experts={4})
        got = mo._apply(x, [[1, 4]], placed, sc, x.dtype, reads)
        assert torch.equal(got, want)
        store.tier_overlap = True
        di2 = torch.tensor([[4, 5]], dtype=torch.int32, device="cuda")   # 5 is new: a real miss
        mo.gate = FixedGate(di2, sc)
        ref = V4ArenaMoE(store, 0, FixedGate(di2, sc), K, swiglu_limit=10.0, shared_expert=sh)
        assert torch.equal(mo(x), ref(x))
    finally:
        store.close()


@pytest.mark.parametrize("T", [1, 5])
def test_gather_hook_follows_the_reference_contract(ckpt, oracle_lib, T):
    """_gather(tier, inputs [n, 1, 1, d], indices [n, k]) -> [n, k, 1, d]
    unweighted per-route expert outputs (reference arena.py:674-681,
    dsv4_arena.py:168-235): each entry within the expert-output tolerance of
    the oracle's expert on that route. A subclass that overrides _gather (the
    reference's _apply -> _gather contract) is called through it by
    __call__, and since each route's output and the combine's arithmetic are
    the fused kernels', its layer output equals the module's own, with and
    without a folded shared expert."""
    from gpu_helpers import assert_close
    from oracle import cref
    truth, index, _ = ckpt
    banner(f"v4 arena _gather hook T={T}")
    store = V4ArenaStore(index, ceiling_gb=(E + 1) * _item(index) / 1e9 + 1e-6, threads=2)
    calls = []

    class Hooked(V4ArenaMoE):
        def _gather(self, tier, inputs, indices):
            calls.append((tier, tuple(inputs.shape), tuple(indices.shape)))
            return super()._gather(tier, inputs, indices)

    try:
        g = torch.Generator().manual_seed(70 + T)
        x = (torch.randn(T, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
        ind = torch.tensor([[1, 4], [4, 5], [0, 1], [2, 3], [5, 0]][:T], dtype=torch.int32, device="cuda")
        sc = torch.tensor([[0.6, 0.4], [0.3, 0.7], [0.5, 0.5], [0.9, 0.1], [0.2, 0.8]][:T], device="cuda")
        shared = _gpu(synth.expert_arena(1, D, DFF, bits_gate_up=2, group=64, dtype=torch.bfloat16,
                                         seed=43, zero_slot=False))
        for sh in (None, shared):
            own = V4ArenaMoE(store, 0, FixedGate(ind, sc), K, swiglu_limit=10.0, shared_expert=sh)(x)
            calls.clear()
            hooked = Hooked(store, 0, FixedGate(ind, sc), K, swiglu_limit=10.0, shared_expert=sh)
            got = hooked(x)
            assert calls == [("cold", (T, 1, 1, D), (T, K))]
            assert torch.equal(got, own), f"hooked layer output differs (shared={sh is not None})"
        placed = store.slots_for(0, sorted(set(ind.reshape(-1).tolist())))
        slots = torch.tensor([[placed[e][1] for e in row] for row in ind.tolist()], dtype=torch.int32,
                             device="cuda")
        y = V4ArenaMoE(store, 0, FixedGate(ind, sc), K, swiglu_limit=10.0)._gather(
            "cold", x[:, None, None, :], slots)
        assert y.shape == (T, K, 1, D) and y.dtype == torch.bfloat16
        want = cref.load().moe_layer(x.float().cpu().numpy().repeat(K, axis=0),
                                     ind.reshape(-1, 1).cpu().numpy(), np.ones((T * K, 1), np.float32),
                                     arena_numpy(truth[0], float_meta=False), "bf16", limit=10.0)
        assert_close(y.reshape(T * K, D).float().cpu().numpy(), want, "_gather vs oracle experts")
    finally:
        store.close()


def test_two_tier_store_streams_cold_and_hot_layers(tmp_path):
    """An index extended with the DSpark/MTP stage (reference
    dsv4_index.py:146-249): main layers in the 2-bit cold tier, the stage as
    logical layer 2 in a 3-bit hot tier, both sharing one ceiling split by
    hot_share. Each layer streams from disk through its own tier and gives
    exactly what the kernels give on the same weights held resident."""
    import json
    from checkpoint_fixture import add_mtp_stage
    from locali_amd.index import build_index, extend_with_mtp
    banner("two-tier store: cold 2-bit + hot 3-bit")
    truth = make_snapshot(tmp_path, layers=2, experts=E, top_k=K, d=D, dff=DFF, seed=9)
    hot_truth = add_mtp_stage(tmp_path, experts=E, d=D, dff=DFF, bits=3, seed=10)
    index = extend_with_mtp(build_index(tmp_path), tmp_path)
    path = tmp_path / "two_tier.idx"
    path.write_text(json.dumps(index))
    cold_item = _item(path)
    hot_item = sum(index["experts"]["L2.E0"][p][a][3] for p in ("gate_proj", "up_proj", "down_proj")
                   for a in ("weight", "scales", "biases"))
    ceiling = 2 * (E + 1) * max(cold_item, hot_item)
    store = V4ArenaStore(path, ceiling_gb=ceiling / 1e9, hot_share=0.5, threads=2, cache_policy="lru")
    try:
        assert store.tiers == ["cold", "hot"]
        assert store.quant("hot", "bits") == 3 and store.expert_arena("hot").gate.bits == 3
        assert store.expert_arena("cold").gate.bits == 2
        g = torch.Generator().manual_seed(13)
        x = (torch.randn(3, D, generator=g) * 0.5).to(torch.bfloat16).cuda()
        ind = torch.tensor([[1, 4], [4, 0], [5, 1]], dtype=torch.int32, device="cuda")
        sc = torch.tensor([[0.6, 0.4], [0.3, 0.7], [0.5, 0.5]], dtype=torch.float32, device="cuda")
        for layer, t in ((0, truth[0]), (2, hot_truth), (1, truth[1])):
            moe_ = V4ArenaMoE(store, layer, FixedGate(ind, sc), K, swiglu_limit=10.0)
            assert torch.equal(moe_(x), _direct(_gpu(t), x, ind, sc)), f"layer {layer}"
            moe_.gate = FixedGate(ind[:1], sc[:1])
            assert torch.equal(moe_(x[:1]), _direct(_gpu(t), x[:1], ind[:1], sc[:1])), f"layer {layer} decode"
    finally:
        store.close()
