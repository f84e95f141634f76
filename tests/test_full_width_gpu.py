"""GPU parity at the benchmarked shapes: d_model 4096, 256 routed experts top-6
+ 1 shared expert, d_ff 2048, group 64, bf16 scales/biases.

  * 64- and 512-token prefill with Zipf(1.1) expert popularity (the grouped
    path: matrix-core 64-position tiles and one- to four-position small tiles at
    K 4096 / 2048, the whole-K metadata staging and the tile list at these
    counts), 2-bit gate/up/down;
  * 32-token batched decode with 2-bit gate/up and 4-bit down projections;
  * a stack of full-width layers decoding through one bounded arena whose
    misses are copied from pinned host memory, with and without the
    reference's cross-layer prefetch (arena.py:520-541).

Each layer call is checked against the C oracle on the GPU's own routing
(router indices against the numpy oracle wherever the selection margin
allows): the experts a call uses are copied to the host and renumbered, so
the oracle sees only those slots. For 512 tokens the checked tokens are the
first and last position of every tile of the heaviest experts and of the
shared expert, plus tokens of one- and two-position tiles: every tile kind
and tile boundary the kernels see."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from gpu_helpers import arena_numpy, assert_close_terms, banner, dt_name, exact_fraction, ulp_distance, values
from locali_amd import ops, synth
from oracle import moe

pytestmark = pytest.mark.gpu
DEV = "cuda"
D, E, DFF, K, GROUP = 4096, 256, 2048, 6, 64
TILE = 64            # positions per matrix-core tile (a tile of 1-4 takes the small-tile kernels)


def _layer(seed, bits_down=2, dtype=torch.bfloat16, group=GROUP):
    arena = synth.expert_arena(E + 1, D, DFF, bits_gate_up=2, bits_down=bits_down, group=group,
                               dtype=dtype, seed=seed, device=DEV)
    shared = synth.expert_arena(1, D, DFF, bits_gate_up=2, bits_down=bits_down, group=group,
                                dtype=dtype, seed=seed + 1, device=DEV, zero_slot=False)
    return arena, shared


def _check_routes(x, w, idx, wts, *, bias=None):
    """Router indices and weights against the numpy oracle where the margin
    exceeds fp32 accumulation noise; returns the number of tokens checked."""
    oi, ow, margin, scores = moe.route(values(x), values(w), K, routed_scale=1.5,
                                       bias=None if bias is None else values(bias))
    scale = np.abs(scores).max(axis=1)
    idx, wts = idx.cpu().numpy(), wts.cpu().numpy()
    checked = 0
    for t in range(idx.shape[0]):
        if margin[t] < 1e-4 * scale[t]:
            continue
        checked += 1
        assert list(idx[t]) == list(oi[t]), f"token {t}"
        np.testing.assert_allclose(wts[t], ow[t], rtol=1e-5, atol=1e-7)
    assert checked >= 0.9 * idx.shape[0]
    return checked


def _oracle_check(oracle_lib, arena, shared, x, slots, wts, out, tokens, what, chunk=16, exact=0.8,
                  dtype=torch.bfloat16):
    """The C oracle on `tokens` of a call, a chunk of tokens at a time (only
    the slots a chunk uses are copied to the host). `exact`: the least
    fraction of outputs equal to the oracle's at bf16 resolution -- equal for
    bf16, within one fp16 spacing for fp16 (None: no such bar; a single
    decode token's 4096 outputs are too few for a stable fraction)."""
    sh = {kk: v for kk, v in arena_numpy(shared, float_meta=False).items()}
    xs, got = values(x), values(out)
    same = []
    for c in range(0, len(tokens), chunk):
        tk = np.asarray(tokens[c:c + chunk])
        used = sorted(set(slots[tk].reshape(-1).tolist()))
        remap = {s: i for i, s in enumerate(used)}
        sub = arena_numpy(arena, float_meta=False, slots=used)
        want, terms = oracle_lib.moe_layer(xs[tk], np.vectorize(remap.get)(slots[tk]).astype(np.int32),
                                           wts[tk], sub, dt_name(dtype), shared=sh, return_terms=True)
        assert_close_terms(got[tk], want, terms, f"{what} tokens {tk[:4].tolist()}...")
        same.append(got[tk] == want if dtype == torch.bfloat16 else ulp_distance(got[tk], want, dtype) <= 1)
    if exact is not None:
        assert exact_fraction(np.concatenate(same), True) > exact


def _tile_sample(idx, T, heavy=6, mid=8, small=8, quad=4, seed=0):
    """Tokens covering every tile kind: the first and last position of every
    64-position tile of the `heavy` most-routed experts and of the shared
    expert (a segment of all T tokens), first/last of `mid` experts with
    5..64 positions, `small` tokens of one- or two-position tiles, and every
    token of `quad` three- or four-position tiles (the small-tile kernels'
    two-pass tiles)."""
    rng = np.random.default_rng(seed)
    seg: dict = {}
    for t in range(T):
        for e in idx[t]:
            seg.setdefault(int(e), []).append(t)
    pick = set()

    def ends(members):
        for a in range(0, len(members), TILE):
            tile = members[a:a + TILE]
            pick.update((tile[0], tile[-1]))

    ends(list(range(T)))                                        # the shared expert's tiles
    by_count = sorted(seg, key=lambda e: -len(seg[e]))
    for e in by_count[:heavy]:
        ends(seg[e])
    mids = [e for e in by_count if 5 <= len(seg[e]) <= TILE]
    for e in rng.permutation(mids)[:mid]:
        ends(seg[int(e)])
    tails = [e for e in seg if len(seg[e]) % TILE in (1, 2)]
    for e in rng.permutation(tails)[:small]:
        pick.add(seg[int(e)][-1])
    quads = [e for e in seg if len(seg[e]) % TILE in (3, 4)]
    for e in rng.permutation(quads)[:quad]:
        members = seg[int(e)]
        pick.update(members[len(members) - len(members) % TILE:])
    return sorted(pick), seg


@pytest.mark.parametrize("T,dtype,group", [(64, torch.bfloat16, 64), (512, torch.bfloat16, 64),
                                           (64, torch.float16, 64), (64, torch.bfloat16, 128),
                                           (512, torch.bfloat16, 128)])
def test_prefill_full_width_zipf(oracle_lib, T, dtype, group):
    banner(f"full-width prefill T={T} zipf 1.1 {dtype} group {group}")
    arena, shared = _layer(seed=300 + T, dtype=dtype, group=group)
    x, w = synth.zipf_router_inputs(T, E, D, 1.1, dtype, seed=310 + T, device=DEV)
    spec = ops.RouterSpec(w, K, routed_scale=1.5)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    out, idx, wts = ops.forward(spec, arena, shared, slot_of, x, ops.Workspace())
    torch.cuda.synchronize()
    _check_routes(x, w, idx, wts)
    ih = idx.cpu().numpy()
    if T <= 64:
        tokens = list(range(T))
    else:
        tokens, seg = _tile_sample(ih, T, seed=T)
        counts = sorted((len(v) for v in seg.values()), reverse=True)
        assert counts[0] > 2 * TILE and any(c % TILE in (1, 2) for c in counts)
        assert any(c % TILE in (3, 4) for c in counts)   # the four-position small down tiles
    _oracle_check(oracle_lib, arena, shared, x, (ih + 1).astype(np.int32), wts.cpu().numpy(), out,
                  tokens, f"C3 T={T} {dtype}", dtype=dtype)


def test_prefill_two_streams_eager_and_graph_replays():
    """Calls of 256 tokens or more run the small-tile kernels on a second
    stream beside the 64-position ones (fork after the preparation, join
    before the down pair and before the combine). Back-to-back eager calls
    on different inputs (the fork's events are reused) give each call's own
    result bit for bit, and a captured call replays bit-exact three times
    with eager calls in between. Parity of the same path with the C oracle
    is the 512-token case above."""
    T = 512
    banner(f"two-stream grouped path T={T}: eager pairs and graph replays")
    arena, shared = _layer(seed=901)
    xa, w = synth.zipf_router_inputs(T, E, D, 1.1, torch.bfloat16, seed=902, device=DEV)
    xb, _ = synth.zipf_router_inputs(T, E, D, 1.1, torch.bfloat16, seed=903, device=DEV)
    xb = xb.flip(0).contiguous()   # other tokens, same router
    spec = ops.RouterSpec(w, K, routed_scale=1.5)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    ws = ops.Workspace()
    ref_a = [t.clone() for t in ops.forward(spec, arena, shared, slot_of, xa, ws)]
    torch.cuda.synchronize()
    ref_b = [t.clone() for t in ops.forward(spec, arena, shared, slot_of, xb, ws)]
    torch.cuda.synchronize()
    assert not torch.equal(ref_a[0], ref_b[0])
    outs = []
    for x in (xa, xb, xa, xb):           # back to back, one synchronisation at the end
        outs.append([t.clone() for t in ops.forward(spec, arena, shared, slot_of, x, ws)])
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        ref = ref_a if i % 2 == 0 else ref_b
        for got, want in zip(o, ref):
            assert torch.equal(got, want), f"eager call {i}"
    xin = xa.clone()
    out = torch.empty(T, D, dtype=torch.bfloat16, device=DEV)
    idx = torch.empty(T, K, dtype=torch.int32, device=DEV)
    wts = torch.empty(T, K, dtype=torch.float32, device=DEV)
    ws_g = ops.Workspace()
    ops.forward(spec, arena, shared, slot_of, xin, ws_g, out=out, idx=idx, weights=wts)   # sizes the workspace
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.forward(spec, arena, shared, slot_of, xin, ws_g, out=out, idx=idx, weights=wts)
    for r, x in enumerate((xa, xb, xa)):
        xin.copy_(x)
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        ref = ref_a if r % 2 == 0 else ref_b
        assert torch.equal(out, ref[0]) and torch.equal(idx, ref[1]) and torch.equal(wts, ref[2]), f"replay {r}"
        e_out = ops.forward(spec, arena, shared, slot_of, xb if r % 2 == 0 else xa, ws)[0]   # eager work between
        torch.cuda.synchronize()
        assert torch.equal(e_out, (ref_b if r % 2 == 0 else ref_a)[0]), f"eager call after replay {r}"


def test_prefill_full_width_long_call(oracle_lib):
    """2048 tokens (a long prompt), Zipf(1.1) routing, 2-bit g64 bf16: tile
    lists of thousands of tiles (experts of hundreds of positions, several
    64-position tiles each), the four-position small down tiles, and the
    shared expert's 32 tiles, checked on every tile kind against the C
    oracle."""
    banner("full-width prefill T=2048 zipf 1.1")
    T = 2048
    arena, shared = _layer(seed=440)
    x, w = synth.zipf_router_inputs(T, E, D, 1.1, torch.bfloat16, seed=441, device=DEV)
    spec = ops.RouterSpec(w, K, routed_scale=1.5)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    out, idx, wts = ops.forward(spec, arena, shared, slot_of, x, ops.Workspace())
    torch.cuda.synchronize()
    _check_routes(x, w, idx, wts)
    ih = idx.cpu().numpy()
    tokens, seg = _tile_sample(ih, T, heavy=4, mid=6, small=6, quad=3, seed=T)
    counts = [len(v) for v in seg.values()]
    assert max(counts) > 4 * TILE and any(1 <= c % TILE <= 4 for c in counts)
    _oracle_check(oracle_lib, arena, shared, x, (ih + 1).astype(np.int32), wts.cpu().numpy(), out,
                  tokens, "C3 T=2048")


def test_mixed_2_4_bit_prefill_full_width(oracle_lib):
    """256 tokens, Zipf(1.1) routing, gate/up 2-bit and down 4-bit: the call
    size from which the down stage's small tiles take up to four positions
    (the 4-bit four-position kernel), checked on every tile kind."""
    banner("full-width mixed 2/4-bit T=256 zipf 1.1")
    T = 256
    arena, shared = _layer(seed=420, bits_down=4)
    x, w = synth.zipf_router_inputs(T, E, D, 1.1, torch.bfloat16, seed=421, device=DEV)
    spec = ops.RouterSpec(w, K, routed_scale=1.5)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    out, idx, wts = ops.forward(spec, arena, shared, slot_of, x, ops.Workspace())
    torch.cuda.synchronize()
    _check_routes(x, w, idx, wts)
    ih = idx.cpu().numpy()
    tokens, seg = _tile_sample(ih, T, seed=T)
    counts = [len(v) for v in seg.values()]
    assert any(c in (3, 4) for c in counts) and any(c <= 2 for c in counts) and max(counts) > TILE
    _oracle_check(oracle_lib, arena, shared, x, (ih + 1).astype(np.int32), wts.cpu().numpy(), out,
                  tokens, "mixed 2/4-bit T=256")


def test_mixed_2_4_bit_batched_decode_full_width(oracle_lib):
    """32 tokens, uniform routing, gate/up 2-bit and down 4-bit."""
    banner("full-width mixed 2/4-bit T=32")
    T = 32
    arena, shared = _layer(seed=400, bits_down=4)
    assert (arena.gate.bits, arena.down.bits) == (2, 4)
    w, bias = synth.uniform_router(E, D, torch.bfloat16, seed=401, device=DEV, bias_std=0.01)
    spec = ops.RouterSpec(w, K, routed_scale=1.5, score_bias=bias)
    x = synth.activations(T, D, torch.bfloat16, seed=402, device=DEV)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    out, idx, wts = ops.forward(spec, arena, shared, slot_of, x, ops.Workspace())
    torch.cuda.synchronize()
    _check_routes(x, w, idx, wts, bias=bias)
    _oracle_check(oracle_lib, arena, shared, x, (idx.cpu().numpy() + 1).astype(np.int32),
                  wts.cpu().numpy(), out, list(range(T)), "C4 T=32")


# ---------------------------------------------------------------------------
# A stack of full-width layers through one bounded arena
# ---------------------------------------------------------------------------
PAYLOADS = 32        # distinct expert payloads: expert e of every layer holds payload e % 32


def _cols(layer):
    return (layer % (D // E)) * E


def _slice_router(layer):
    """Wg = identity on x's columns [256 (layer % 16), +256): x . Wg^T is
    that slice of x."""
    w = torch.zeros(E, D, dtype=torch.bfloat16, device=DEV)
    c = _cols(layer)
    w[:, c:c + E] = torch.eye(E, dtype=torch.bfloat16, device=DEV)
    return w


class _Stack:
    """`layers` full-width layers (each with its own shared expert) over one
    V4ArenaStore with `per_layer` usable slots per layer, misses copied from
    pinned host memory; routing by the router kernel on an identity gate, x
    carrying Zipf(1.1) logits with AR(1) cross-layer noise (rho 0.6)."""

    def __init__(self, tmp_path, layers, per_layer, policy, seed, steps, predict_next=False,
                 device_planner=False):
        from locali_amd.dsv4_arena import V4ArenaMoE, V4ArenaStore, V4Gate
        self.layers = layers
        index = tmp_path / "stack.idx"
        index.write_text(json.dumps(synth.stack_index(layers, E, K, D, DFF, bits=2, group=GROUP)))
        self.payload = synth.expert_arena(PAYLOADS + 1, D, DFF, bits_gate_up=2, group=GROUP,
                                          dtype=torch.bfloat16, seed=seed, device=DEV)
        self.host = synth.host_payloads(self.payload)
        item = self.host.shape[1]
        self.store = V4ArenaStore(index, ceiling_gb=(layers * per_layer + 1) * item / 1e9 + 1e-6,
                                  threads=1, cache_policy=policy, device=DEV, device_planner=device_planner,
                                  host_source=lambda layer, e: self.host[1 + e % PAYLOADS])
        sh = synth.expert_arena(layers, D, DFF, bits_gate_up=2, group=GROUP, dtype=torch.bfloat16,
                                seed=seed + 1, device=DEV, zero_slot=False)
        self.shared = [ops.ExpertArenaT(*(ops.ProjArena(p.weight[i:i + 1], p.scales[i:i + 1],
                                                        p.biases[i:i + 1], p.bits, p.group_size)
                                          for p in (sh.gate, sh.up, sh.down)))
                       for i in range(layers)]
        # layer l's gate reads its logits from columns [256 (l % 16), +256) of x
        self.gates = [V4Gate(_slice_router(layer), top_k=K, routed_scaling_factor=1.5)
                      for layer in range(layers)]
        self.mods = [V4ArenaMoE(self.store, layer, self.gates[layer], K, shared_expert=self.shared[layer])
                     for layer in range(layers)]
        logits = synth.layered_zipf_logits(steps, layers, E, 1.1, 0.6, seed=seed + 3).to(DEV, torch.bfloat16)
        self.X = synth.activations(steps * layers, D, torch.bfloat16, seed=seed + 2,
                                   device=DEV).view(steps, layers, D)
        for layer in range(layers):
            c = _cols(layer)
            self.X[:, layer, c:c + E] = logits[:, layer]
            # the next layer's logits ride in this layer's input for every
            # other token: a next-layer gate on this input (the reference's
            # cross-layer predictor) then guesses right half the time
            if predict_next and layer + 1 < layers:
                n = _cols(layer + 1)
                self.X[::2, layer, n:n + E] = logits[::2, layer + 1]

    def resident(self, layer, x):
        """The same call on the payloads held resident: expert e in slot
        1 + e % 32 of one all-resident arena."""
        idx, wts = self.gates[layer](x)
        slots = (1 + idx.reshape(-1, K) % PAYLOADS).to(torch.int32).contiguous()
        return ops.expert_decode(self.payload, self.shared[layer], x, slots, wts.reshape(-1, K)), idx

    def close(self):
        self.store.close()


def _run_stack(stack, steps, oracle_lib=None, check_every=0):
    outs = []
    for t in range(steps):
        for layer in range(stack.layers):
            x = stack.X[t, layer:layer + 1]
            got = stack.mods[layer](x)
            want, idx = stack.resident(layer, x)
            assert torch.equal(got, want), f"token {t} layer {layer}"
            outs.append(got)
            if oracle_lib is not None and check_every and (t * stack.layers + layer) % check_every == 0:
                slots = (1 + idx.reshape(-1, K).cpu().numpy() % PAYLOADS).astype(np.int32)
                _, wts = stack.gates[layer](x)
                _oracle_check(oracle_lib, stack.payload, stack.shared[layer], x, slots,
                              wts.reshape(-1, K).cpu().numpy(), got, [0], f"stack token {t} layer {layer}",
                              exact=None)
    torch.cuda.synchronize()
    return outs


@pytest.mark.parametrize("policy", ["slru-all", "lfu-decay"])
def test_bounded_stack_full_width_host_fills(tmp_path, oracle_lib, policy):
    """Four full-width layers, 12 usable slots per layer (49 slots, 385 MB),
    16 decode tokens: every layer call equals the same routes on resident
    weights bit for bit, through misses and evictions; oracle spot checks."""
    banner(f"full-width bounded stack policy={policy}")
    steps = 16
    stack = _Stack(tmp_path, layers=4, per_layer=12, policy=policy, seed=500, steps=steps)
    try:
        _run_stack(stack, steps, oracle_lib, check_every=7)
        st = stack.store.stats()
        assert st["misses"] > 0 and st["evictions"] > 0 and st["hits"] > 0
        assert st["bytes_read"] == st["misses"] * stack.store.item["cold"]
    finally:
        stack.close()


@pytest.mark.parametrize("policy", ["slru-all", "lfu-decay"])
def test_bounded_stack_device_planner_equals_host_planner(tmp_path, policy):
    """The same four-layer stack planned on the GPU (V4ArenaStore
    device_planner=True: router, planner, fills and experts queued with no
    host round trip): every layer call equals the resident weights bit for
    bit, and hits, misses, evictions and bytes equal the host-planned run's."""
    banner(f"full-width bounded stack, device planner, policy={policy}")
    steps = 16
    counts = []
    for device_planner in (False, True):
        stack = _Stack(tmp_path, layers=4, per_layer=12, policy=policy, seed=500, steps=steps,
                       device_planner=device_planner)
        try:
            _run_stack(stack, steps)
            st = stack.store.stats()
            counts.append((st["hits"], st["misses"], st["evictions"], st["bytes_read"]))
        finally:
            stack.close()
    assert counts[0] == counts[1]
    assert counts[0][1] > 0 and counts[0][2] > 0


def test_device_planner_prefill_batches_equal_host_planner(tmp_path):
    """Multi-token calls (16 tokens per layer: the routes are planned on the
    device and the grouped kernels read its slot table) give the same
    outputs, bit for bit, and the same counters as the host-planned store."""
    banner("full-width bounded stack, 16-token calls, device planner")
    steps = 16
    outs, counts = [], []
    for device_planner in (False, True):
        # 96 usable slots per layer: probation (the half not protected) then
        # holds the 96 routes of a call plus the previous call's 96 pinned
        stack = _Stack(tmp_path, layers=4, per_layer=96, policy="slru-all", seed=520, steps=steps,
                       device_planner=device_planner)
        try:
            got = []
            for rep in range(2):
                for layer in range(stack.layers):
                    # twice in a row: the second call hits what the first placed
                    got.append(stack.mods[layer](stack.X[:, layer]))
                    got.append(stack.mods[layer](stack.X[:, layer]))
            torch.cuda.synchronize()
            outs.append(got)
            st = stack.store.stats()
            counts.append((st["hits"], st["misses"], st["evictions"], st["bytes_read"]))
        finally:
            stack.close()
    assert counts[0] == counts[1] and counts[0][0] > 0 and counts[0][1] > 0
    for i, (a, b) in enumerate(zip(*outs)):
        assert torch.equal(a, b), f"call {i}"


def test_device_planner_refuses_a_call_it_might_not_place(tmp_path):
    """A device-planned call whose keys plus the previous call's pinned
    slots exceed what probation holds could leave a demanded expert without
    a slot, which the kernel would answer with the zero slot: V4ArenaMoE
    raises before queueing anything instead. 4 layers x 2 usable slots (9
    slots, 4 protected): a decode call's six experts do not fit probation's
    four."""
    banner("device planner refuses an unplaceable call")
    stack = _Stack(tmp_path, layers=4, per_layer=2, policy="slru-all", seed=530, steps=1, device_planner=True)
    try:
        with pytest.raises(RuntimeError, match="may find no unpinned slot"):
            stack.mods[0](stack.X[0, 0:1])
        assert stack.store.stats()["misses"] == 0
    finally:
        stack.close()


def test_cross_layer_prefetch_is_exact_and_accounted(tmp_path):
    """The reference's cross-layer prefetch (arena.py:520-541, wired by
    dsv4_engine.py:237-246): each layer's call also routes the next layer's
    (depth 1, its three highest-gate experts) and the one after (depth 2, all
    six) on the current input and claims and fills those slots before the
    later layers run. Outputs equal the resident kernels bit for bit; the
    prefetch counters move (prefetched, then used or wasted)."""
    banner("full-width stack with cross-layer prefetch")
    steps = 12
    stack = _Stack(tmp_path, layers=4, per_layer=16, policy="slru-all", seed=600, steps=steps,
                   predict_next=True)
    try:
        for layer, mod in enumerate(stack.mods):
            mod.nxt = stack.mods[layer + 1] if layer + 1 < stack.layers else None
            mod.prefetch_k = 3
            mod.nxt2 = stack.mods[layer + 2] if layer + 2 < stack.layers else None
            mod.prefetch_k2 = None
        _run_stack(stack, steps)
        st = stack.store.stats()
        assert st["prefetched"] > 0 and st["prefetch_used"] > 0 and st["prefetch_wasted"] > 0
        assert st["prefetch_used"] + st["prefetch_wasted"] <= st["prefetched"]
    finally:
        stack.close()


def test_cross_layer_prefetch_device_planner_equals_host_planner(tmp_path):
    """The same cross-layer prefetch (depth 1: the three highest-gate
    experts of the next layer's routing on the current input; depth 2: all
    six of the layer after) planned on the GPU: the lookahead gates run on
    the fill stream, and the prefetch planner calls and their copies follow
    each layer's demand call there (locali_dplan_prefetch). Every layer call
    equals the resident weights bit for bit, and hits, misses, evictions,
    bytes and the prefetch counters equal the host-planned run's."""
    banner("full-width stack with cross-layer prefetch, device planner")
    steps = 12
    counts = []
    for device_planner in (False, True):
        stack = _Stack(tmp_path, layers=4, per_layer=16, policy="slru-all", seed=600, steps=steps,
                       predict_next=True, device_planner=device_planner)
        try:
            for layer, mod in enumerate(stack.mods):
                mod.nxt = stack.mods[layer + 1] if layer + 1 < stack.layers else None
                mod.prefetch_k = 3
                mod.nxt2 = stack.mods[layer + 2] if layer + 2 < stack.layers else None
                mod.prefetch_k2 = None
            _run_stack(stack, steps)
            st = stack.store.stats()
            counts.append(tuple(st[k] for k in ("hits", "misses", "evictions", "bytes_read", "prefetched",
                                                "prefetch_used", "prefetch_wasted")))
        finally:
            stack.close()
    assert counts[0] == counts[1], counts
    assert counts[0][4] > 0 and counts[0][5] > 0
