"""Synthetic workload generators: the layer-stack routing keeps each layer's
Zipf marginal and has the stated cross-layer dependence; the stack index and
host payloads have the store's layout."""

from __future__ import annotations

import math

import numpy as np
import torch

from locali_amd import synth
from locali_amd.arena import ArenaStore


def _ranks(a):
    return np.argsort(np.argsort(a, axis=0), axis=0).astype(np.float64)


def test_layered_zipf_marginal_and_copula_correlation():
    T, L, E, s, rho = 20000, 3, 16, 1.1, 0.6
    logits = synth.layered_zipf_logits(T, L, E, s, rho, seed=3).double().numpy()
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    for layer in range(L):
        # Gumbel-max: the top-1 expert is distributed as p over the layer's ranks
        freq = np.bincount(logits[:, layer].argmax(1), minlength=E) / T
        assert abs(np.sort(freq)[::-1][0] - p[0]) < 4 * math.sqrt(p[0] * (1 - p[0]) / T)
        assert abs(np.sort(freq)[::-1][:4].sum() - p[:4].sum()) < 0.02
    # per expert, the noise across tokens has Spearman correlation
    # (6/pi) asin(r/2) with r = rho^|dl| between layers
    for dl in (1, 2):
        r = rho ** dl
        want = 6 / math.pi * math.asin(r / 2)
        a, b = _ranks(logits[:, 0]), _ranks(logits[:, dl])
        got = np.mean([np.corrcoef(a[:, e], b[:, e])[0, 1] for e in range(E)])
        assert abs(got - want) < 0.02, (dl, got, want)


def test_stack_index_and_host_payloads_fit_the_store(tmp_path):
    import json
    L, E, d, dff = 2, 4, 256, 128
    idx = synth.stack_index(L, E, 2, d, dff)
    path = tmp_path / "stack.idx"
    path.write_text(json.dumps(idx))
    arena = synth.expert_arena(E, d, dff, seed=4, zero_slot=False)
    host = synth.host_payloads(arena)
    st = ArenaStore(path, ceiling_gb=3 * host.shape[1] / 1e9 + 1e-9, threads=1, device="cpu",
                    host_source=lambda layer, e: host[e])
    try:
        assert st.item["cold"] == host.shape[1] == idx["expert_bytes"] // (L * E)
        placed = st.slots_for(1, [2, 3])
        ea = st.expert_arena("cold")
        for e, (_, slot) in placed.items():
            for mine, theirs in zip((ea.gate, ea.up, ea.down), (arena.gate, arena.up, arena.down)):
                assert torch.equal(mine.weight[slot], theirs.weight[e])
                assert torch.equal(mine.scales[slot], theirs.scales[e])
                assert torch.equal(mine.biases[slot], theirs.biases[e])
    finally:
        st.close()
