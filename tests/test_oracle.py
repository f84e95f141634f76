"""Pins the CPU oracle itself (CPU only).

Each oracle function is checked against something that does not restate its
own formula: literal packed words worked out by hand, the reference's kernel
text for code extraction (dsv4_kernels.py:59-73), special cases with closed
forms, torch/numpy library routines, an independent C restatement
(oracle/expert_ref.c), and golden router vectors from the transformers
DeepSeek-V4 router classes (tests/golden/make_router_vectors.py).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import affine, moe

GOLD = Path(__file__).resolve().parent / "golden"


# -- affine layout ------------------------------------------------------------

def test_pack_literal_words():
    # 4-bit LSB-first: value j in bits [4j, 4j+3]
    assert affine.pack(np.array([[1, 2, 3, 4, 5, 6, 7, 8]]), 4)[0, 0] == 0x87654321
    # 2-bit: codes 1,2,3,0 -> byte 0b00111001 = 0x39, repeated
    assert affine.pack(np.array([[1, 2, 3, 0] * 4]), 2)[0, 0] == 0x39393939
    # 8-bit: bytes in order
    assert affine.pack(np.array([[0x11, 0x22, 0x33, 0xF4]]), 8)[0, 0] == 0xF4332211
    # 3-bit: codes 0..7 are the 24-bit stream 0o76543210 = 0xFAC688 (bytes
    # 88 C6 FA), repeated; 32 values fill three words, values 10 and 21
    # crossing word boundaries
    assert list(affine.pack(np.array([list(range(8)) * 4]), 3)[0]) == [0x88FAC688, 0xC688FAC6, 0xFAC688FA]


def test_3bit_stream_is_one_little_endian_integer():
    """Value j of a 3-bit row is bits [3j, 3j+3) of the row's words read as
    one little-endian integer (checked with Python integers)."""
    rng = np.random.default_rng(9)
    q = rng.integers(0, 8, size=(4, 96), dtype=np.uint8)
    w = affine.pack(q, 3)
    assert w.shape == (4, 9)
    for r in range(4):
        big = sum(int(v) << (32 * i) for i, v in enumerate(w[r]))
        assert [(big >> (3 * j)) & 7 for j in range(96)] == list(q[r])


def test_unpack_matches_reference_kernel_text_extraction():
    """dsv4_kernels.py:59-73: lane reads word block/16 + lane/2, shifts by
    (lane & 1) * 16 and peels 8 two-bit values LSB first."""
    rng = np.random.default_rng(3)
    K = 512
    words = rng.integers(0, 2**32, size=(3, K // 16), dtype=np.uint64).astype(np.uint32)
    ours = affine.unpack(words, 2)
    for row in range(3):
        for block in range(0, K, 256):
            for lane in range(32):
                uw = int(words[row, block // 16 + lane // 2]) >> ((lane & 1) * 16)
                for j in range(8):
                    assert ours[row, block + lane * 8 + j] == (uw & 3)
                    uw >>= 2


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_pack_unpack_roundtrip(bits):
    rng = np.random.default_rng(bits)
    q = rng.integers(0, 2**bits, size=(5, 256), dtype=np.uint8)
    assert np.array_equal(affine.unpack(affine.pack(q, bits), bits), q)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    a = np.concatenate([rng.standard_normal(10000) * 10.0 ** rng.integers(-30, 30, 10000),
                        [0.0, -0.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 65504.0, 1e-40]]).astype(np.float32)
    want = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    assert np.array_equal(affine.round_to(a, "bf16"), want)


def test_c_oracle_rounding_matches_torch(oracle_lib):
    rng = np.random.default_rng(1)
    a = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
                        [65504.0, 65519.0, 65520.0, 6.0e-8, 2.0**-24 * 1.5, 2.0**-25, -3e-6]])
    a = a.astype(np.float32)
    assert np.array_equal(oracle_lib.round_array(a, "f16"),
                          torch.from_numpy(a).half().float().numpy())
    assert np.array_equal(oracle_lib.round_array(a, "bf16"),
                          torch.from_numpy(a).bfloat16().float().numpy())


# -- qmv ----------------------------------------------------------------------

def _rand_proj(rng, N, K, bits, group, dt="bf16"):
    q = rng.integers(0, 2**bits, size=(N, K), dtype=np.uint8)
    s = affine.round_to(rng.uniform(0.01, 0.05, size=(N, K // group)), dt)
    b = affine.round_to(rng.uniform(-0.1, 0.0, size=(N, K // group)), dt)
    return q, affine.pack(q, bits), s, b


@pytest.mark.parametrize("bits,group", [(2, 64), (4, 64), (2, 128), (4, 32), (8, 64), (3, 64), (3, 32)])
def test_qmv_equals_torch_dense_matmul(bits, group):
    rng = np.random.default_rng(bits * 1000 + group)
    N, K = 48, 512
    q, w, s, b = _rand_proj(rng, N, K, bits, group)
    x = rng.standard_normal((3, K))
    dense = torch.from_numpy(q.astype(np.float64)) * torch.from_numpy(s).double().repeat_interleave(group, 1) \
        + torch.from_numpy(b).double().repeat_interleave(group, 1)
    want = torch.from_numpy(x) @ dense.T
    np.testing.assert_allclose(affine.qmv(x, w, s, b, bits, group), want.numpy(), rtol=1e-12, atol=1e-12)


def test_qmv_special_cases():
    rng = np.random.default_rng(5)
    N, K, G = 8, 256, 64
    s = rng.uniform(0.5, 1.0, (N, K // G))
    b = rng.uniform(-1.0, 1.0, (N, K // G))
    x = rng.standard_normal(K)
    zero_codes = affine.pack(np.zeros((N, K), np.uint8), 2)
    # all-zero codes -> sum_g bias_g * sum(x in g)
    want = (b * x.reshape(K // G, G).sum(1)).sum(1)
    np.testing.assert_allclose(affine.qmv(x, zero_codes, s, b, 2, G), want, rtol=1e-12)
    # one-hot x picks column j of the dequantised matrix: s*q + b
    q = rng.integers(0, 4, (N, K), dtype=np.uint8)
    j = 77
    e = np.zeros(K)
    e[j] = 1.0
    np.testing.assert_allclose(affine.qmv(e, affine.pack(q, 2), s, b, 2, G),
                               s[:, j // G] * q[:, j] + b[:, j // G], rtol=1e-12)
    # zero slot (all-zero words, scales, biases) contributes exactly 0
    assert np.all(affine.qmv(x, zero_codes, 0 * s, 0 * b, 2, G) == 0.0)


@pytest.mark.parametrize("dt,bits", [("bf16", (2, 4)), ("f16", (2, 4)), ("bf16", (3, 3))])
def test_c_oracle_layer_matches_numpy_oracle(oracle_lib, dt, bits):
    rng = np.random.default_rng(11)
    S, d, dff, k, T = 5, 256, 128, 2, 3
    arena, arena_c = {}, {}
    for name, (N, K, bits) in {"gate_proj": (dff, d, bits[0]), "up_proj": (dff, d, bits[0]),
                               "down_proj": (d, dff, bits[1])}.items():
        ws, ss, bs = [], [], []
        for _ in range(S):
            _, w, s, b = _rand_proj(rng, N, K, bits, 64, dt)
            ws.append(w), ss.append(s), bs.append(b)
        w, s, b = np.stack(ws), np.stack(ss), np.stack(bs)
        arena[name] = (w, s, b, bits, 64)
        arena_c[name] = (w, affine.to_bits16(s, dt), affine.to_bits16(b, dt), bits, 64)
    x = affine.round_to(rng.standard_normal((T, d)) * 3, dt)
    idx = np.array([[1, 3], [4, 1], [2, 2]])
    wts = rng.uniform(0.1, 1.0, (T, k)).astype(np.float32)
    slot_of = {e: e for e in range(S)}
    want = moe.moe_layer(x, idx, wts, arena, slot_of, dt, limit=1.5)
    got = oracle_lib.moe_layer(x, idx, wts, arena_c, dt, limit=1.5)
    # fp32 vs fp64 accumulation: equal up to an occasional last-place flip
    np.testing.assert_allclose(got, want, rtol=2e-2 if dt == "bf16" else 4e-3, atol=2e-3)
    assert np.mean(got == want) > 0.9


# -- SwiGLU and the expert: transformers DeepSeek-V4 expert classes ------------
# tests/golden/make_swiglu_vectors.py ran DeepseekV4Experts._apply_gate,
# DeepseekV4MLP and DeepseekV4Experts (modeling_deepseek_v4.py:965-1021) in
# float64 on dense matrices expanded from affine codes; "f64" runs the oracle
# with no rounding, so the two must agree to float64 noise.

PROJ_NAMES = ("gate_proj", "up_proj", "down_proj")


def _swiglu_gold():
    return np.load(GOLD / "swiglu_vectors.npz")


def _gold_experts(g, case):
    bits, group, E = (int(v) for v in g[f"{case}_meta"][:3])
    return [{p: (affine.pack(g[f"{case}_{p}_q_{e}"], bits), g[f"{case}_{p}_s_{e}"],
                 g[f"{case}_{p}_b_{e}"], bits, group) for p in PROJ_NAMES} for e in range(E)]


def _check_against_transformers(g):
    """Every golden comparison for the SwiGLU and the expert (AssertionError
    on the first mismatch)."""
    for i, limit in enumerate(g["limits"]):
        np.testing.assert_allclose(moe.swiglu(g["gate"], g["up"], "f64", limit=float(limit)),
                                   g[f"h64_{i}"], rtol=1e-13, atol=1e-13)
    for case in ("a", "b"):
        limit = float(g[f"{case}_limit"])
        x = g[f"{case}_x"]
        experts = _gold_experts(g, case)
        for e, proj in enumerate(experts):
            np.testing.assert_allclose(moe.expert(x, proj, "f64", limit), g[f"{case}_mlp"][:, e],
                                       rtol=1e-11, atol=1e-11)
        arena = {p: (np.stack([ex[p][0] for ex in experts]), np.stack([ex[p][1] for ex in experts]),
                     np.stack([ex[p][2] for ex in experts]), experts[0][p][3], experts[0][p][4])
                 for p in PROJ_NAMES}
        routed = moe.moe_layer(x, g[f"{case}_idx"], g[f"{case}_wts"], arena,
                               {e: e for e in range(len(experts))}, "f64", limit=limit)
        np.testing.assert_allclose(routed, g[f"{case}_routed"], rtol=1e-11, atol=1e-10)


def test_swiglu_and_expert_match_transformers_deepseek_v4():
    g = _swiglu_gold()
    assert min(float(g["a_clamped"]), float(g["b_clamped"])) > 0.2    # the clamp is exercised
    _check_against_transformers(g)


@pytest.mark.parametrize("i", [0, 1, 2])
def test_fp32_swiglu_matches_transformers_float32_gate(i):
    """fp32_swiglu (dsv4_arena.py:228-232): SiLU(gate) * up in float32, one
    rounding to the activation dtype. Against _apply_gate run in float32 and
    rounded to bf16: float32 SiLU implementations may differ in the last fp32
    place, which can move a bf16 rounding by one place, never more."""
    g = _swiglu_gold()
    limit = float(g["limits"][i])
    got = moe.swiglu(g["gate"], g["up"], "bf16", limit=limit, fp32_swiglu=True)
    want = affine.round_to(g[f"h32_{i}"], "bf16")
    assert np.mean(got == want) > 0.97
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)


def _silu(v):
    return v / (1.0 + np.exp(-v))


SWIGLU_MUTANTS = {
    "gate clipped from below too": lambda g, u, L: _silu(np.clip(g, -L, L)) * np.clip(u, -L, L),
    "cap applied after SiLU": lambda g, u, L: np.minimum(_silu(g), L) * np.clip(u, -L, L),
    "up not clipped": lambda g, u, L: _silu(np.minimum(g, L)) * u,
    "up clipped from above only": lambda g, u, L: _silu(np.minimum(g, L)) * np.minimum(u, L),
    "gate and up swapped": lambda g, u, L: _silu(np.minimum(u, L)) * np.clip(g, -L, L),
    "sigmoid in place of SiLU": lambda g, u, L: (1 / (1 + np.exp(-np.minimum(g, L)))) * np.clip(u, -L, L),
}


@pytest.mark.parametrize("mutant", sorted(SWIGLU_MUTANTS))
def test_golden_vectors_reject_planted_swiglu_mistakes(mutant, monkeypatch):
    """A misreading of the clamp (dsv4_arena.py:225-227) planted in the oracle
    must fail the transformers comparison."""
    wrong = SWIGLU_MUTANTS[mutant]

    def planted(gate, up, dtype, limit=10.0, fp32_swiglu=False):
        g64, u64 = np.asarray(gate, np.float64), np.asarray(up, np.float64)
        return affine.round_to(wrong(g64, u64, limit) if limit > 0 else _silu(g64) * u64, dtype)

    monkeypatch.setattr(moe, "swiglu", planted)
    with pytest.raises(AssertionError):
        _check_against_transformers(_swiglu_gold())


def test_swiglu_closed_forms():
    rng = np.random.default_rng(17)
    gate, up = rng.uniform(-20, 20, 500), rng.uniform(-20, 20, 500)
    # limit <= 0: no clamp at all (dsv4_arena.py:225); SiLU from torch
    silu = torch.nn.functional.silu(torch.from_numpy(gate)).numpy()
    for limit in (0.0, -1.0):
        np.testing.assert_allclose(moe.swiglu(gate, up, "f64", limit=limit), silu * up, rtol=1e-14)
    # gate at or above the limit: SiLU(limit) * clip(up)
    L = 3.0
    hi = L + rng.uniform(0, 50, 500)
    np.testing.assert_allclose(moe.swiglu(hi, up, "f64", limit=L),
                               (L / (1 + np.exp(-L))) * np.clip(up, -L, L), rtol=1e-14)
    # up beyond +-limit saturates at +-limit; gate is not raised from below
    low = np.full(4, -40.0)
    out = moe.swiglu(low, np.array([-50.0, -5.0, 5.0, 50.0]), "f64", limit=10.0)
    np.testing.assert_allclose(out, _silu(-40.0) * np.array([-10.0, -5.0, 5.0, 10.0]), rtol=1e-14)


def test_expert_closed_form_all_zero_codes():
    """All-zero codes leave w = bias: with constant biases and x = 0.1 the
    projections are bias * sum(x), worked out by hand; the clamp then acts on
    the hand values."""
    d, dff, group = 128, 64, 64

    def proj(rows, cols, bias):
        return (affine.pack(np.zeros((rows, cols), np.uint8), 2), np.full((rows, cols // group), 0.03),
                np.full((rows, cols // group), bias), 2, group)

    experts = {"gate_proj": proj(dff, d, 0.25), "up_proj": proj(dff, d, 0.5), "down_proj": proj(d, dff, 0.125)}
    x = np.full((1, d), 0.1)
    sx = 0.1 * d                                      # 12.8: up = 6.4, gate = 3.2
    for limit, (g, u) in ((10.0, (3.2, 6.4)), (2.0, (2.0, 2.0)), (0.0, (3.2, 6.4))):
        assert (0.25 * sx, 0.5 * sx) == pytest.approx((3.2, 6.4))
        h = g / (1 + np.exp(-g)) * u
        y = moe.expert(x, experts, "f64", limit)
        np.testing.assert_allclose(y, np.full((1, d), 0.125 * dff * h), rtol=1e-13)


# -- router -------------------------------------------------------------------

@pytest.mark.parametrize("case", ["a", "b", "c"])
def test_router_matches_transformers_golden_vectors(case):
    g = np.load(GOLD / "router_vectors.npz")
    x, w, bias = g[f"{case}_x"], g[f"{case}_w"], g[f"{case}_bias"]
    k, scale = int(g[f"{case}_k"]), float(g[f"{case}_scale"])
    idx, wts, margin, _ = moe.route(x, w, k, bias=bias, routed_scale=scale)
    for t in range(x.shape[0]):
        ref = dict(zip(g[f"{case}_idx"][t].tolist(), g[f"{case}_weights"][t].tolist()))
        assert set(idx[t].tolist()) == set(ref), f"token {t}"
        for e, v in zip(idx[t].tolist(), wts[t].tolist()):
            assert v == pytest.approx(ref[e], rel=1e-5)
    np.testing.assert_allclose(wts.sum(1), scale, rtol=1e-9)
    hidx, hw, _, _ = moe.route(x, w, k, routed_scale=scale, tid2eid=g[f"{case}_table"],
                               input_ids=g[f"{case}_ids"])
    assert np.array_equal(hidx, g[f"{case}_hash_idx"])
    np.testing.assert_allclose(hw, g[f"{case}_hash_weights"], rtol=1e-5)


def test_router_sigmoid_variant_and_canonical_order():
    """arena.py:501-506: sigmoid scores, selection on score + bias, weights
    renormalised without scaling; in-row order descending, ties to lower id."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 16))
    w = rng.standard_normal((10, 16))
    bias = rng.standard_normal(10) * 0.1
    idx, wts, _, scores = moe.route(x, w, 3, bias=bias, score_func="sigmoid")
    sel = scores + bias
    for t in range(4):
        assert list(idx[t]) == sorted(range(10), key=lambda e: (-sel[t, e], e))[:3]
        np.testing.assert_allclose(wts[t], scores[t, idx[t]] / scores[t, idx[t]].sum(), rtol=1e-12)
    tie_idx, _, _, _ = moe.route(np.zeros((1, 16)), w, 4, score_func="sigmoid")
    assert list(tie_idx[0]) == [0, 1, 2, 3]


def test_router_sigmoid_pinned_by_torch_and_a_hand_built_case():
    """arena.py:501-506 pinned without the oracle's own formula: scores equal
    torch.sigmoid of the logits, and a hand-built router where the selection
    bias changes which experts are chosen but never enters the weights."""
    import math

    import torch
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 32))
    w = rng.standard_normal((12, 32)) / 4
    _, _, _, scores = moe.route(x, w, 4, score_func="sigmoid")
    ref = torch.sigmoid(torch.from_numpy(x) @ torch.from_numpy(w).T).numpy()
    np.testing.assert_allclose(scores, ref, rtol=1e-13, atol=0)
    # logits [2, 1, 0, -1] (x = e0 .. e3 rows of the identity, times these)
    gate = np.diag([2.0, 1.0, 0.0, -1.0])
    xs = np.ones((1, 4))
    sig = [1.0 / (1.0 + math.exp(-v)) for v in (2.0, 1.0, 0.0, -1.0)]
    idx, wts, _, _ = moe.route(xs, gate, 2, score_func="sigmoid")
    assert idx[0].tolist() == [0, 1]
    np.testing.assert_allclose(wts[0], [sig[0] / (sig[0] + sig[1]), sig[1] / (sig[0] + sig[1])], rtol=1e-14)
    # a bias of 5 on the weakest expert selects it first; its weight is
    # still its own score, renormalised with the other chosen one
    idx, wts, _, _ = moe.route(xs, gate, 2, bias=np.array([0.0, 0.0, 0.0, 5.0]), score_func="sigmoid")
    assert idx[0].tolist() == [3, 0]
    np.testing.assert_allclose(wts[0], [sig[3] / (sig[3] + sig[0]), sig[0] / (sig[3] + sig[0])], rtol=1e-14)
    # routed_scale multiplies after the renormalisation
    _, w2, _, _ = moe.route(xs, gate, 2, bias=np.array([0.0, 0.0, 0.0, 5.0]), score_func="sigmoid",
                            routed_scale=2.5)
    np.testing.assert_allclose(w2, 2.5 * wts, rtol=1e-14)


def test_c_oracle_router_matches_numpy(oracle_lib):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 128)).astype(np.float32)
    w = (rng.standard_normal((64, 128)) / 11).astype(np.float32)
    bias = (rng.standard_normal(64) * 0.05).astype(np.float32)
    idx, wts = oracle_lib.router(x, w, bias, 6, 0, True, 1.5)
    nidx, nw, margin, _ = moe.route(x, w, 6, bias=bias, routed_scale=1.5)
    for t in range(6):
        if margin[t] > 1e-5:
            assert list(idx[t]) == list(nidx[t])
            np.testing.assert_allclose(wts[t], nw[t], rtol=1e-5)


# -- combine / dispatch -------------------------------------------------------

def test_combine_closed_forms():
    y = affine.round_to(np.random.default_rng(0).standard_normal((2, 3, 8)), "bf16")
    # unit weights on one route and zero elsewhere returns that route exactly
    w = np.array([[1.0, 0.0, 0.0], [0.0, 0.0, 1.0]])
    out = moe.combine(y, w, "bf16")
    assert np.array_equal(out[0], y[0, 0]) and np.array_equal(out[1], y[1, 2])
    # powers of two scale exactly
    out = moe.combine(y, np.full((2, 3), 0.25), "bf16")
    np.testing.assert_allclose(out, affine.round_to(y.sum(1) * 0.25, "bf16"), rtol=0, atol=0) \
        if np.all(affine.round_to(y * 0.25, "bf16") == y * 0.25) else None
    # shared add is a rounded sum
    s = affine.round_to(np.ones((2, 8)) * 0.5, "bf16")
    assert np.array_equal(moe.add_shared(np.zeros((2, 8)), s, "bf16"), s)


def test_dispatch_is_stable_slot_sort():
    rng = np.random.default_rng(4)
    slots = rng.integers(1, 9, size=(40, 4))
    order, counts, undo = moe.dispatch(slots)
    flat = slots.reshape(-1)
    assert np.all(np.diff(flat[order]) >= 0)
    for s in np.unique(flat):
        members = order[flat[order] == s]
        assert np.all(np.diff(members) > 0)          # route order kept within a slot
        assert counts[int(s)] == members.size
    assert np.array_equal(order[undo], np.arange(flat.size))
    assert moe.first_appearance([[3, 1], [1, 4], [3, 2]]) == [3, 1, 4, 2]


def test_mixed_tiers_reduces_to_fp32_combine():
    """With weights 1 and 0.5 and two routes per token every float32 product
    and sum is exact, so the mixed-tier accumulation (arena.py:626-672) must
    equal the fp32 combine of the same routes -- whether the routes sit in
    one tier or are split across two tiers holding the same weights at other
    slots. A wrong tier, slot or weight index breaks the equality; the zero
    slot contributes nothing."""
    rng = np.random.default_rng(21)
    S, d, dff, k, T = 5, 256, 128, 2, 4
    arena = {}
    for name, (N, K, bits) in {"gate_proj": (dff, d, 2), "up_proj": (dff, d, 2),
                               "down_proj": (d, dff, 4)}.items():
        ws, ss, bs = [], [], []
        for _ in range(S):
            _, w, s, b = _rand_proj(rng, N, K, bits, 64, "bf16")
            ws.append(w), ss.append(s), bs.append(b)
        arena[name] = (np.stack(ws), np.stack(ss), np.stack(bs), bits, 64)
    # tier "b" holds the same experts in reversed slot order
    rev = {p: (a[0][::-1].copy(), a[1][::-1].copy(), a[2][::-1].copy(), a[3], a[4]) for p, a in arena.items()}
    x = affine.round_to(rng.standard_normal((T, d)), "bf16")
    idx = np.array([[1, 3], [4, 1], [2, 2], [3, 4]])
    wts = np.array([[1.0, 0.5], [0.5, 1.0], [1.0, 1.0], [0.5, 0.5]], dtype=np.float32)
    want = moe.moe_layer(x, idx, wts, arena, {e: e for e in range(S)}, "bf16", limit=1.5,
                         combine_mode="fp32")
    one, _ = moe.mixed_tiers(x, [["a"] * k] * T, idx, wts, {"a": arena}, ["a"], "bf16", limit=1.5)
    assert np.array_equal(one, want)
    tier_of = [["a", "b"], ["b", "a"], ["b", "b"], ["a", "a"]]
    slot = np.array([[e if t == "a" else S - 1 - e for t, e in zip(tr, row)] for tr, row in zip(tier_of, idx)])
    two, _ = moe.mixed_tiers(x, tier_of, slot, wts, {"a": arena, "b": rev}, ["a", "b"], "bf16", limit=1.5)
    assert np.array_equal(two, want)
    # a route in the zero slot adds exactly nothing
    zero = {p: (np.zeros_like(a[0]), np.zeros_like(a[1]), np.zeros_like(a[2]), a[3], a[4]) for p, a in arena.items()}
    z, _ = moe.mixed_tiers(x, [["a", "z"]] * T, np.array([[r[0], 0] for r in idx]),
                           wts, {"a": arena, "z": zero}, ["a", "z"], "bf16", limit=1.5)
    w1 = wts.copy()
    w1[:, 1] = 0.0
    assert np.array_equal(z, moe.moe_layer(x, idx, w1, arena, {e: e for e in range(S)}, "bf16", limit=1.5,
                                           combine_mode="fp32"))
