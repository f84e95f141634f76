"""GPU parity: the HIP kernels (through the liblocali_amd.so C ABI) against the
CPU oracle on identical seeded inputs.

Bars: router indices bit-exact as sets wherever the oracle's
selection margin exceeds the fp32 accumulation-order noise (1e-4); weights
within 1e-5 relative; slot assignment exact; expert outputs within 1e-2
relative / 2e-3 absolute of the oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_helpers import (arena_numpy, assert_close, assert_close_terms, banner, dt_name,
                         exact_fraction, ulp, ulp_distance, values)
from locali_amd import ops, synth
from oracle import affine, moe

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dev(arena):
    return ops.ExpertArenaT(*(ops.ProjArena(p.weight.to(DEV), p.scales.to(DEV), p.biases.to(DEV),
                                            p.bits, p.group_size)
                              for p in (arena.gate, arena.up, arena.down)))


def _oracle_layer(x, idx, wts, arena, slot_of, dtype, shared=None, limit=10.0, fp32_swiglu=False,
                  return_terms=False):
    dt = dt_name(dtype)
    sh = None
    if shared is not None:
        sh = {k: (v[0][0], v[1][0], v[2][0], v[3], v[4]) for k, v in arena_numpy(shared).items()}
    return moe.moe_layer(values(x), idx, wts, arena_numpy(arena), slot_of, dt, limit=limit,
                         fp32_swiglu=fp32_swiglu, shared=sh, return_terms=return_terms)


def close_fraction(got, want, dtype) -> float:
    """Fraction of combined outputs equal to the oracle at bf16 resolution:
    exactly equal for bf16; for fp16 (three more significant bits) within
    one fp16 spacing, an eighth of the bf16 spacing, so a deviation it allows
    is smaller than any the bf16 bar could see."""
    if dtype == torch.bfloat16:
        return exact_fraction(got, want)
    return float(np.mean(ulp_distance(got, want, dtype) <= 1))


# ---------------------------------------------------------------------------
# Router
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("T", [1, 3, 40, 130])
@pytest.mark.parametrize("score", ["sqrtsoftplus", "sigmoid", "softmax"])
def test_router_matches_oracle(T, score):
    banner(f"router T={T} score={score}")
    E, d, k = 256, 1024, 6
    w, bias = synth.uniform_router(E, d, torch.bfloat16, seed=T, bias_std=0.01)
    x = synth.activations(T, d, torch.bfloat16, seed=T + 7)
    slot_of = torch.randperm(E, generator=torch.Generator().manual_seed(5)).to(torch.int32) + 1
    spec = ops.RouterSpec(w.to(DEV), k, score_func=score, routed_scale=1.5,
                          score_bias=bias.to(DEV))
    ws = ops.Workspace()
    idx, wts, rs = ops.router(spec, x.to(DEV), ws, slot_of_expert=slot_of.to(DEV), n_slots=E + 1)
    torch.cuda.synchronize()
    oi, ow, margin, _ = moe.route(values(x), values(w), k, bias=values(bias), score_func=score,
                                  routed_scale=1.5)
    idx, wts, rs = idx.cpu().numpy(), wts.cpu().numpy(), rs.cpu().numpy()
    _, _, _, scores = moe.route(values(x), values(w), k, bias=values(bias), score_func=score)
    scale = np.abs(scores).max(axis=1) + np.abs(values(bias)).max()
    checked = 0
    for t in range(T):
        if margin[t] < 1e-4 * scale[t]:      # fp32 accumulation-order noise can reorder a near-tie
            continue
        checked += 1
        assert list(idx[t]) == list(oi[t]), f"token {t}"
        np.testing.assert_allclose(wts[t], ow[t], rtol=1e-5, atol=1e-7)
        assert list(rs[t]) == [int(slot_of[e]) for e in idx[t]]
    assert checked >= 0.9 * T


@pytest.mark.parametrize("E,k", [(64, 1), (384, 8), (512, 16)])
@pytest.mark.parametrize("T", [1, 40])
def test_router_expert_count_and_top_k_limits(E, k, T):
    """Expert counts up to 512 (eight per lane) and top-k from 1 to 16, on the
    gemv (T=1) and matrix-core (T=40) logits paths; and the decode forward,
    which selects in its own kernel only for E <= 256, agrees with router +
    expert_decode."""
    banner(f"router limits E={E} k={k} T={T}")
    d = 1024
    w, bias = synth.uniform_router(E, d, torch.bfloat16, seed=E + k, bias_std=0.01)
    x = synth.activations(T, d, torch.bfloat16, seed=T + E)
    spec = ops.RouterSpec(w.to(DEV), k, routed_scale=1.5, score_bias=bias.to(DEV))
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    idx, wts, rs = ops.router(spec, x.to(DEV), ops.Workspace(), slot_of_expert=slot_of, n_slots=E + 1)
    torch.cuda.synchronize()
    oi, ow, margin, scores = moe.route(values(x), values(w), k, bias=values(bias), routed_scale=1.5)
    scale = np.abs(scores).max(axis=1) + np.abs(values(bias)).max()
    idx, wts, rs = idx.cpu().numpy(), wts.cpu().numpy(), rs.cpu().numpy()
    checked = 0
    for t in range(T):
        if margin[t] < 1e-4 * scale[t]:
            continue
        checked += 1
        assert list(idx[t]) == list(oi[t]), f"token {t}"
        np.testing.assert_allclose(wts[t], ow[t], rtol=1e-5, atol=1e-7)
        assert list(rs[t]) == [e + 1 for e in idx[t]]
    assert checked >= 0.9 * T
    if T == 1:
        dff = 512
        arena = synth.expert_arena(E + 1, d, dff, seed=E, device=DEV)
        out, fi, fw = ops.forward(spec, arena, None, slot_of, x.to(DEV), ops.Workspace())
        ri, rw, rslot = ops.router(spec, x.to(DEV), ops.Workspace(), slot_of_expert=slot_of, n_slots=E + 1)
        assert torch.equal(fi, ri) and torch.equal(fw, rw)
        assert torch.equal(out, ops.expert_decode(arena, None, x.to(DEV), rslot, rw))


def test_router_hash_mode():
    banner("router hash")
    E, d, k, V, T = 64, 512, 6, 50, 20
    w, _ = synth.uniform_router(E, d, torch.bfloat16, seed=3)
    table = torch.stack([torch.randperm(E, generator=torch.Generator().manual_seed(i))[:k]
                         for i in range(V)]).to(torch.int32)
    ids = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(1))
    x = synth.activations(T, d, torch.bfloat16, seed=4)
    spec = ops.RouterSpec(w.to(DEV), k, routed_scale=1.5, tid2eid=table.to(DEV))
    idx, wts, _ = ops.router(spec, x.to(DEV), ops.Workspace(), input_ids=ids.to(DEV))
    oi, ow, _, _ = moe.route(values(x), values(w), k, routed_scale=1.5, tid2eid=table.numpy(),
                             input_ids=ids.numpy())
    assert np.array_equal(idx.cpu().numpy(), oi)
    np.testing.assert_allclose(wts.cpu().numpy(), ow, rtol=1e-5)


def test_router_precomputed_logits_zipf():
    banner("router logits_in zipf")
    T, E, k = 64, 256, 6
    logits = synth.zipf_logits(T, E, seed=2)
    w = torch.zeros(E, 256, dtype=torch.bfloat16)
    spec = ops.RouterSpec(w.to(DEV), k, routed_scale=1.5)
    idx, wts, _ = ops.router(spec, torch.zeros(T, 256, dtype=torch.bfloat16, device=DEV),
                             ops.Workspace(), logits=logits.to(DEV))
    oi = np.argsort(-logits.numpy(), axis=1, kind="stable")[:, :k]
    assert np.array_equal(idx.cpu().numpy(), oi)


@pytest.mark.parametrize("T", [1, 5, 40])
def test_select_exact_ties(T):
    """Integer logits in [-3, 3] tie often. They reach the router exactly:
    x[:, :E] holds them and the identity router makes x . Wg^T = x[:, :E]
    with one nonzero product per logit. The select kernel and (T <= 8) the
    decode gate/up kernel's own selection must both return the stable
    order -- descending score, ties to the lower expert id -- which is the
    oracle's order."""
    banner(f"select exact ties T={T}")
    d, E, dff, k = 1024, 256, 512, 6
    g = torch.Generator().manual_seed(40 + T)
    x = torch.randn(T, d, generator=g)
    x[:, :E] = torch.randint(-3, 4, (T, E), generator=g).float()
    x = x.to(torch.bfloat16)
    w = synth.identity_router(E, d, torch.bfloat16)
    logits = values(x)[:, :E].astype(np.float64)
    want = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    oi, _, _, _ = moe.route(values(x), values(w), k, routed_scale=1.5)
    assert np.array_equal(oi, want)
    spec = ops.RouterSpec(w.to(DEV), k, routed_scale=1.5)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    xd = x.to(DEV)
    ridx, rw, rs = ops.router(spec, xd, ops.Workspace(), slot_of_expert=slot_of, n_slots=E + 1)
    arena = synth.expert_arena(E + 1, d, dff, dtype=torch.bfloat16, seed=41, device=DEV)
    out, idx, wts = ops.forward(spec, arena, None, slot_of, xd, ops.Workspace())
    torch.cuda.synchronize()
    assert np.array_equal(ridx.cpu().numpy(), want)
    assert np.array_equal(idx.cpu().numpy(), want)
    assert torch.equal(wts, rw)
    assert torch.equal(rs.cpu(), (ridx + 1).cpu())


# ---------------------------------------------------------------------------
# Expert math, decode path
# ---------------------------------------------------------------------------
DECODE_CASES = [
    # (dtype, bits_gu, bits_down, group, d, dff); rows need cols*bits >= 1024
    (torch.bfloat16, 2, 2, 64, 1024, 512),
    (torch.bfloat16, 2, 4, 64, 512, 512),
    (torch.bfloat16, 4, 4, 64, 1024, 512),
    (torch.bfloat16, 2, 2, 128, 1024, 512),
    (torch.bfloat16, 2, 2, 32, 1024, 512),
    (torch.bfloat16, 8, 8, 64, 512, 256),
    (torch.bfloat16, 4, 4, 32, 256, 256),
    (torch.float16, 4, 4, 64, 1024, 512),
    (torch.float16, 2, 2, 64, 1024, 512),
    (torch.float16, 8, 4, 128, 512, 256),
    (torch.bfloat16, 2, 2, 64, 4096, 2048),
    (torch.bfloat16, 2, 4, 64, 4096, 2048),
    (torch.float16, 2, 2, 64, 4096, 2048),
    # groups of 128 (the real checkpoint's 2-bit experts) on the matrix cores
    (torch.bfloat16, 2, 2, 128, 4096, 2048),
    (torch.float16, 2, 2, 128, 4096, 2048),
    (torch.bfloat16, 4, 4, 128, 4096, 2048),
    # 3-bit codes (the DSpark/MTP tier): 4-bit kernels widening 3-bit rows
    # (the matrix-core gate/up for groups of 64 and 128, VALU for 32)
    (torch.bfloat16, 3, 3, 64, 1024, 512),
    (torch.float16, 3, 3, 32, 1024, 512),
    (torch.bfloat16, 2, 3, 64, 1024, 512),
    (torch.bfloat16, 3, 2, 64, 4096, 2048),
    (torch.bfloat16, 3, 3, 64, 4096, 2048),
    (torch.float16, 3, 3, 128, 4096, 2048),
]


@pytest.mark.parametrize("case", DECODE_CASES, ids=lambda c: "-".join(map(str, c)))
@pytest.mark.parametrize("T", [1, 2])
def test_expert_decode_matches_oracle(case, T):
    dtype, bgu, bdn, group, d, dff = case
    banner(f"expert_decode {case} T={T}")
    S, k = 9, 4
    arena = synth.expert_arena(S, d, dff, bits_gate_up=bgu, bits_down=bdn, group=group, dtype=dtype,
                               seed=d + bgu)
    shared = synth.expert_arena(1, d, dff, bits_gate_up=bgu, bits_down=bdn, group=group, dtype=dtype,
                                seed=99, zero_slot=False)
    x = synth.activations(T, d, dtype, seed=T)
    gen = torch.Generator().manual_seed(T + d)
    slots = torch.stack([torch.randperm(S - 1, generator=gen)[:k] + 1 for _ in range(T)]).to(torch.int32)
    wts = torch.rand(T, k, generator=gen) * 1.5
    out = ops.expert_decode(_dev(arena), _dev(shared), x.to(DEV), slots.to(DEV), wts.to(DEV),
                            swiglu_limit=10.0)
    torch.cuda.synchronize()
    slot_of = {s: s for s in range(S)}
    want, terms = _oracle_layer(x, slots.numpy(), wts.numpy(), arena, slot_of, dtype, shared=shared,
                                return_terms=True)
    got = values(out)
    assert_close_terms(got, want, terms, f"decode {case}")
    assert close_fraction(got, want, dtype) > 0.8
    # Pure expert outputs (one route, weight 1, no shared): 1e-2 rel / 2e-3 abs.
    one = ops.expert_decode(_dev(arena), None, x.to(DEV), slots[:, :1].contiguous().to(DEV),
                            torch.ones(T, 1, device=DEV))
    want1 = _oracle_layer(x, slots[:, :1].numpy(), np.ones((T, 1)), arena, slot_of, dtype)
    assert_close(values(one), want1, f"expert output {case}")


STAGE_CASES = [c for c in DECODE_CASES if c[1] == c[2] and c[1] != 8] + [DECODE_CASES[1], DECODE_CASES[11]]


FP32_SUM = 2.0 ** -12     # worst-case relative error of an fp32 sum of up to 4096 terms, (n - 1) 2^-24


@pytest.mark.parametrize("case", STAGE_CASES, ids=lambda c: "-".join(map(str, c)))
def test_expert_decode_stagewise_ulp(case):
    """Each stage of the decode path against the exact (fp64) oracle on the
    GPU's own stage inputs.

    Down projection: y = round(down(h)) from the kernel's own h. The kernel
    sums in fp32, the oracle exactly; the roundings can differ only where the
    exact value lies within the fp32 error of a rounding midpoint, so at least
    99 % of the elements are equal, and every element is within one spacing
    (ulp) plus the fp32 worst case, 2^-12 times the sum of |h_j W_nj|.

    Gate/up + SwiGLU: h from x. gate and up are bounded like y; h = SiLU(min(
    gate, L)) * clip(up) moves by at most 1.1 |up| dgate + |SiLU(gate)| dup
    (|SiLU'| < 1.1) plus its three op roundings. The projections' flips and
    the SiLU's own roundings (the GPU's exp against the oracle's) leave at
    least 97 % of h equal."""
    dtype, bgu, bdn, group, d, dff = case
    banner(f"decode stage-wise ulp {case}")
    S, k, T = 9, 4, 2
    dt = dt_name(dtype)
    limit = 10.0
    arena = synth.expert_arena(S, d, dff, bits_gate_up=bgu, bits_down=bdn, group=group, dtype=dtype,
                               seed=d + 3 * bgu)
    x = synth.activations(T, d, dtype, seed=5)
    gen = torch.Generator().manual_seed(7 + d)
    slots = torch.stack([torch.randperm(S - 1, generator=gen)[:k] + 1 for _ in range(T)]).to(torch.int32)
    dev_arena = _dev(arena)
    h_gpu = np.empty((T * k, dff))
    y1 = np.empty((T * k, d))
    for r in range(T * k):             # each route alone, weight 1: its y rounded once
        hidden = torch.empty(1, dff, dtype=dtype, device=DEV)
        y = ops.expert_decode(dev_arena, None, x[r // k:r // k + 1].to(DEV),
                              slots[r // k, r % k].reshape(1, 1).to(DEV), torch.ones(1, 1, device=DEV),
                              hidden=hidden)
        h_gpu[r], y1[r] = values(hidden)[0], values(y)[0]
    ar = arena_numpy(arena)
    xs = values(x)
    for r in range(T * k):
        s_ = int(slots[r // k, r % k])
        proj = {p: (a[0][s_], a[1][s_], a[2][s_], a[3], a[4]) for p, a in ar.items()}
        dense = {p: np.abs(affine.dequant(*proj[p])) for p in proj}
        xr = xs[r // k]
        up = affine.round_to(affine.qmv(xr, *proj["up_proj"]), dt)
        gate = affine.round_to(affine.qmv(xr, *proj["gate_proj"]), dt)
        h_want = moe.swiglu(gate, up, dt, limit=limit)
        d_up = ulp(up, dtype) + FP32_SUM * (np.abs(xr) @ dense["up_proj"].T)
        d_gate = ulp(gate, dtype) + FP32_SUM * (np.abs(xr) @ dense["gate_proj"].T)
        gc = np.minimum(gate, limit)
        silu = gc / (1.0 + np.exp(-gc))
        h_tol = 1.1 * np.minimum(np.abs(up), limit) * d_gate + np.abs(silu) * d_up + 3 * ulp(h_want, dtype)
        dh = np.abs(h_gpu[r] - h_want)
        assert np.all(dh <= h_tol), f"h route {r}: worst {np.max(dh / h_tol):.3g} of the bound"
        assert np.mean(dh == 0) >= 0.97, f"h route {r}: exact {np.mean(dh == 0):.4f}"
        y_want = affine.round_to(affine.qmv(h_gpu[r], *proj["down_proj"]), dt)
        y_tol = ulp(y_want, dtype) + FP32_SUM * (np.abs(h_gpu[r]) @ dense["down_proj"].T)
        dy = np.abs(y1[r] - y_want)
        assert np.all(dy <= y_tol), f"y route {r}: worst {np.max(dy / y_tol):.3g} of the bound"
        assert np.mean(dy == 0) >= 0.99, f"y route {r}: exact {np.mean(dy == 0):.4f}"
        print(f"route {r}: h exact {np.mean(dh == 0):.4f} worst {np.max(dh / h_tol):.3g} of bound; "
              f"y exact {np.mean(dy == 0):.4f} worst {np.max(dy / y_tol):.3g} of bound")


@pytest.mark.parametrize("fp32_swiglu", [False, True])
def test_expert_decode_swiglu_modes_and_limit(fp32_swiglu):
    banner(f"swiglu fp32={fp32_swiglu}")
    d, dff, S, k = 1024, 512, 5, 2
    arena = synth.expert_arena(S, d, dff, seed=5)
    x = (synth.activations(1, d, seed=3).float() * 4).to(torch.bfloat16)   # drive the clamp
    slots = torch.tensor([[1, 3]], dtype=torch.int32)
    wts = torch.tensor([[0.7, 0.3]])
    for limit in (10.0, 0.5, 0.0):
        out = ops.expert_decode(_dev(arena), None, x.to(DEV), slots.to(DEV), wts.to(DEV),
                                swiglu_limit=limit, fp32_swiglu=fp32_swiglu)
        want, terms = _oracle_layer(x, slots.numpy(), wts.numpy(), arena, {s: s for s in range(S)},
                                    torch.bfloat16, limit=limit, fp32_swiglu=fp32_swiglu,
                                    return_terms=True)
        assert_close_terms(values(out), want, terms, f"limit {limit}")


def test_zero_slot_and_invalid_slots_contribute_zero():
    banner("zero / invalid slots")
    d, dff, S = 1024, 512, 4
    arena = synth.expert_arena(S, d, dff, seed=8)
    x = synth.activations(1, d, seed=1)
    for bad in (0, -1, S, 1000):
        slots = torch.tensor([[bad, bad]], dtype=torch.int32)
        out = ops.expert_decode(_dev(arena), None, x.to(DEV), slots.to(DEV),
                                torch.ones(1, 2, device=DEV))
        assert torch.count_nonzero(out).item() == 0


def test_expert_decode_rejects_bad_shapes():
    banner("shape checks")
    arena = _dev(synth.expert_arena(3, 1024, 512, seed=1))
    x = torch.zeros(1, 512, dtype=torch.float16, device=DEV)      # dtype mismatch
    with pytest.raises(ops._lib.LocaliError):
        ops.expert_decode(arena, None, x, torch.ones(1, 2, dtype=torch.int32, device=DEV),
                          torch.ones(1, 2, device=DEV))
    odd = synth.expert_arena(3, 576, 256, seed=1)                 # 576*2/128 chunks unsupported
    with pytest.raises(ops._lib.LocaliError):
        ops.expert_decode(_dev(odd), None, torch.zeros(1, 576, dtype=torch.bfloat16, device=DEV),
                          torch.ones(1, 2, dtype=torch.int32, device=DEV), torch.ones(1, 2, device=DEV))


def test_empty_batch_is_a_no_op():
    """Zero tokens: every entry point returns at once with empty outputs (the
    reference's layer call on an empty batch returns an empty output), and
    the arena MoE returns an empty tensor of x's shape without routing."""
    from locali_amd.arena import ArenaMoE
    banner("empty batch")
    d, dff, E, k = 1024, 512, 16, 4
    arena = synth.expert_arena(E + 1, d, dff, seed=3, device=DEV)
    shared = synth.expert_arena(1, d, dff, seed=4, device=DEV, zero_slot=False)
    x = torch.zeros(0, d, dtype=torch.bfloat16, device=DEV)
    w, _ = synth.uniform_router(E, d, torch.bfloat16, seed=5, device=DEV)
    spec = ops.RouterSpec(w, k, routed_scale=1.5)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    idx, wts, _ = ops.router(spec, x, ops.Workspace(), slot_of_expert=slot_of, n_slots=E + 1)
    assert tuple(idx.shape) == (0, k) and tuple(wts.shape) == (0, k)
    none_i = torch.zeros(0, k, dtype=torch.int32, device=DEV)
    none_w = torch.zeros(0, k, device=DEV)
    assert tuple(ops.expert_decode(arena, shared, x, none_i, none_w).shape) == (0, d)
    assert tuple(ops.expert_grouped(arena, shared, x, none_i, slot_of, none_w, ops.Workspace(),
                                    n_experts=E).shape) == (0, d)
    out, idx, wts = ops.forward(spec, arena, shared, slot_of, x, ops.Workspace())
    assert tuple(out.shape) == (0, d) and tuple(idx.shape) == (0, k)
    moe_ = ArenaMoE(None, 0, None, None, k)
    y = moe_(torch.zeros(1, 0, d, dtype=torch.bfloat16, device=DEV))
    assert tuple(y.shape) == (1, 0, d) and y.dtype == torch.bfloat16
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# Grouped path, dispatch, combine
# ---------------------------------------------------------------------------
def test_dispatch_stable_sort():
    banner("dispatch")
    T, k, S = 37, 6, 40
    gen = torch.Generator().manual_seed(0)
    rs = torch.stack([torch.randperm(S - 1, generator=gen)[:k] + 1 for _ in range(T)]).to(torch.int32)
    rs[3, 2] = -1
    sorted_route, seg = ops.dispatch(rs.to(DEV), S)
    order, counts, _ = moe.dispatch(rs.numpy())
    flat = rs.numpy().reshape(-1)
    valid = order[flat[order] >= 0]
    n = int(seg[-1].item())
    assert n == valid.size
    assert np.array_equal(sorted_route.cpu().numpy()[:n], valid)
    seg = seg.cpu().numpy()
    for s in range(S):
        assert seg[s + 1] - seg[s] == counts.get(s, 0)


@pytest.mark.parametrize("T", [2, 9, 40])
def test_fp32_combine_mode_in_the_layer_kernels(T):
    """combine_mode 1 (float32 products, the mixed-tier form) through the
    decode kernels' fused combine (T=2) and the grouped path's (T=9, 40),
    with the shared expert added after one rounding."""
    banner(f"fp32 combine T={T}")
    d, dff, E, k = 1024, 512, 16, 4
    arena = synth.expert_arena(E + 1, d, dff, seed=61)
    shared = synth.expert_arena(1, d, dff, seed=62, zero_slot=False)
    x = synth.activations(T, d, seed=63)
    gen = torch.Generator().manual_seed(64)
    idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)]).to(torch.int32)
    slot_of = torch.arange(E, dtype=torch.int32) + 1
    wts = torch.rand(T, k, generator=gen)
    if T <= 2:
        out = ops.expert_decode(_dev(arena), _dev(shared), x.to(DEV), (idx + 1).to(DEV), wts.to(DEV),
                                combine_mode=ops.COMBINE_FP32)
    else:
        out = ops.expert_grouped(_dev(arena), _dev(shared), x.to(DEV), idx.to(DEV), slot_of.to(DEV),
                                 wts.to(DEV), ops.Workspace(), n_experts=E, combine_mode=ops.COMBINE_FP32)
    torch.cuda.synchronize()
    sh = {kk: (v[0][0], v[1][0], v[2][0], v[3], v[4]) for kk, v in arena_numpy(shared).items()}
    want, terms = moe.moe_layer(values(x), idx.numpy(), wts.numpy(), arena_numpy(arena),
                                {e: e + 1 for e in range(E)}, "bf16", limit=10.0, shared=sh,
                                combine_mode="fp32", return_terms=True)
    assert_close_terms(values(out), want, terms, f"fp32 combine T={T}")


@pytest.mark.parametrize("fp32_swiglu", [False, True])
@pytest.mark.parametrize("bits", [(2, 2), (3, 3)])
def test_expert_grouped_swiglu_modes_and_limit(fp32_swiglu, bits):
    """The grouped kernels' SwiGLU epilogues (matrix-core 64-position and
    small tiles for 2-bit, 64-position tiles of every size for 3-bit) with
    the clamp driven (x scaled
    by 4) at limits 10 and 0.5, and with it off (limit 0, unscaled x: with
    no clamp the scaled inputs make h large enough that a last-place flip of
    one h value moves y past the combine-term bound), op by op in the
    activation dtype or in fp32."""
    banner(f"grouped swiglu fp32={fp32_swiglu} bits={bits}")
    d, dff, E, k, T = 1024, 512, 16, 4, 24
    arena = synth.expert_arena(E + 1, d, dff, bits_gate_up=bits[0], bits_down=bits[1], seed=45)
    x1 = synth.activations(T, d, seed=46)
    x4 = (x1.float() * 4).to(torch.bfloat16)
    gen = torch.Generator().manual_seed(47)
    idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)]).to(torch.int32)
    idx[: T // 2, 0] = 3                      # one expert with a 64-position-kernel tile
    slot_of = torch.arange(E, dtype=torch.int32) + 1
    wts = torch.rand(T, k, generator=gen)
    for limit in (10.0, 0.5, 0.0):
        x = x4 if limit > 0 else x1
        out = ops.expert_grouped(_dev(arena), None, x.to(DEV), idx.to(DEV), slot_of.to(DEV), wts.to(DEV),
                                 ops.Workspace(), n_experts=E, swiglu_limit=limit, fp32_swiglu=fp32_swiglu)
        torch.cuda.synchronize()
        want, terms = _oracle_layer(x, idx.numpy(), wts.numpy(), arena, {e: e + 1 for e in range(E)},
                                    torch.bfloat16, limit=limit, fp32_swiglu=fp32_swiglu, return_terms=True)
        assert_close_terms(values(out), want, terms, f"grouped limit {limit}")


@pytest.mark.parametrize("T,dtype,bits", [(3, torch.bfloat16, (2, 2)), (17, torch.bfloat16, (2, 4)),
                                          (64, torch.bfloat16, (2, 2)), (9, torch.float16, (4, 4)),
                                          (5, torch.bfloat16, (3, 3)), (33, torch.float16, (3, 3)),
                                          (9, torch.bfloat16, (2, 3))])
def test_expert_grouped_matches_oracle(T, dtype, bits):
    banner(f"grouped T={T} {dtype} {bits}")
    d, dff, E, k = 1024, 512, 16, 4
    arena = synth.expert_arena(E + 1, d, dff, bits_gate_up=bits[0], bits_down=bits[1], dtype=dtype,
                               seed=T)
    shared = synth.expert_arena(1, d, dff, bits_gate_up=bits[0], bits_down=bits[1], dtype=dtype,
                                seed=77, zero_slot=False)
    x = synth.activations(T, d, dtype, seed=T + 1)
    gen = torch.Generator().manual_seed(T)
    idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)]).to(torch.int32)
    for t in range(0, T, 2):            # skew: expert 0 in every other token
        if not (idx[t] == 0).any():
            idx[t, 0] = 0
    slot_of = (torch.arange(E, dtype=torch.int32) + 1)
    wts = torch.rand(T, k, generator=gen)
    out = ops.expert_grouped(_dev(arena), _dev(shared), x.to(DEV), idx.to(DEV), slot_of.to(DEV),
                             wts.to(DEV), ops.Workspace())
    torch.cuda.synchronize()
    want, terms = _oracle_layer(x, idx.numpy(), wts.numpy(), arena, {e: e + 1 for e in range(E)},
                                dtype, shared=shared, return_terms=True)
    assert_close_terms(values(out), want, terms, "grouped")
    assert close_fraction(values(out), want, dtype) > 0.8


@pytest.mark.parametrize("T,dtype,bits,group,d,dff", [(9, torch.bfloat16, (8, 8), 64, 1024, 512),
                                                      (12, torch.float16, (2, 2), 32, 1024, 512),
                                                      (5, torch.bfloat16, (3, 3), 32, 1024, 512),
                                                      (20, torch.bfloat16, (4, 8), 128, 1024, 512)])
def test_expert_grouped_other_shapes_match_oracle(T, dtype, bits, group, d, dff):
    """The formats the matrix-core grouped kernels do not take (8-bit codes,
    groups of 32) on the VALU grouped kernels, with the shared expert and a
    skewed expert."""
    banner(f"grouped other shapes T={T} {dtype} {bits} g{group} d{d} dff{dff}")
    E, k = 16, 4
    arena = synth.expert_arena(E + 1, d, dff, bits_gate_up=bits[0], bits_down=bits[1], group=group, dtype=dtype,
                               seed=T + 300)
    shared = synth.expert_arena(1, d, dff, bits_gate_up=bits[0], bits_down=bits[1], group=group, dtype=dtype,
                                seed=T + 301, zero_slot=False)
    x = synth.activations(T, d, dtype, seed=T + 302)
    gen = torch.Generator().manual_seed(T + 303)
    idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)]).to(torch.int32)
    idx[: (2 * T) // 3, 0] = 5
    slot_of = (torch.arange(E, dtype=torch.int32) + 1)
    wts = torch.rand(T, k, generator=gen)
    out = ops.expert_grouped(_dev(arena), _dev(shared), x.to(DEV), idx.to(DEV), slot_of.to(DEV),
                             wts.to(DEV), ops.Workspace())
    torch.cuda.synchronize()
    want, terms = _oracle_layer(x, idx.numpy(), wts.numpy(), arena, {e: e + 1 for e in range(E)},
                                dtype, shared=shared, return_terms=True)
    assert_close_terms(values(out), want, terms, "grouped")
    assert close_fraction(values(out), want, dtype) > 0.8


def test_expert_prefill_is_the_grouped_path():
    """locali_moe_expert_prefill (the prefill name of the grouped entry
    point) returns locali_moe_expert_grouped's output bit for bit."""
    import ctypes
    from locali_amd._lib import lib
    banner("expert_prefill == expert_grouped")
    d, dff, E, k, T = 1024, 512, 16, 4, 24
    arena = _dev(synth.expert_arena(E + 1, d, dff, bits_gate_up=2, dtype=torch.bfloat16, seed=5))
    x = synth.activations(T, d, torch.bfloat16, seed=6).to(DEV)
    gen = torch.Generator().manual_seed(7)
    idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)]).to(torch.int32).to(DEV)
    slot_of = (torch.arange(E, dtype=torch.int32) + 1).to(DEV)
    wts = torch.rand(T, k, generator=gen).to(DEV)
    ws = ops.Workspace()
    want = ops.expert_grouped(arena, None, x, idx, slot_of, wts, ws, n_experts=E)
    out = torch.empty_like(x)
    buf = ws.reserve(T, d, dff, E, k, False)
    a = arena.struct()
    rc = lib().locali_moe_expert_prefill(ctypes.byref(a), None, x.data_ptr(), ops.DT_BF16, T, k, E,
                                         idx.data_ptr(), slot_of.data_ptr(), wts.data_ptr(), 10.0, 0,
                                         ops.COMBINE_ROUNDED, out.data_ptr(), buf.data_ptr(), buf.numel(),
                                         torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out, want)


def test_arena_fill_batch_lands_every_byte():
    """Batched fills: pinned, 16-byte aligned pieces through the copy kernel
    (more pieces than one launch takes), plus an odd-sized piece and a
    pageable source through the asynchronous-copy fallback."""
    banner("arena fill batch")
    g = torch.Generator().manual_seed(5)
    sizes = [2 << 20, 256 << 10, 256 << 10, 16, 48 * 1024 + 16] * 14      # 70 pieces
    host = torch.randint(0, 256, (sum(sizes) + 64,), generator=g, dtype=torch.uint8).pin_memory()
    dev = torch.zeros(sum(sizes) + 64, dtype=torch.uint8, device=DEV)
    pieces, off = [], 0
    for n in sizes:
        pieces.append((dev[off:off + n], host[off:off + n]))
        off += n
    odd = (dev[off:off + 37], host[off:off + 37])                           # not a multiple of 16
    pageable = torch.randint(0, 256, (4096,), generator=g, dtype=torch.uint8)
    dev2 = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    ops.arena_fill_batch(pieces + [odd, (dev2, pageable)])
    torch.cuda.synchronize()
    assert torch.equal(dev[:off + 37].cpu(), host[:off + 37])
    assert torch.equal(dev[off + 37:].cpu(), torch.zeros(64 - 37, dtype=torch.uint8))
    assert torch.equal(dev2.cpu(), pageable)


def test_combine_kernel():
    banner("combine")
    T, k, d = 5, 6, 300
    gen = torch.Generator().manual_seed(2)
    y = torch.randn(T, k, d, generator=gen).to(torch.bfloat16)
    sh = torch.randn(T, d, generator=gen).to(torch.bfloat16)
    w = torch.rand(T, k, generator=gen)
    for mode, name in ((ops.COMBINE_ROUNDED, "single"), (ops.COMBINE_FP32, "fp32")):
        out = ops.combine(y.to(DEV), w.to(DEV), sh.to(DEV), mode)
        want = moe.add_shared(moe.combine(values(y), w.numpy(), "bf16", name), values(sh), "bf16")
        assert_close(values(out), want, f"combine {name}", rtol=8e-3, atol=1e-6)
        assert exact_fraction(values(out), want) > 0.99


@pytest.mark.parametrize("ydt", [torch.float32, torch.float16, torch.bfloat16])
def test_combine_routes_gathers_by_position(ydt):
    """locali_moe_combine_routes: route (t, j) reads row route_pos[t, j] of y
    (none when negative), summed in j order, for y rows in fp32 / fp16 / bf16
    and bf16 or fp16 outputs, against the oracle combine of the gathered rows."""
    banner(f"combine_routes y={ydt}")
    T, k, d, n = 6, 5, 260, 23
    gen = torch.Generator().manual_seed(3)
    y = torch.randn(n, d, generator=gen).to(ydt)
    pos = torch.stack([torch.randperm(n, generator=gen)[:k] for _ in range(T)]).to(torch.int32)
    pos[1, 3] = -1
    pos[4, 0] = -1
    w = torch.rand(T, k, generator=gen)
    for out_dt in (torch.bfloat16, torch.float16):
        dt = dt_name(out_dt)
        sh = torch.randn(T, d, generator=gen).to(out_dt)
        gathered = np.where(pos.numpy()[..., None] >= 0, values(y)[np.maximum(pos.numpy(), 0)], 0.0)
        for mode, name in ((ops.COMBINE_ROUNDED, "single"), (ops.COMBINE_FP32, "fp32")):
            out = ops.combine_routes(y.to(DEV), pos.to(DEV), w.to(DEV), out_dt, shared_y=sh.to(DEV), mode=mode)
            want = moe.add_shared(moe.combine(gathered, w.numpy(), dt, name), values(sh), dt)
            assert_close(values(out), want, f"combine_routes {name} {dt}", rtol=8e-3, atol=1e-6)
            assert exact_fraction(values(out), want) > 0.99


# ---------------------------------------------------------------------------
# Whole layer (router + experts + combine + shared) on the benchmark shapes
# ---------------------------------------------------------------------------
def test_forward_small_cpu_config_fp16():
    """d 1024, 32 experts + 1 shared, d_ff 512, 4-bit g64 fp16, decode and 8-token prefill."""
    banner("forward C1")
    d, E, dff, k = 1024, 32, 512, 6
    arena = synth.expert_arena(E + 1, d, dff, bits_gate_up=4, group=64, dtype=torch.float16, seed=1)
    shared = synth.expert_arena(1, d, dff, bits_gate_up=4, dtype=torch.float16, seed=2, zero_slot=False)
    w, bias = synth.uniform_router(E, d, torch.float16, seed=3, bias_std=0.01)
    spec = ops.RouterSpec(w.to(DEV), k, routed_scale=1.5, score_bias=bias.to(DEV))
    slot_of = torch.arange(1, E + 1, dtype=torch.int32)
    for T in (1, 8):
        x = synth.activations(T, d, torch.float16, seed=10 + T)
        out, idx, wts = ops.forward(spec, _dev(arena), _dev(shared), slot_of.to(DEV), x.to(DEV),
                                    ops.Workspace())
        torch.cuda.synchronize()
        oi, ow, margin, _ = moe.route(values(x), values(w), k, bias=values(bias), routed_scale=1.5)
        assert (margin > 1e-4).all()
        assert np.array_equal(idx.cpu().numpy(), oi)
        want, terms = _oracle_layer(x, oi, ow, arena, {e: e + 1 for e in range(E)}, torch.float16,
                                    shared=shared, return_terms=True)
        assert_close_terms(values(out), want, terms, f"forward C1 T={T}")


@pytest.mark.parametrize("mode", ["hash", "sigmoid_bias", "softmax"])
def test_forward_decode_selects_in_gateup(mode):
    """Decode forward selects each token's routes inside the gate/up kernel;
    the result must equal router + expert_decode run separately (same kernels
    and arithmetic: bit-exact), for hash routing, sigmoid scores with a
    selection bias, and softmax scores; and the routes must match the oracle."""
    banner(f"forward decode fused select {mode}")
    d, E, dff, k, T, V = 1024, 64, 512, 6, 2, 40
    arena = synth.expert_arena(E + 1, d, dff, dtype=torch.bfloat16, seed=31, device=DEV)
    shared = synth.expert_arena(1, d, dff, dtype=torch.bfloat16, seed=32, device=DEV, zero_slot=False)
    w, bias = synth.uniform_router(E, d, torch.bfloat16, seed=33, device=DEV, bias_std=0.05)
    kw = dict(routed_scale=1.5)
    ids = None
    if mode == "hash":
        table = torch.stack([torch.randperm(E, generator=torch.Generator().manual_seed(i))[:k]
                             for i in range(V)]).to(torch.int32)
        kw["tid2eid"] = table.to(DEV)
        ids = torch.randint(0, V, (T,), generator=torch.Generator().manual_seed(3)).to(DEV)
    elif mode == "sigmoid_bias":
        kw.update(score_func="sigmoid", score_bias=bias)
    else:
        kw.update(score_func="softmax")
    spec = ops.RouterSpec(w, k, **kw)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    x = synth.activations(T, d, torch.bfloat16, seed=34, device=DEV)
    out, idx, wts = ops.forward(spec, arena, shared, slot_of, x, ops.Workspace(), input_ids=ids)
    ridx, rw, rs = ops.router(spec, x, ops.Workspace(), input_ids=ids, slot_of_expert=slot_of,
                              n_slots=E + 1)
    sep = ops.expert_decode(arena, shared, x, rs, rw)
    torch.cuda.synchronize()
    assert torch.equal(idx, ridx) and torch.equal(wts, rw)
    assert torch.equal(out, sep)
    score = {"hash": "sqrtsoftplus", "sigmoid_bias": "sigmoid", "softmax": "softmax"}[mode]
    oi, ow, margin, _ = moe.route(values(x), values(w), k, routed_scale=1.5, score_func=score,
                                  bias=values(bias) if mode == "sigmoid_bias" else None,
                                  tid2eid=table.numpy() if mode == "hash" else None,
                                  input_ids=ids.cpu().numpy() if mode == "hash" else None)
    for t in range(T):
        if mode == "hash" or margin[t] > 1e-4:
            assert list(idx[t].cpu().numpy()) == list(oi[t])
            np.testing.assert_allclose(wts[t].cpu().numpy(), ow[t], rtol=1e-5)


@pytest.mark.parametrize("T", [1, 2])
def test_decode_forward_in_separate_stages(T):
    """router_logits -> decode_gateup_select -> decode_down_combine are the
    decode forward's own kernels called one at a time: routes, weights and
    output equal locali_moe_forward's bit for bit, and routing on the
    returned logits through the router equals the router's own."""
    banner(f"decode forward stages T={T}")
    d, E, dff, k = 4096, 256, 2048, 6
    arena = synth.expert_arena(E + 1, d, dff, dtype=torch.bfloat16, seed=81, device=DEV)
    shared = synth.expert_arena(1, d, dff, dtype=torch.bfloat16, seed=82, device=DEV, zero_slot=False)
    w, bias = synth.uniform_router(E, d, torch.bfloat16, seed=83, device=DEV, bias_std=0.01)
    spec = ops.RouterSpec(w, k, routed_scale=1.5, score_bias=bias)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    x = synth.activations(T, d, torch.bfloat16, seed=84, device=DEV)
    ref, ridx, rw = ops.forward(spec, arena, shared, slot_of, x, ops.Workspace())
    ws = ops.Workspace()
    logits = ops.router_logits(spec, x)
    hidden = torch.empty(T * (k + 1), dff, dtype=torch.bfloat16, device=DEV)
    idx, wts, rs = ops.decode_gateup_select(spec, arena, shared, slot_of, x, logits, hidden, ws)
    out = torch.empty_like(x)
    ops.decode_down_combine(arena, shared, rs, wts, out, ws)
    li, lw, lrs = ops.router(spec, x, ops.Workspace(), logits=logits, slot_of_expert=slot_of, n_slots=E + 1)
    torch.cuda.synchronize()
    assert torch.equal(idx, ridx) and torch.equal(wts, rw) and torch.equal(out, ref)
    assert torch.equal(li, idx) and torch.equal(lw, wts) and torch.equal(lrs, rs)
    assert torch.equal(rs, idx + 1)


@pytest.mark.parametrize("d,dtype,dff,bits", [(4096, torch.bfloat16, 1024, 2), (2048, torch.float16, 1024, 2),
                                              (1024, torch.bfloat16, 1024, 2), (4096, torch.bfloat16, 2048, 2),
                                              (4096, torch.float16, 2048, 2), (4096, torch.bfloat16, 2048, 3)])
def test_fused_router_rows_across_calls_and_replays(d, dtype, dff, bits):
    """The decode forward computes the logits in router rows of its gate/up
    kernel and hands them over as tagged words. Consecutive calls on one
    workspace alternate between routers and between 1 and 2 tokens, so a call
    that read the previous call's words would route like that call: every
    call must equal the separate logits -> gate/up -> down chain bit for bit,
    eagerly and under repeated graph replays (d_ff 1024 and the benchmarked
    2048; 2-bit codes and the 3-bit MTP tier's)."""
    banner(f"fused router rows d={d} {dt_name(dtype)} dff={dff} bits={bits}")
    E, k = 256, 6
    arena = synth.expert_arena(E + 1, d, dff, bits_gate_up=bits, dtype=dtype, seed=91, device=DEV)
    shared = synth.expert_arena(1, d, dff, bits_gate_up=bits, dtype=dtype, seed=92, device=DEV,
                                zero_slot=False)
    specs = []
    for i in range(3):
        w, bias = synth.uniform_router(E, d, dtype, seed=93 + i, device=DEV, bias_std=0.01)
        specs.append(ops.RouterSpec(w, k, routed_scale=1.5, score_bias=bias))
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    xs = [synth.activations(1 + (i % 2), d, dtype, seed=95 + i, device=DEV) for i in range(6)]
    xs[1] = torch.cat([xs[0], xs[0]])          # same input, next router
    calls = [(specs[i % 3], xs[i]) for i in range(6)]

    def chain(spec, x):
        T = x.shape[0]
        ws = ops.Workspace()
        logits = ops.router_logits(spec, x)
        hidden = torch.empty(T * (k + 1), dff, dtype=dtype, device=DEV)
        idx, wts, rs = ops.decode_gateup_select(spec, arena, shared, slot_of, x, logits, hidden, ws)
        out = torch.empty_like(x)
        ops.decode_down_combine(arena, shared, rs, wts, out, ws)
        return out, idx, wts

    want = [chain(s, x) for s, x in calls]
    ws = ops.Workspace()
    got = [ops.forward(s, arena, shared, slot_of, x, ws) for s, x in calls]
    torch.cuda.synchronize()
    for i, (g, w_) in enumerate(zip(got, want)):
        for a, b in zip(g, w_):
            assert torch.equal(a, b), f"eager call {i}"
    assert not torch.equal(got[0][1][0], got[1][1][0]), "consecutive routers chose alike; the test is blind"
    outs = [torch.empty_like(x) for _, x in calls]
    idxs = [torch.empty(x.shape[0], k, dtype=torch.int32, device=DEV) for _, x in calls]
    wtss = [torch.empty(x.shape[0], k, dtype=torch.float32, device=DEV) for _, x in calls]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i, (s, x) in enumerate(calls):
            ops.forward(s, arena, shared, slot_of, x, ws, out=outs[i], idx=idxs[i], weights=wtss[i])
    for rep in range(3):
        for t in outs + idxs + wtss:
            t.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        for i, w_ in enumerate(want):
            assert torch.equal(outs[i], w_[0]) and torch.equal(idxs[i], w_[1]) and torch.equal(wtss[i], w_[2]), \
                f"replay {rep} call {i}"
        # eager work between replays on the same workspace
        ops.forward(calls[0][0], arena, shared, slot_of, calls[0][1], ws)
        torch.cuda.synchronize()


@pytest.mark.parametrize("group,bits", [(64, 2), (128, 2), (64, 3)])
def test_forward_full_width_decode(oracle_lib, group, bits):
    """d 4096, 256 experts + shared, d_ff 2048, bf16, 2-bit in groups of 64
    and of 128 (the real checkpoint's) and 3-bit in groups of 64 (the MTP
    tier's width), 1 token; checked against the C oracle (fp32) on the GPU's
    own routing."""
    banner(f"forward C2 group {group} bits {bits}")
    d, E, dff, k = 4096, 256, 2048, 6
    arena = synth.expert_arena(E + 1, d, dff, bits_gate_up=bits, group=group, dtype=torch.bfloat16, seed=21,
                               device=DEV)
    shared = synth.expert_arena(1, d, dff, bits_gate_up=bits, group=group, dtype=torch.bfloat16, seed=22,
                                device=DEV, zero_slot=False)
    w, _ = synth.uniform_router(E, d, torch.bfloat16, seed=23, device=DEV)
    spec = ops.RouterSpec(w, k, routed_scale=1.5)
    slot_of = torch.arange(1, E + 1, dtype=torch.int32, device=DEV)
    ws = ops.Workspace()
    for step in range(3):
        x = synth.activations(1, d, torch.bfloat16, seed=100 + step, device=DEV)
        out, idx, wts = ops.forward(spec, arena, shared, slot_of, x, ws)
        torch.cuda.synchronize()
        oi, ow, margin, _ = moe.route(values(x), values(w), k, routed_scale=1.5)
        if margin[0] > 1e-4:
            assert list(idx[0].cpu().numpy()) == list(oi[0])
        slots = (idx.cpu().numpy() + 1).astype(np.int32)
        used = sorted(set(slots.reshape(-1).tolist()))
        remap = {s: i for i, s in enumerate(used)}
        sub = arena_numpy(arena, float_meta=False, slots=used)
        sh = {kk: (v[0], v[1], v[2], v[3], v[4]) for kk, v in arena_numpy(shared, float_meta=False).items()}
        want, terms = oracle_lib.moe_layer(values(x), np.vectorize(remap.get)(slots),
                                           wts.cpu().numpy(), sub, "bf16", shared=sh,
                                           return_terms=True)
        assert_close_terms(values(out), want, terms, f"C2 bits {bits} step {step}")
        assert exact_fraction(values(out), want) > 0.8

