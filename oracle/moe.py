"""Streamed-MoE arithmetic restated in numpy -- TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Router      transformers DeepseekV4TopKRouter / HashRouter semantics
            (tf:models/deepseek_v4/modeling_deepseek_v4.py:1024-1073, score
            fn sqrtsoftplus tf:activations.py:217-220) as called through the
            reference gate protocol (dsv4_arena.py:165-166), and Locali's own
            sigmoid router (arena.py:501-506). Logits and scores in fp64.
            Canonical in-row order: descending (score + bias), ties to the
            lower expert id (argpartition order is implementation-defined in
            the reference, arena.py:503).
Expert      dsv4_arena.py:168-235: up/gate projections rounded to the
            activation dtype, clip(up, +-L), min(gate, L) when L > 0, then
            silu(gate) * up op by op in that dtype (silu = gate * sigmoid(gate),
            each op rounded) or in fp32 with one final rounding when
            fp32_swiglu; the down projection rounded again.
Combine     arena.py:543, 619-624, 547: weights cast to the activation dtype,
            product rounded, k-sum accumulated wide and rounded once; the
            mixed-tier form (arena.py:636-672) keeps fp32 products. The caller
            adds the shared expert (dsv4_engine.py:259) with one more rounding.
Dispatch    arena.py:641-659: stable sort of (token, k) entries by slot id,
            inverse permutation to undo it.
Products of dequantised weights are exact fp64 (affine.qmv).
"""

from __future__ import annotations

import numpy as np

from . import affine


# -- router -----------------------------------------------------------------

def _score(logits: np.ndarray, func: str) -> np.ndarray:
    if func == "sqrtsoftplus":
        sp = np.where(logits > 20.0, logits, np.log1p(np.exp(np.minimum(logits, 20.0))))
        return np.sqrt(sp)
    if func == "sigmoid":
        return 1.0 / (1.0 + np.exp(-logits))
    if func == "softmax":
        z = np.exp(logits - logits.max(axis=-1, keepdims=True))
        return z / z.sum(axis=-1, keepdims=True)
    raise ValueError(func)


def route(x, gate_weight, top_k, *, bias=None, score_func="sqrtsoftplus",
          routed_scale=1.0, norm_topk=True, tid2eid=None, input_ids=None):
    """Returns (idx int64 [T,k], weights fp64 [T,k], margin fp64 [T], scores)."""
    x = np.asarray(x, dtype=np.float64).reshape(-1, np.shape(gate_weight)[-1])
    logits = x @ np.asarray(gate_weight, dtype=np.float64).T
    scores = _score(logits, score_func)
    T, E = scores.shape
    if tid2eid is not None:
        idx = np.asarray(tid2eid)[np.asarray(input_ids).reshape(-1)].astype(np.int64)
        margin = np.full(T, np.inf)
    else:
        sel = scores + (0.0 if bias is None else np.asarray(bias, dtype=np.float64))
        order = np.lexsort((np.broadcast_to(np.arange(E), sel.shape), -sel), axis=-1)
        idx = order[:, :top_k]
        srt = np.take_along_axis(sel, order, axis=-1)
        margin = srt[:, top_k - 1] - srt[:, top_k] if top_k < E else np.full(T, np.inf)
    w = np.take_along_axis(scores, idx, axis=-1)
    if norm_topk:
        w = w / (w.sum(axis=-1, keepdims=True) + 1e-20)
    return idx, w * routed_scale, margin, scores


# -- experts ----------------------------------------------------------------

def _sigmoid(v):
    return 1.0 / (1.0 + np.exp(-np.asarray(v, dtype=np.float64)))


def swiglu(gate, up, dtype, limit=10.0, fp32_swiglu=False):
    """gate/up already rounded to dtype -> hidden rounded to dtype."""
    gate = np.asarray(gate, dtype=np.float64)
    up = np.asarray(up, dtype=np.float64)
    if limit > 0:
        up = np.clip(up, -limit, limit)
        gate = np.minimum(gate, limit)
    if fp32_swiglu:
        g32 = gate.astype(np.float32)
        silu = g32 * (1.0 / (1.0 + np.exp(-g32.astype(np.float64)))).astype(np.float32)
        return affine.round_to(silu.astype(np.float64) * up, dtype)
    sig = affine.round_to(_sigmoid(gate), dtype)
    act = affine.round_to(gate * sig, dtype)
    return affine.round_to(act * up, dtype)


def expert(x, proj, dtype, limit=10.0, fp32_swiglu=False):
    """One expert on vectors x [R, d] (values representable in dtype).

    proj: {"gate_proj"|"up_proj"|"down_proj": (w, scales, biases, bits, group)}
    with scales/biases as float arrays. Returns y [R, d] rounded to dtype."""
    def qmm(v, name):
        w, s, b, bits, group = proj[name]
        return affine.round_to(affine.qmv(v, w, s, b, bits, group), dtype)

    up = qmm(x, "up_proj")
    gate = qmm(x, "gate_proj")
    h = swiglu(gate, up, dtype, limit, fp32_swiglu)
    return qmm(h, "down_proj")


def combine(y, weights, dtype, mode="single"):
    """y [T,k,d] rounded to dtype, weights [T,k] (fp32/fp64 router output)."""
    w = affine.round_to(weights, dtype).astype(np.float64)
    if mode == "single":
        prod = affine.round_to(np.asarray(y, dtype=np.float64) * w[..., None], dtype)
        return affine.round_to(prod.astype(np.float64).sum(axis=1), dtype)
    if mode == "fp32":
        prod = (np.asarray(y, dtype=np.float32) * w[..., None].astype(np.float32))
        return affine.round_to(prod.astype(np.float64).sum(axis=1), dtype)
    raise ValueError(mode)


def mixed_tiers(x, tier_of, slot, weights, arenas, order, dtype, *, limit=10.0, fp32_swiglu=False):
    """Routes spanning tiers (arena.py:626-672). tier_of/slot [T, k] place
    route (t, j) in arena arenas[tier_of[t, j]] at slot[t, j]; order is the
    tiers' accumulation order (the store's tier list). Each route's y is the
    expert output rounded to dtype; a float32 accumulator takes the float32
    product y * w, w the weight rounded to dtype (arena.py:543, 661-662),
    tier by tier in `order` and within a tier in row-major (token, k) order
    (arena.py:669-672); the sum is rounded once. Returns (out, terms), terms
    the per-element sum of |y * w|."""
    x = np.asarray(x, dtype=np.float64)
    T, k = np.shape(slot)
    w = affine.round_to(weights, dtype).astype(np.float32)
    out = np.zeros((T, x.shape[-1]), dtype=np.float32)
    terms = np.zeros((T, x.shape[-1]))
    for tier in order:
        arena = arenas[tier]
        for t in range(T):
            for j in range(k):
                if tier_of[t][j] != tier:
                    continue
                s = int(slot[t][j])
                proj = {p: (a[0][s], a[1][s], a[2][s], a[3], a[4]) for p, a in arena.items()}
                y = expert(x[t:t + 1], proj, dtype, limit, fp32_swiglu)[0]
                val = y.astype(np.float32) * w[t, j]
                out[t] = out[t] + val
                terms[t] += np.abs(val.astype(np.float64))
    return affine.round_to(out.astype(np.float64), dtype), terms


def add_shared(routed, shared, dtype):
    return affine.round_to(np.asarray(routed, np.float64) + np.asarray(shared, np.float64), dtype)


# -- dispatch ---------------------------------------------------------------

def dispatch(slots: np.ndarray):
    """slots [T,k] -> (order, counts_by_slot dict, undo) with order a stable
    argsort of the flattened (token, k) entries by slot id."""
    flat = np.asarray(slots).reshape(-1)
    order = np.argsort(flat, kind="stable")
    undo = np.empty_like(order)
    undo[order] = np.arange(order.size)
    uniq, counts = np.unique(flat, return_counts=True)
    return order, dict(zip(uniq.tolist(), counts.tolist())), undo


def first_appearance(idx) -> list[int]:
    """Unique experts of a call in first-appearance order (arena.py:375)."""
    return list(dict.fromkeys(int(e) for e in np.asarray(idx).reshape(-1)))


# -- whole layer ------------------------------------------------------------

def moe_layer(x, idx, weights, arena, slot_of_expert, dtype, *, limit=10.0,
              fp32_swiglu=False, shared=None, combine_mode="single", return_terms=False):
    """Routed MoE over an arena plus optional shared expert.

    arena: {proj: (w[S,...], scales[S,...], biases[S,...], bits, group)}
    slot_of_expert: mapping expert -> slot. Returns out [T, d] rounded, and
    with return_terms the per-element sum of |rounded terms| that were added
    (each term's rounding spacing bounds how far one last-place flip of that
    term moves the output)."""
    x = np.asarray(x, dtype=np.float64)
    T, k = np.shape(idx)
    y = np.zeros((T, k, x.shape[-1]))
    for t in range(T):
        for j in range(k):
            s = slot_of_expert[int(idx[t, j])]
            proj = {p: (a[0][s], a[1][s], a[2][s], a[3], a[4]) for p, a in arena.items()}
            y[t, j] = expert(x[t:t + 1], proj, dtype, limit, fp32_swiglu)[0]
    out = combine(y, weights, dtype, combine_mode)
    wq = affine.round_to(weights, dtype).astype(np.float64)
    terms = np.abs(y * wq[..., None]).sum(axis=1)
    if shared is not None:
        ys = expert(x, shared, dtype, limit, fp32_swiglu)
        out = add_shared(out, ys, dtype)
        terms = terms + np.abs(ys)
    return (out, terms) if return_terms else out
