"""Seeded synthetic MoE layers for tests and benchmarks.

Arenas follow the reference layout: slot 0 is the reserved all-zero slot
(arena.py:123-126) and expert e of an all-resident layer sits in slot e + 1.
Codes are uniform random; scales/biases are those of a 2^bits-level affine
quantisation of N(0, 1/cols) weights (scale ~ 4.8 sigma / (2^bits - 1),
bias ~ -scale * (2^bits - 1) / 2), so projections of N(0, 1) activations stay
O(1).

Routing inputs:
  uniform  Wg ~ N(0, 1/d): logits of N(0, 1) activations are ~ N(0, 1) and
           every expert is equally likely.
  zipf     Wg = [I_E | 0] and x[:, :E] = log p(rank_e) + Gumbel noise with
           p(rank) ~ rank^-s over a seeded permutation, so x . Wg^T equals
           those logits exactly and the top-k of every token is a Zipf(s)
           sample without replacement (bias 0).
"""

from __future__ import annotations

import math

import torch

from .ops import ExpertArenaT, ProjArena


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def affine_proj(n_slots: int, rows: int, cols: int, bits: int, group: int, dtype, *, seed: int,
                device="cpu", zero_slot: bool = True) -> ProjArena:
    g = _gen(seed, device)
    words = cols * bits // 32
    w = torch.randint(-2**31, 2**31, (n_slots, rows, words), generator=g, device=device,
                      dtype=torch.int64).to(torch.int32)
    levels = (1 << bits) - 1
    sigma = 1.0 / math.sqrt(cols)
    base = 4.8 * sigma / levels
    s = base * (0.8 + 0.4 * torch.rand(n_slots, rows, cols // group, generator=g, device=device))
    b = -s * levels / 2 * (0.9 + 0.2 * torch.rand(n_slots, rows, cols // group, generator=g,
                                                  device=device))
    s, b = s.to(dtype), b.to(dtype)
    if zero_slot:
        w[0].zero_()
        s[0].zero_()
        b[0].zero_()
    return ProjArena(w, s, b, bits, group)


def expert_arena(n_slots: int, d_model: int, d_ff: int, *, bits_gate_up: int = 2,
                 bits_down: int | None = None, group: int = 64, dtype=torch.bfloat16, seed: int = 0,
                 device="cpu", zero_slot: bool = True) -> ExpertArenaT:
    bits_down = bits_gate_up if bits_down is None else bits_down
    return ExpertArenaT(
        gate=affine_proj(n_slots, d_ff, d_model, bits_gate_up, group, dtype, seed=seed * 3 + 1,
                         device=device, zero_slot=zero_slot),
        up=affine_proj(n_slots, d_ff, d_model, bits_gate_up, group, dtype, seed=seed * 3 + 2,
                       device=device, zero_slot=zero_slot),
        down=affine_proj(n_slots, d_model, d_ff, bits_down, group, dtype, seed=seed * 3 + 3,
                         device=device, zero_slot=zero_slot),
    )


def activations(tokens: int, d_model: int, dtype=torch.bfloat16, *, seed: int, device="cpu"):
    g = _gen(seed, device)
    return torch.randn(tokens, d_model, generator=g, device=device).to(dtype)


def uniform_router(n_experts: int, d_model: int, dtype=torch.bfloat16, *, seed: int, device="cpu",
                   bias_std: float = 0.0):
    g = _gen(seed, device)
    w = (torch.randn(n_experts, d_model, generator=g, device=device) / math.sqrt(d_model)).to(dtype)
    bias = None
    if bias_std:
        bias = (torch.randn(n_experts, generator=g, device=device) * bias_std).float()
    return w, bias


def zipf_logits(tokens: int, n_experts: int, s: float = 1.1, *, seed: int, device="cpu"):
    g = _gen(seed, device)
    perm = torch.randperm(n_experts, generator=g, device=device)
    logp = -s * torch.log(torch.arange(1, n_experts + 1, device=device, dtype=torch.float64))
    base = torch.empty(n_experts, dtype=torch.float64, device=device)
    base[perm] = logp
    u = torch.rand(tokens, n_experts, generator=g, device=device, dtype=torch.float64)
    gumbel = -torch.log(-torch.log(u.clamp_min(1e-12)))
    return (base + gumbel).float()


def zipf_router_inputs(tokens: int, n_experts: int, d_model: int, s: float = 1.1,
                       dtype=torch.bfloat16, *, seed: int, device="cpu"):
    """(x [T, d], Wg [E, d]) with x . Wg^T == Zipf-skewed logits exactly."""
    if d_model < n_experts:
        raise ValueError("zipf routing inputs need d_model >= n_experts")
    x = activations(tokens, d_model, dtype, seed=seed + 1, device=device)
    x[:, :n_experts] = zipf_logits(tokens, n_experts, s, seed=seed, device=device).to(dtype)
    w = torch.zeros(n_experts, d_model, dtype=dtype, device=device)
    w[:, :n_experts] = torch.eye(n_experts, dtype=dtype, device=device)
    return x, w
