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


def layered_zipf_logits(tokens: int, layers: int, n_experts: int, s: float = 1.1, rho: float = 0.6,
                        *, seed: int, device="cpu"):
    """Router logits [tokens, layers, E] for a decode loop over a layer stack:
    layer l ranks the experts by its own seeded permutation with
    p(rank) ~ rank^-s, and adds Gumbel noise whose Gaussian copula is AR(1)
    across layers with coefficient rho (z_l = rho z_{l-1} + sqrt(1-rho^2) n_l,
    g = -log(-log Phi(z))). Each layer's marginal is therefore exactly the
    Zipf sample without replacement of zipf_logits, and a token's noise at
    consecutive layers is correlated."""
    return _layered_zipf(tokens, layers, n_experts, s, rho, seed, device)[0]


def layered_zipf_lookahead(tokens: int, layers: int, n_experts: int, s: float = 1.1, rho: float = 0.6,
                           lookahead_rho: float = 0.9, *, seed: int, device="cpu"):
    """(logits [tokens, layers, E], lookahead [tokens, layers - 1, E]).

    logits are layered_zipf_logits(seed)'s. lookahead[:, l] is a noisy view
    of layer l + 1's logits: the same Zipf ranking with Gumbel noise whose
    Gaussian copula has correlation lookahead_rho with that layer's
    (z' = r z_{l+1} + sqrt(1-r^2) n). It stands for the next layer's gate
    applied to the current hidden state, the input of a cross-layer
    prefetch: r = 1 predicts the next layer's routing exactly."""
    out, base, zs = _layered_zipf(tokens, layers, n_experts, s, rho, seed, device)
    g = _gen(seed + 1_000_003, device)
    ahead = torch.empty(tokens, max(layers - 1, 0), n_experts, dtype=torch.float32, device=device)
    c = math.sqrt(max(0.0, 1.0 - lookahead_rho * lookahead_rho))
    for layer in range(layers - 1):
        z = lookahead_rho * zs[layer + 1] + c * torch.randn(tokens, n_experts, generator=g, device=device,
                                                            dtype=torch.float64)
        u = (0.5 * torch.erfc(-z / math.sqrt(2.0))).clamp(1e-12, 1.0 - 1e-12)
        ahead[:, layer] = (base[layer + 1] - torch.log(-torch.log(u))).float()
    return out, ahead


def _layered_zipf(tokens, layers, n_experts, s, rho, seed, device):
    g = _gen(seed, device)
    logp = -s * torch.log(torch.arange(1, n_experts + 1, device=device, dtype=torch.float64))
    base = torch.empty(layers, n_experts, dtype=torch.float64, device=device)
    for layer in range(layers):
        base[layer, torch.randperm(n_experts, generator=g, device=device)] = logp
    z = torch.randn(tokens, n_experts, generator=g, device=device, dtype=torch.float64)
    out = torch.empty(tokens, layers, n_experts, dtype=torch.float32, device=device)
    c = math.sqrt(1.0 - rho * rho)
    zs = []
    for layer in range(layers):
        if layer:
            z = rho * z + c * torch.randn(tokens, n_experts, generator=g, device=device,
                                          dtype=torch.float64)
        zs.append(z)
        u = (0.5 * torch.erfc(-z / math.sqrt(2.0))).clamp(1e-12, 1.0 - 1e-12)
        out[:, layer] = (base[layer] - torch.log(-torch.log(u))).float()
    return out, base, zs


def identity_router(n_experts: int, d_model: int, dtype=torch.bfloat16, device="cpu"):
    """Wg = [I_E | 0]: x . Wg^T is x[:, :E], so router inputs carry the logits."""
    if d_model < n_experts:
        raise ValueError("identity routing needs d_model >= n_experts")
    w = torch.zeros(n_experts, d_model, dtype=dtype, device=device)
    w[:, :n_experts] = torch.eye(n_experts, dtype=dtype, device=device)
    return w


def stack_index(layers: int, n_experts: int, top_k: int, d_model: int, d_ff: int, *, bits: int = 2,
                bits_down: int | None = None, group: int = 64, meta: str = "BF16") -> dict:
    """Expert index (locali_amd.index schema) of a synthetic layer stack whose
    bytes live in host memory, not in files: records name a shard that is
    never opened, so the store must be given a host_source."""
    bits_down = bits if bits_down is None else bits_down
    msz = 2
    shapes = {"gate_proj": (d_ff, d_model, bits), "up_proj": (d_ff, d_model, bits),
              "down_proj": (d_model, d_ff, bits_down)}
    entry = {"tier": "cold"}
    for proj, (rows, cols, b) in shapes.items():
        words = cols * b // 32
        entry[proj] = {"weight": ["", "host", 0, rows * words * 4, [rows, words], "U32"],
                       "scales": ["", "host", 0, rows * (cols // group) * msz, [rows, cols // group], meta],
                       "biases": ["", "host", 0, rows * (cols // group) * msz, [rows, cols // group], meta]}
    experts = {f"L{layer}.E{e}": entry for layer in range(layers) for e in range(n_experts)}
    total = sum(entry[p][a][3] for p in shapes for a in ("weight", "scales", "biases"))
    return {"format": 1, "model": "synthetic", "snapshot": "", "layers": layers,
            "num_experts": n_experts, "top_k": top_k,
            "quantization": {"cold": {"bits": bits, "group_size": group, "mode": "affine"}},
            "expert_bytes": total * layers * n_experts, "experts": experts}


def host_payloads(arena: ExpertArenaT) -> torch.Tensor:
    """[n_slots, expert bytes] uint8 on the host (pinned when a GPU is present):
    every slot's nine records back to back in (gate, up, down) x (weight,
    scales, biases) order, the host_source layout."""
    projs = (arena.gate, arena.up, arena.down)
    parts = [t.reshape(t.shape[0], -1).view(torch.uint8) for p in projs
             for t in (p.weight, p.scales, p.biases)]
    n, per = parts[0].shape[0], sum(t.shape[1] for t in parts)
    out = torch.empty(n, per, dtype=torch.uint8, pin_memory=torch.cuda.is_available())
    off = 0
    for t in parts:
        out[:, off:off + t.shape[1]].copy_(t)
        off += t.shape[1]
    return out
