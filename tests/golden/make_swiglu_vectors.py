"""Writes tests/golden/swiglu_vectors.npz from the DeepSeek-V4 expert classes of
the installed `transformers` package (5.15.0, models/deepseek_v4/
modeling_deepseek_v4.py): DeepseekV4Experts._apply_gate (:1014-1021: gate
capped at +limit, up clipped to +-limit, then act(gate) * up with act = SiLU,
config.hidden_act "silu"), DeepseekV4MLP.forward (:977-980, the same clamp
around one dense expert) and DeepseekV4Experts.forward (:997-1012: per routed
expert, gate_up product, the gate above, down product, times the route
weight, summed over routes). This is the in-container restatement of the
expert contract the reference applies (dsv4_arena.py:223-235); it pins the
oracle's clamp placement, SiLU and combine independently of the oracle's own
code.

Inputs are affine-quantised experts (codes, scales, biases, the MLX affine
layout) expanded here to dense matrices w = scale * q + bias in float64 -- the
definition of the format -- and loaded into the transformers modules, which
run in float64 (pure formula, no rounding) and, for the fp32 SwiGLU case, in
float32. Values are chosen so that gate and up cross +-limit often.
"""

from pathlib import Path

import numpy as np
import torch
from transformers.models.deepseek_v4 import modeling_deepseek_v4 as m
from transformers.models.deepseek_v4.configuration_deepseek_v4 import DeepseekV4Config

HERE = Path(__file__).resolve().parent


def _bf16(a: torch.Tensor) -> torch.Tensor:
    return a.to(torch.bfloat16).to(torch.float64)


def _affine(gen, rows, cols, bits, group):
    q = torch.randint(0, 2 ** bits, (rows, cols), generator=gen, dtype=torch.int64)
    s = _bf16(torch.rand(rows, cols // group, generator=gen, dtype=torch.float64) * 0.04 + 0.01)
    b = _bf16(-torch.rand(rows, cols // group, generator=gen, dtype=torch.float64) * 0.1)
    dense = q.double() * s.repeat_interleave(group, 1) + b.repeat_interleave(group, 1)
    return q, s, b, dense


def main():
    gen = torch.Generator().manual_seed(20261202)
    out = {}
    # _apply_gate on pre-activations spanning the clamp, bf16-representable
    gate = _bf16(torch.linspace(-30, 30, 241, dtype=torch.float64))
    up = _bf16(torch.randn(241, generator=gen, dtype=torch.float64) * 15)
    pair = torch.stack([gate, up], dim=-1)            # [241, 2] -> chunk(2) = gate | up
    limits = np.array([10.0, 7.0, 0.5], dtype=np.float64)
    out["gate"], out["up"], out["limits"] = gate.numpy(), up.numpy(), limits
    for i, limit in enumerate(limits):
        cfg = DeepseekV4Config(hidden_size=8, moe_intermediate_size=1, num_local_experts=1,
                               n_routed_experts=1, swiglu_limit=float(limit), hidden_act="silu")
        ex = m.DeepseekV4Experts(cfg)
        with torch.no_grad():
            out[f"h64_{i}"] = ex._apply_gate(pair.clone()).reshape(-1).numpy()
            out[f"h32_{i}"] = ex._apply_gate(pair.float()).reshape(-1).double().numpy()

    # whole experts: d 128, d_ff 64, 4 experts; x scaled so the clamp bites
    for name, (bits, group, limit, xscale) in {"a": (2, 64, 10.0, 24.0), "b": (4, 32, 2.0, 2.0)}.items():
        E, d, dff, T, k = 4, 128, 64, 5, 3
        cfg = DeepseekV4Config(hidden_size=d, moe_intermediate_size=dff, num_local_experts=E,
                               n_routed_experts=E, swiglu_limit=limit, hidden_act="silu")
        ex = m.DeepseekV4Experts(cfg).double()
        mlps = []
        gu = torch.empty(E, 2 * dff, d, dtype=torch.float64)
        dn = torch.empty(E, d, dff, dtype=torch.float64)
        for e in range(E):
            parts = {}
            for proj, (rows, cols) in (("gate_proj", (dff, d)), ("up_proj", (dff, d)), ("down_proj", (d, dff))):
                q, s, b, dense = _affine(gen, rows, cols, bits, group)
                parts[proj] = dense
                out[f"{name}_{proj}_q_{e}"] = q.numpy().astype(np.uint8)
                out[f"{name}_{proj}_s_{e}"] = s.numpy()
                out[f"{name}_{proj}_b_{e}"] = b.numpy()
            gu[e, :dff], gu[e, dff:], dn[e] = parts["gate_proj"], parts["up_proj"], parts["down_proj"]
            mlp = m.DeepseekV4MLP(cfg).double()
            with torch.no_grad():
                mlp.gate_proj.weight.copy_(parts["gate_proj"])
                mlp.up_proj.weight.copy_(parts["up_proj"])
                mlp.down_proj.weight.copy_(parts["down_proj"])
            mlps.append(mlp)
        with torch.no_grad():
            ex.gate_up_proj.copy_(gu)
            ex.down_proj.copy_(dn)
        x = _bf16(torch.randn(T, d, generator=gen, dtype=torch.float64) * xscale)
        idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(T)])
        wts = torch.rand(T, k, generator=gen, dtype=torch.float64) + 0.25
        with torch.no_grad():
            per_expert = torch.stack([mlp(x) for mlp in mlps], dim=1)      # [T, E, d]
            routed = ex(x, idx, wts)
            gate_pre = torch.einsum("td,efd->tef", x, gu[:, :dff])
            up_pre = torch.einsum("td,efd->tef", x, gu[:, dff:])
        out.update({
            f"{name}_meta": np.array([bits, group, E, d, dff, T, k], dtype=np.int64),
            f"{name}_limit": np.float64(limit), f"{name}_x": x.numpy(),
            f"{name}_idx": idx.numpy().astype(np.int32), f"{name}_wts": wts.numpy(),
            f"{name}_mlp": per_expert.numpy(), f"{name}_routed": routed.numpy(),
            # fraction of pre-activations beyond the limit, kept for the test's own check
            f"{name}_clamped": np.float64(((gate_pre > limit).double().mean()
                                           + (up_pre.abs() > limit).double().mean()) / 2),
        })
    np.savez_compressed(HERE / "swiglu_vectors.npz", **out)
    print("wrote", len(out), "arrays")


if __name__ == "__main__":
    main()
