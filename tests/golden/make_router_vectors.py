"""Writes tests/golden/router_vectors.npz from the DeepSeek-V4 router classes of
the installed `transformers` package (5.15.0: DeepseekV4TopKRouter and
DeepseekV4HashRouter, models/deepseek_v4/modeling_deepseek_v4.py:1024-1073,
sqrtsoftplus from activations.py:217-220). This is the in-container
restatement of the gate the reference delegates to (dsv4_arena.py:165-166);
it pins the oracle's router formula (score function, selection-only bias,
renormalisation with 1e-20, routed scaling, hash lookup). fp32 on the CPU.
"""

from pathlib import Path

import numpy as np
import torch
from transformers.models.deepseek_v4 import modeling_deepseek_v4 as m
from transformers.models.deepseek_v4.configuration_deepseek_v4 import DeepseekV4Config

HERE = Path(__file__).resolve().parent


def main():
    torch.manual_seed(1234)
    out = {}
    for name, (E, d, T, k, scale) in {
        "a": (32, 64, 8, 6, 1.5),
        "b": (64, 128, 5, 4, 2.5),
        "c": (256, 256, 3, 6, 1.5),
    }.items():
        cfg = DeepseekV4Config(hidden_size=d, num_local_experts=E, n_routed_experts=E,
                               num_experts_per_tok=k, scoring_func="sqrtsoftplus",
                               routed_scaling_factor=scale, vocab_size=97)
        topk = m.DeepseekV4TopKRouter(cfg).float()
        hashr = m.DeepseekV4HashRouter(cfg).float()
        with torch.no_grad():
            w = torch.randn(E, d) / d ** 0.5
            bias = torch.randn(E) * 0.3
            topk.weight.copy_(w)
            topk.e_score_correction_bias.copy_(bias)
            hashr.weight.copy_(w)
            table = torch.stack([torch.randperm(E)[:k] for _ in range(97)])
            hashr.tid2eid.copy_(table)
            x = torch.randn(T, d)
            ids = torch.randint(0, 97, (T,))
            logits, weights, idx = topk(x)
            hl, hw, hidx = hashr(x, ids)
        out.update({
            f"{name}_x": x.numpy(), f"{name}_w": w.numpy(), f"{name}_bias": bias.numpy(),
            f"{name}_scale": np.float32(scale), f"{name}_k": np.int32(k),
            f"{name}_logits": logits.numpy(), f"{name}_idx": idx.numpy().astype(np.int32),
            f"{name}_weights": weights.numpy(),
            f"{name}_table": table.numpy().astype(np.int32), f"{name}_ids": ids.numpy().astype(np.int32),
            f"{name}_hash_idx": hidx.numpy().astype(np.int32), f"{name}_hash_weights": hw.numpy(),
        })
    np.savez(HERE / "router_vectors.npz", **out)
    print("wrote", sorted(out)[:4], "...")


if __name__ == "__main__":
    main()
