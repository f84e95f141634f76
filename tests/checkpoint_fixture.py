"""Synthetic MLX-layout DeepSeek-V4 checkpoints on disk for the index and
arena tests: stacked [E, ...] switch_mlp tensors in safetensors shards (one
shard per layer), config.json and model.safetensors.index.json, plus an
optional expert-major packed file whose nine records per expert are
contiguous (one preadv per expert)."""

from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import torch

from locali_amd import synth
from locali_amd.index import ARRS, PROJS, build_index

NP_DT = {"U32": "<u4", "BF16": "<u2", "F16": "<u2", "I32": "<i4"}


def write_safetensors(path: Path, tensors: dict) -> None:
    """tensors: name -> (numpy array, safetensors dtype name)."""
    header, blobs, off = {}, [], 0
    for name, (arr, dt) in tensors.items():
        raw = np.ascontiguousarray(arr).astype(NP_DT[dt], copy=False).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    head = json.dumps(header).encode()
    Path(path).write_bytes(struct.pack("<Q", len(head)) + head + b"".join(blobs))


def _bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def make_snapshot(root: Path, *, layers=2, experts=6, top_k=2, d=256, dff=128, bits=2, group=64,
                  meta_dtype=torch.bfloat16, seed=0):
    """Writes the snapshot; returns [per-layer ExpertArenaT on the CPU with
    slot e = expert e]."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    dt = "BF16" if meta_dtype == torch.bfloat16 else "F16"
    weight_map, truth = {}, []
    for layer in range(layers):
        arena = synth.expert_arena(experts, d, dff, bits_gate_up=bits, group=group, dtype=meta_dtype,
                                   seed=seed * 100 + layer, zero_slot=False)
        truth.append(arena)
        shard = f"model-{layer + 1:05d}-of-{layers:05d}.safetensors"
        tensors = {}
        for proj, p in zip(PROJS, (arena.gate, arena.up, arena.down)):
            base = f"model.layers.{layer}.ffn.switch_mlp.{proj}"
            tensors[f"{base}.weight"] = (p.weight.numpy().view(np.uint32), "U32")
            tensors[f"{base}.scales"] = (_bits16(p.scales), dt)
            tensors[f"{base}.biases"] = (_bits16(p.biases), dt)
            for arr in ARRS:
                weight_map[f"{base}.{arr}"] = shard
        write_safetensors(root / shard, tensors)
    config = {"num_hidden_layers": layers, "n_routed_experts": experts,
              "num_experts_per_tok": top_k, "hidden_size": d, "moe_intermediate_size": dff,
              "quantization_config": {"bits": bits, "group_size": group, "mode": "affine"}}
    (root / "config.json").write_text(json.dumps(config))
    (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    return truth


def make_index(root: Path, *, packed=False) -> Path:
    """Index of the snapshot at root (build_index); packed=True rewrites every
    expert's nine records contiguously into one expert-major file."""
    index = build_index(root)
    if packed:
        out = root / "experts.pack"
        off = 0
        with out.open("wb") as f:
            for key in sorted(index["experts"], key=lambda k: tuple(int(v[1:]) for v in k.split("."))):
                entry = index["experts"][key]
                for proj in PROJS:
                    for arr in ARRS:
                        r = entry[proj][arr]
                        with open(Path(r[0]) / r[1], "rb") as src:
                            src.seek(r[2])
                            f.write(src.read(r[3]))
                        entry[proj][arr] = [str(root), out.name, off, r[3], r[4], r[5]]
                        off += r[3]
        index["pack"] = {"file": out.name, "order": "expert-major"}
    path = root / ("v4_packed.idx" if packed else "v4.idx")
    path.write_text(json.dumps(index))
    return path


def expert_bytes(truth, layer: int, expert: int) -> bytes:
    """The nine arrays of one expert, in record order, as raw bytes."""
    a = truth[layer]
    out = b""
    for p in (a.gate, a.up, a.down):
        out += p.weight[expert].contiguous().numpy().tobytes()
        out += p.scales[expert].contiguous().view(torch.int16).numpy().tobytes()
        out += p.biases[expert].contiguous().view(torch.int16).numpy().tobytes()
    return out


def add_mtp_stage(root: Path, *, experts, d, dff, bits=3, group=64, seed=0):
    """Appends one embedded DSpark (MTP) stage to the snapshot at root: its
    stacked routed experts as mtp.0.ffn.switch_mlp.* in a shard of their own
    (bits-bit codes, bf16 metadata) and the config fields that declare the
    head. Returns the stage's ExpertArenaT (slot e = expert e)."""
    root = Path(root)
    arena = synth.expert_arena(experts, d, dff, bits_gate_up=bits, group=group, dtype=torch.bfloat16,
                               seed=seed, zero_slot=False)
    shard = "model-mtp.safetensors"
    wm = json.loads((root / "model.safetensors.index.json").read_text())["weight_map"]
    tensors = {}
    for proj, p in zip(PROJS, (arena.gate, arena.up, arena.down)):
        base = f"mtp.0.ffn.switch_mlp.{proj}"
        tensors[f"{base}.weight"] = (p.weight.numpy().view(np.uint32), "U32")
        tensors[f"{base}.scales"] = (_bits16(p.scales), "BF16")
        tensors[f"{base}.biases"] = (_bits16(p.biases), "BF16")
        for arr in ARRS:
            wm[f"{base}.{arr}"] = shard
    write_safetensors(root / shard, tensors)
    (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    cfg = json.loads((root / "config.json").read_text())
    cfg.update(n_mtp_layers=1, dspark_block_size=2, dspark_target_layer_ids=[cfg["num_hidden_layers"] - 1])
    (root / "config.json").write_text(json.dumps(cfg))
    return arena
