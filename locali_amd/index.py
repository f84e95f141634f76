"""Expert index over an MLX DeepSeek-V4 checkpoint (no weight bytes copied).

Same JSON schema as the reference's index (dsv4_index.py:63-143, extended by
:146-249 for the 3-bit DSpark tier), so an index built by either tool drives
either store:

    {"format": 1, "model": ..., "snapshot": <abs path>, "layers": L,
     "num_experts": E, "top_k": k,
     "quantization": {"cold": {"bits", "group_size", "mode"}, ["hot": ...]},
     "expert_bytes": total,
     "experts": {"L<layer>.E<expert>": {"tier": "cold"|"hot",
                 "<proj>": {"<array>": [root, shard, offset, nbytes, shape, dtype]}}}}

Each safetensors tensor is stacked over experts along its first axis and
stored contiguously, so expert e of a tensor is the byte range
[data_start + data_offsets[0] + e * stride, + stride) of its shard: the store
reads it straight into pinned staging with preadv.

    python -m locali_amd.index --snapshot <dir> --out models/dsv4.idx [--mtp]
"""

from __future__ import annotations

import argparse
import json
import struct
from copy import deepcopy
from pathlib import Path

PROJS = ("gate_proj", "up_proj", "down_proj")
ARRS = ("weight", "scales", "biases")
DTSIZE = {"U8": 1, "I8": 1, "F16": 2, "BF16": 2, "U16": 2, "I16": 2, "U32": 4, "I32": 4,
          "F32": 4, "U64": 8, "I64": 8, "F64": 8}


def shard_header(path: Path) -> tuple[dict, int]:
    """(tensor table, byte offset of the data section) of one safetensors file."""
    with Path(path).open("rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ValueError(f"invalid safetensors header: {path}")
        (n,) = struct.unpack("<Q", head)
        table = json.loads(f.read(n))
    table.pop("__metadata__", None)
    return table, 8 + n


def _per_expert(entry: dict, experts: int, name: str) -> tuple[int, list[int], str]:
    shape, dtype = list(entry["shape"]), entry["dtype"]
    if not shape or shape[0] != experts:
        raise ValueError(f"{name}: expected first dimension {experts}, got {shape}")
    if dtype not in DTSIZE:
        raise ValueError(f"{name}: unsupported safetensors dtype {dtype}")
    n = DTSIZE[dtype]
    for dim in shape[1:]:
        n *= dim
    return n, shape[1:], dtype


class _Shards:
    """Lazily parsed headers of a snapshot's shards."""

    def __init__(self, snapshot: Path):
        self.snapshot = snapshot
        self.weight_map = json.loads((snapshot / "model.safetensors.index.json").read_text())[
            "weight_map"]
        self.headers: dict[str, tuple[dict, int]] = {}

    def locate(self, name: str) -> tuple[str, dict, int]:
        try:
            shard = self.weight_map[name]
        except KeyError:
            raise ValueError(f"checkpoint is missing {name}") from None
        if shard not in self.headers:
            self.headers[shard] = shard_header(self.snapshot / shard)
        table, data_start = self.headers[shard]
        return shard, table[name], data_start

    def add_records(self, entries: dict, module: str, layer: int, experts: int, tier: str) -> int:
        """Index the nine arrays of every expert of one switch_mlp module."""
        total = 0
        root = str(self.snapshot)
        for proj in PROJS:
            for arr in ARRS:
                name = f"{module}.{proj}.{arr}"
                shard, entry, data_start = self.locate(name)
                stride, shape, dtype = _per_expert(entry, experts, name)
                base = data_start + entry["data_offsets"][0]
                for e in range(experts):
                    rec = [root, shard, base + e * stride, stride, shape, dtype]
                    entries.setdefault(f"L{layer}.E{e}", {"tier": tier}).setdefault(proj, {})[arr] = rec
                    total += stride
        return total


def build_index(snapshot: Path) -> dict:
    """Index every routed expert of the main layers as tier "cold"
    (reference dsv4_index.py:63-143)."""
    snapshot = Path(snapshot).expanduser().resolve()
    config = json.loads((snapshot / "config.json").read_text())
    layers = int(config["num_hidden_layers"])
    experts = int(config["n_routed_experts"])
    top_k = int(config["num_experts_per_tok"])
    quant = config.get("quantization_config", {})
    bits = int(quant.get("bits", 2))
    group = int(quant.get("group_size", 128))
    mode = quant.get("mode", "affine")
    if mode != "affine":
        raise ValueError(f"the expert arena needs MLX affine experts; checkpoint mode is {mode!r}")
    shards = _Shards(snapshot)
    entries: dict[str, dict] = {}
    total = 0
    for layer in range(layers):
        module = f"model.layers.{layer}.ffn.switch_mlp"
        for proj in PROJS:
            q = quant.get(f"{module}.{proj}", quant)
            got = (int(q.get("bits", bits)), int(q.get("group_size", group)), q.get("mode", mode))
            if got != (bits, group, mode):
                raise ValueError(f"{module}.{proj}: heterogeneous routed-expert quantization "
                                 "is not supported by this arena")
        total += shards.add_records(entries, module, layer, experts, "cold")
    return {
        "format": 1,
        "model": "DeepSeek-V4-Flash-0731",
        "snapshot": str(snapshot),
        "layers": layers,
        "num_experts": experts,
        "top_k": top_k,
        "quantization": {"cold": {"bits": bits, "group_size": group, "mode": mode}},
        "expert_bytes": total,
        "experts": entries,
    }


def extend_with_mtp(index: dict, snapshot: Path) -> dict:
    """Append the embedded DSpark (MTP) experts as logical layers L..L+S-1 of
    tier "hot", inferring their bit width from the packed shapes (reference
    dsv4_index.py:146-249). The input index is not modified."""
    snapshot = Path(snapshot).expanduser().resolve()
    config = json.loads((snapshot / "config.json").read_text())
    stages = int(config.get("n_mtp_layers", 0) or 0) or len(config.get("dspark_target_layer_ids", ()))
    if stages <= 0 or int(config.get("dspark_block_size", 0) or 0) <= 0:
        raise ValueError("checkpoint does not declare an embedded DSpark head")
    out = deepcopy(index)
    main_layers = int(config["num_hidden_layers"])
    if int(out["layers"]) != main_layers:
        raise ValueError(f"base index has {out['layers']} layers, expected {main_layers}")
    experts = int(config["n_routed_experts"])
    if int(out["num_experts"]) != experts:
        raise ValueError("base index expert count does not match checkpoint")
    shards = _Shards(snapshot)
    width_in = {"gate_proj": int(config["hidden_size"]), "up_proj": int(config["hidden_size"]),
                "down_proj": int(config["moe_intermediate_size"])}
    tier_quant = None
    added = 0
    for stage in range(stages):
        module = f"mtp.{stage}.ffn.switch_mlp"
        for proj in PROJS:
            _, w, _ = shards.locate(f"{module}.{proj}.weight")
            _, s, _ = shards.locate(f"{module}.{proj}.scales")
            packed, groups, k = int(w["shape"][-1]), int(s["shape"][-1]), width_in[proj]
            if packed * 32 % k or k % groups:
                raise ValueError(f"cannot infer DSpark quantization for {module}.{proj}")
            q = (packed * 32 // k, k // groups, "affine")
            if tier_quant is None:
                tier_quant = q
            elif q != tier_quant:
                raise ValueError("DSpark routed projections use mixed quantization")
        added += shards.add_records(out["experts"], module, main_layers + stage, experts, "hot")
    out["layers"] = main_layers + stages
    out["main_layers"] = main_layers
    out["mtp_layers"] = stages
    out["quantization"]["hot"] = {"bits": tier_quant[0], "group_size": tier_quant[1],
                                  "mode": tier_quant[2]}
    out["expert_bytes"] = int(out["expert_bytes"]) + added
    return out


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description="Index MLX DeepSeek-V4 routed experts for the HBM arena")
    ap.add_argument("--snapshot", required=True, type=Path)
    ap.add_argument("--out", type=Path, default=Path("models/dsv4.idx"))
    ap.add_argument("--base-index", type=Path, help="extend an existing (possibly packed) index")
    ap.add_argument("--mtp", action="store_true", help="add the DSpark experts as tier 'hot'")
    args = ap.parse_args(argv)
    index = (json.loads(args.base_index.read_text()) if args.base_index
             else build_index(args.snapshot))
    if args.mtp:
        index = extend_with_mtp(index, args.snapshot)
    args.out.parent.mkdir(parents=True, exist_ok=True)
    args.out.write_text(json.dumps(index))
    per = index["expert_bytes"] / (index["layers"] * index["num_experts"])
    print(f"wrote {args.out}: {index['layers']} x {index['num_experts']} experts, "
          f"{index['expert_bytes'] / 1e9:.2f} GB, {per / 1e6:.2f} MB/expert, 0 weight bytes copied")


if __name__ == "__main__":
    main()
