"""The expert index (locali_amd.index): schema, byte addressing and the DSpark
tier, following the reference's index tests (tests/test_dsv4_index.py:43-117)
on snapshots written here."""

from __future__ import annotations

import json
import struct

import pytest

from checkpoint_fixture import expert_bytes, make_snapshot, write_safetensors
from locali_amd.index import ARRS, PROJS, build_index, extend_with_mtp, main, shard_header

import numpy as np


def _tiny_snapshot(root, layers=2, experts=2):
    """Every array [experts, 1, 1] U32, four bytes per expert."""
    config = {"num_hidden_layers": layers, "n_routed_experts": experts, "num_experts_per_tok": 1,
              "quantization_config": {"bits": 2, "group_size": 128, "mode": "affine"}}
    (root / "config.json").write_text(json.dumps(config))
    shard = "model-00001-of-00001.safetensors"
    tensors, weight_map = {}, {}
    for layer in range(layers):
        for proj in PROJS:
            for arr in ARRS:
                name = f"model.layers.{layer}.ffn.switch_mlp.{proj}.{arr}"
                tensors[name] = (np.arange(experts, dtype=np.uint32).reshape(experts, 1, 1)
                                 + 1000 * layer, "U32")
                weight_map[name] = shard
    write_safetensors(root / shard, tensors)
    (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    return shard


def test_build_index_points_to_each_expert_without_copying(tmp_path):
    _tiny_snapshot(tmp_path)
    index = build_index(tmp_path)
    assert index["format"] == 1
    assert index["layers"] == 2 and index["num_experts"] == 2 and index["top_k"] == 1
    assert index["expert_bytes"] == 2 * 2 * 3 * 3 * 4
    assert index["quantization"]["cold"] == {"bits": 2, "group_size": 128, "mode": "affine"}
    first = index["experts"]["L0.E0"]["gate_proj"]["weight"]
    second = index["experts"]["L0.E1"]["gate_proj"]["weight"]
    assert second[2] == first[2] + first[3]
    assert first[4:] == [[1, 1], "U32"]
    assert first[0] == str(tmp_path.resolve())


def test_index_records_all_nine_arrays_per_expert(tmp_path):
    _tiny_snapshot(tmp_path)
    entry = build_index(tmp_path)["experts"]["L1.E1"]
    assert set(entry) == {"tier", *PROJS}
    assert all(set(entry[p]) == set(ARRS) for p in PROJS)
    assert entry["tier"] == "cold"


def test_records_address_exactly_the_experts_bytes(tmp_path):
    truth = make_snapshot(tmp_path, layers=2, experts=3, d=128, dff=64)
    index = build_index(tmp_path)
    for layer in range(2):
        for e in range(3):
            got = b""
            for p in PROJS:
                for a in ARRS:
                    root, shard, off, n, _, _ = index["experts"][f"L{layer}.E{e}"][p][a]
                    with open(f"{root}/{shard}", "rb") as f:
                        f.seek(off)
                        got += f.read(n)
            assert got == expert_bytes(truth, layer, e)


def test_header_parse_and_bad_header(tmp_path):
    write_safetensors(tmp_path / "a.safetensors", {"t": (np.zeros((2, 3), np.uint32), "U32")})
    table, start = shard_header(tmp_path / "a.safetensors")
    assert table["t"]["shape"] == [2, 3] and start > 8
    (tmp_path / "b.safetensors").write_bytes(b"\x01\x02")
    with pytest.raises(ValueError):
        shard_header(tmp_path / "b.safetensors")


def test_non_affine_and_heterogeneous_quantization_are_rejected(tmp_path):
    _tiny_snapshot(tmp_path)
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg["quantization_config"]["mode"] = "mxfp4"
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="affine"):
        build_index(tmp_path)
    cfg["quantization_config"]["mode"] = "affine"
    cfg["quantization_config"]["model.layers.1.ffn.switch_mlp.down_proj"] = {"bits": 4}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="heterogeneous"):
        build_index(tmp_path)


def test_missing_tensor_and_wrong_expert_axis_are_rejected(tmp_path):
    _tiny_snapshot(tmp_path)
    wm = json.loads((tmp_path / "model.safetensors.index.json").read_text())
    wm["weight_map"].pop("model.layers.1.ffn.switch_mlp.up_proj.biases")
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(wm))
    with pytest.raises(ValueError, match="missing"):
        build_index(tmp_path)
    _tiny_snapshot(tmp_path, experts=3)
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg["n_routed_experts"] = 2
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="first dimension"):
        build_index(tmp_path)


def test_extend_index_adds_three_bit_dspark_tier(tmp_path):
    shard = _tiny_snapshot(tmp_path)
    cfg = json.loads((tmp_path / "config.json").read_text())
    cfg.update(hidden_size=128, moe_intermediate_size=128, dspark_block_size=2,
               dspark_target_layer_ids=[1])
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    table, start = shard_header(tmp_path / shard)
    raw = (tmp_path / shard).read_bytes()[start:]
    tensors = {n: (np.frombuffer(raw[m["data_offsets"][0]:m["data_offsets"][1]], "<u4")
                   .reshape(m["shape"]), "U32") for n, m in table.items()}
    wm = json.loads((tmp_path / "model.safetensors.index.json").read_text())["weight_map"]
    for proj in PROJS:
        for arr in ARRS:
            name = f"mtp.0.ffn.switch_mlp.{proj}.{arr}"
            width = 12 if arr == "weight" else 1        # 12 * 32 / 128 = 3 bits, group 128
            tensors[name] = (np.zeros((2, 1, width), np.uint32), "U32")
            wm[name] = shard
    write_safetensors(tmp_path / shard, tensors)
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    base = build_index(tmp_path)
    index = extend_with_mtp(base, tmp_path)
    assert index["layers"] == 3 and index["main_layers"] == 2 and index["mtp_layers"] == 1
    assert index["quantization"]["hot"] == {"bits": 3, "group_size": 128, "mode": "affine"}
    assert index["experts"]["L2.E1"]["tier"] == "hot"
    assert index["expert_bytes"] == base["expert_bytes"] + 2 * 3 * (12 + 1 + 1) * 4
    assert "L2.E0" not in base["experts"]          # input left untouched


def test_cli_writes_the_index(tmp_path, capsys):
    _tiny_snapshot(tmp_path)
    out = tmp_path / "models" / "x.idx"
    main(["--snapshot", str(tmp_path), "--out", str(out)])
    assert json.loads(out.read_text())["num_experts"] == 2
    assert "0 weight bytes copied" in capsys.readouterr().out
