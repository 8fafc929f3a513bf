"""Checkpoint import, host side: shard headers, FP8-pair validation
(manifest.py:300-374 rules), layer discovery and memory-mapped reads on small
synthetic safetensors checkpoints."""

from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from checkpoint_files import layer_tensors, write_checkpoint
from conftest import submodule

E, H, I = 4, 256, 128
CONFIG = {"hidden_size": H, "moe_intermediate_size": I, "swiglu_limit": 7.0, "n_routed_experts": E,
          "num_experts_per_tok": 2, "n_shared_experts": 1, "routed_scaling_factor": 2.5, "norm_topk_prob": True}


def _layer(rng, prefix="model.language_model.", layer=3, router_bf16=False):
    gu = rng.integers(0, 256, size=(E, 2 * I, H), dtype=np.uint8)
    gus = rng.uniform(size=(E, 2, 2)).astype(np.float32)
    dw = rng.integers(0, 256, size=(E, H, I), dtype=np.uint8)
    dws = rng.uniform(size=(E, 2, 1)).astype(np.float32)
    shared = {"gate": (rng.integers(0, 256, size=(I, H), dtype=np.uint8), rng.uniform(size=(1, 2)).astype(np.float32)),
              "up": (rng.integers(0, 256, size=(I, H), dtype=np.uint8), rng.uniform(size=(1, 2)).astype(np.float32)),
              "down": (rng.integers(0, 256, size=(H, I), dtype=np.uint8), rng.uniform(size=(2, 1)).astype(np.float32))}
    rw = rng.integers(0, 1 << 16, size=(E, H), dtype=np.uint16) if router_bf16 else \
        rng.normal(size=(E, H)).astype(np.float32)
    rb = rng.normal(size=E).astype(np.float32)
    arrays = dict(gate_up=gu, gate_up_s=gus, down=dw, down_s=dws, shared=shared, router_w=rw, router_b=rb)
    return arrays, layer_tensors(prefix, layer, gu, gus, dw, dws, shared, rw, rb, router_bf16=router_bf16)


@pytest.fixture
def C():
    return submodule("checkpoint")


def test_two_layer_checkpoint_reads_back(C, tmp_path):
    rng = np.random.default_rng(1)
    a3, t3 = _layer(rng, layer=3)
    _, t4 = _layer(rng, layer=4)
    root = write_checkpoint(tmp_path / "ck", {**t3, **t4}, CONFIG, shards=3)
    tensors, failures = C.read_headers(root)
    assert failures == [] and C.validate_fp8_pairs(tensors) == []
    keys = C.moe_layer_keys(tensors, 3)
    assert len(keys.experts) == E and keys.shared is not None
    assert keys.router == "model.language_model.layers.3.mlp.gate.weight"
    for e in range(E):
        assert np.array_equal(C.read_array(root, tensors[keys.experts[e]["gate"]]), a3["gate_up"][e, :I])
        assert np.array_equal(C.read_array(root, tensors[keys.experts[e]["up"]]), a3["gate_up"][e, I:])
        assert np.array_equal(C.read_array(root, tensors[keys.experts[e]["down"] + "_scale_inv"]), a3["down_s"][e])
    assert np.array_equal(C.read_array(root, tensors[keys.router]), a3["router_w"])
    cfg = C.layer_config(root)
    assert (cfg.hidden_size, cfg.n_routed_experts, cfg.num_experts_per_tok, cfg.swiglu_limit) == (H, E, 2, 7.0)
    assert cfg.routed_scaling_factor == 2.5 and cfg.norm_topk_prob is True


def test_bf16_router_widens_exactly(C, tmp_path):
    rng = np.random.default_rng(2)
    a, t = _layer(rng, router_bf16=True)
    root = write_checkpoint(tmp_path / "ck", t, CONFIG)
    tensors, _ = C.read_headers(root)
    w = C._float32(root, tensors[C.moe_layer_keys(tensors, 3).router])
    assert np.array_equal(w.view(np.uint32), a["router_w"].astype(np.uint32) << 16)


def test_fp8_pair_rules(C, tmp_path):
    """The failures manifest.py:352-374 names: a missing scale, a scale of
    the wrong shape or dtype, an FP8 tensor that is not a 2-D .weight."""
    rng = np.random.default_rng(3)
    _, t = _layer(rng)
    import torch

    mlp = "model.language_model.layers.3.mlp."
    del t[f"{mlp}experts.1.up_proj.weight_scale_inv"]
    t[f"{mlp}experts.2.down_proj.weight_scale_inv"] = torch.ones((3, 1))
    t[f"{mlp}experts.0.gate_proj.weight_scale_inv"] = torch.ones((1, 2), dtype=torch.float64)
    t[f"{mlp}stray_fp8"] = torch.zeros((4,), dtype=torch.uint8).view(torch.float8_e4m3fn)
    root = write_checkpoint(tmp_path / "ck", t, CONFIG)
    tensors, failures = C.read_headers(root)
    assert failures == []
    got = C.validate_fp8_pairs(tensors)
    assert any("block scales" in f and "are missing" in f and "experts.1.up_proj" in f for f in got)
    assert any("invalid FP8 scale" in f and "experts.2.down_proj" in f and "(2, 1)" in f for f in got)
    assert any("invalid FP8 scale" in f and "experts.0.gate_proj" in f and "F64" in f for f in got)
    assert any("must be a 2-D '.weight'" in f and "stray_fp8" in f for f in got)
    assert len(got) == 4


def test_header_rules(C, tmp_path):
    rng = np.random.default_rng(4)
    _, t = _layer(rng)
    root = write_checkpoint(tmp_path / "ck", t, CONFIG, shards=2)
    shard = sorted(root.glob("*.safetensors"))[0]
    with shard.open("ab") as f:  # trailing byte: data no longer ends the file
        f.write(b"\0")
    index = json.loads((root / "model.safetensors.index.json").read_text())
    index["weight_map"]["model.language_model.layers.3.mlp.not_there"] = shard.name
    (root / "model.safetensors.index.json").write_text(json.dumps(index))
    _, failures = C.read_headers(root)
    assert any("the header accounts for" in f and shard.name in f for f in failures)
    assert any("no shard header holds" in f and "not_there" in f for f in failures)


def test_overlapping_and_bad_ranges(C, tmp_path):
    root = tmp_path / "one"
    root.mkdir()
    header = {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
              "b": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]},
              "c": {"dtype": "BF16", "shape": [3], "data_offsets": [12, 16]}}
    raw = json.dumps(header).encode()
    (root / "model.safetensors").write_bytes(struct.pack("<Q", len(raw)) + raw + bytes(16))
    _, failures = C.read_headers(root)
    assert any("tensors a and b claim overlapping bytes" in f for f in failures)
    assert any(f.startswith("c: data_offsets [12, 16) do not hold the 6 bytes") for f in failures)
    assert len(failures) == 2


def test_layer_discovery_errors(C, tmp_path):
    rng = np.random.default_rng(5)
    _, t = _layer(rng)
    mlp = "model.language_model.layers.3.mlp."
    missing = {k: v for k, v in t.items() if not k.startswith(f"{mlp}experts.2.")}
    root = write_checkpoint(tmp_path / "a", missing, CONFIG)
    tensors, _ = C.read_headers(root)
    with pytest.raises(C.CheckpointError, match="expert ids are not"):
        C.moe_layer_keys(tensors, 3)
    with pytest.raises(C.CheckpointError, match="no routed experts"):
        C.moe_layer_keys(tensors, 7)
    partial = {k: v for k, v in t.items() if k != f"{mlp}shared_experts.up_proj.weight"}
    root = write_checkpoint(tmp_path / "b", partial, CONFIG)
    tensors, _ = C.read_headers(root)
    with pytest.raises(C.CheckpointError, match="shared expert is incomplete"):
        C.moe_layer_keys(tensors, 3)
