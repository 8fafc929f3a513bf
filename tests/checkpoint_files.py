"""Writes small block-FP8 safetensors checkpoints for the import tests
(safetensors' own writer; FP8 codes stored as F8_E4M3)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np


def _fp8(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).view(torch.float8_e4m3fn)


def _f32(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def _bf16(bits):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(torch.bfloat16)


def layer_tensors(prefix: str, layer: int, gate_up, gate_up_s, down, down_s, shared, router_w, router_b,
                  router_bf16: bool = False) -> dict:
    """Tensor dict of one MoE layer from reference-layout numpy arrays:
    gate_up u8 [E, 2I, H], gate_up_s f32 [E, 2 ceil(I/128), ceil(H/128)],
    down u8 [E, H, I], down_s f32 [E, ceil(H/128), ceil(I/128)]; shared =
    {proj: (weight u8, scale f32)} or None; router_w f32 [E, H] (or BF16
    bits when router_bf16), router_b f32 [E]."""
    out = {}
    E, two_i, _ = gate_up.shape
    inter, sr = two_i // 2, gate_up_s.shape[1] // 2
    mlp = f"{prefix}layers.{layer}.mlp."
    for e in range(E):
        parts = {"gate": (gate_up[e, :inter], gate_up_s[e, :sr]), "up": (gate_up[e, inter:], gate_up_s[e, sr:]),
                 "down": (down[e], down_s[e])}
        for p, (w, s) in parts.items():
            out[f"{mlp}experts.{e}.{p}_proj.weight"] = _fp8(w)
            out[f"{mlp}experts.{e}.{p}_proj.weight_scale_inv"] = _f32(s)
    if shared is not None:
        for p, (w, s) in shared.items():
            out[f"{mlp}shared_experts.{p}_proj.weight"] = _fp8(w)
            out[f"{mlp}shared_experts.{p}_proj.weight_scale_inv"] = _f32(s)
    out[f"{mlp}gate.weight"] = _bf16(router_w) if router_bf16 else _f32(router_w)
    out[f"{mlp}gate.e_score_correction_bias"] = _f32(router_b)
    return out


def write_checkpoint(root, tensors: dict, config: dict, shards: int = 2) -> Path:
    """Sharded checkpoint: model-0000k-of-0000n.safetensors + index + config."""
    from safetensors.torch import save_file

    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    keys = sorted(tensors)
    weight_map = {}
    for i in range(shards):
        name = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        part = {k: tensors[k] for k in keys[i::shards]}
        save_file(part, str(root / name))
        weight_map.update({k: name for k in part})
    (root / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    (root / "config.json").write_text(json.dumps({"model_type": "glm5_next", "text_config": config}))
    return root
