"""Import one MoE layer of a block-FP8 safetensors checkpoint.

The reference validates a checkpoint's tensor headers and its FP8 pairs
(manifest.py:300-374: every ``F8_E4M3`` tensor is a 2-D ``.weight`` with an
FP32 ``.weight_scale_inv`` of shape [ceil(rows/128), ceil(cols/128)]) and
packs a layer's routed experts into the four bank buffers
(packed.py:782-850: gate rows then up rows per expert, scales likewise).
This module does the same from the files themselves: shard headers are
parsed as JSON and tensor bytes are memory-mapped (nothing in a file is
executed), checked, and copied expert by expert into device buffers of the
reference layout, so host memory holds one expert at a time.

Tensor names are found by pattern, whatever their prefix:
``<p>layers.<L>.mlp.experts.<e>.{gate,up,down}_proj.weight`` (+
``_scale_inv``), ``<p>layers.<L>.mlp.shared_experts.{gate,up,down}_proj
.weight``, ``<p>layers.<L>.mlp.gate.weight`` (BF16 or FP32, widened to
FP32 as patch.py:131-142 evaluates it) and
``<p>layers.<L>.mlp.gate.e_score_correction_bias`` (kept in FP32, the cast
of patch.py:296-311).
"""

from __future__ import annotations

import json
import math
import re
import struct
from dataclasses import dataclass
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch

from . import _native as N
from .fp8 import ClampedMLP
from .ownership import TensorLayout, owned_tensor
from .packed import PackedFP8ExpertBank
from .router import Float32Gate

BLOCK = 128
_DTYPE_BYTES = {"F8_E4M3": 1, "U8": 1, "I8": 1, "BOOL": 1, "BF16": 2, "F16": 2, "I16": 2, "F32": 4, "I32": 4,
                "F64": 8, "I64": 8}
_EXPERT_KEY = re.compile(r"^(?P<prefix>.*?)layers\.(?P<layer>\d+)\.mlp\.experts\.(?P<expert>\d+)\."
                         r"(?P<proj>gate|up|down)_proj\.weight$")


class CheckpointError(ValueError):
    """The checkpoint's headers or FP8 pairs fail validation."""


@dataclass(frozen=True)
class TensorHeader:
    shard: str
    dtype: str
    shape: tuple
    start: int  # absolute byte offsets in the shard file
    end: int


def _shard_header(path: Path):
    with path.open("rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise CheckpointError(f"truncated safetensors file: {path.name}")
        (length,) = struct.unpack("<Q", raw)
        if length > path.stat().st_size - 8:
            raise CheckpointError(f"header length exceeds file: {path.name}")
        header = json.loads(f.read(length))
    return header, length, path.stat().st_size


def read_headers(root) -> tuple[dict[str, TensorHeader], list[str]]:
    """Every tensor header of the checkpoint, and the validation failures
    (manifest.py:300-350: known dtype, byte range = shape x dtype size, no
    overlap, shard size = 8 + header + data, index and headers agree)."""
    root = Path(root)
    index_path = root / "model.safetensors.index.json"
    if index_path.is_file():
        weight_map = json.loads(index_path.read_text())["weight_map"]
    elif (root / "model.safetensors").is_file():
        weight_map = None
    else:
        raise CheckpointError(f"no model.safetensors.index.json or model.safetensors in {root}")
    shards = sorted(set(weight_map.values())) if weight_map is not None else ["model.safetensors"]
    tensors: dict[str, TensorHeader] = {}
    failures: list[str] = []
    for shard in shards:
        header, length, size = _shard_header(root / shard)
        base = 8 + length
        ranges, data_end = [], 0
        for key in sorted(k for k in header if k != "__metadata__"):
            meta = header[key]
            try:
                dtype = str(meta["dtype"])
                shape = tuple(int(d) for d in meta["shape"])
                start, end = (int(v) for v in meta["data_offsets"])
            except (KeyError, TypeError, ValueError):
                failures.append(f"malformed tensor header {key} in {shard}")
                continue
            if dtype not in _DTYPE_BYTES:
                failures.append(f"unsupported dtype {dtype} for {key}")
                continue
            if start < 0 or end < start or end - start != math.prod(shape) * _DTYPE_BYTES[dtype]:
                failures.append(f"invalid data range for {key}")
            if key in tensors:
                failures.append(f"duplicate tensor header {key}")
            tensors[key] = TensorHeader(shard, dtype, shape, base + start, base + end)
            ranges.append((start, end, key))
            data_end = max(data_end, end)
        ranges.sort()
        for (_, prev_end, prev_key), (cur_start, _, cur_key) in zip(ranges, ranges[1:]):
            if prev_end > cur_start:
                failures.append(f"overlapping tensors {prev_key} and {cur_key}")
        if base + data_end != size:
            failures.append(f"shard size/header mismatch: {shard}")
    if weight_map is not None:
        mapped, present = set(weight_map), set(tensors)
        if mapped - present:
            failures.append(f"{len(mapped - present)} indexed tensor(s) absent from headers: {min(mapped - present)}")
        if present - mapped:
            failures.append(f"{len(present - mapped)} unindexed tensor(s) in headers: {min(present - mapped)}")
    return tensors, failures


def validate_fp8_pairs(tensors: dict[str, TensorHeader]) -> list[str]:
    """manifest.py:352-374: each F8_E4M3 tensor is a 2-D .weight whose
    .weight_scale_inv is F32 [ceil(rows/128), ceil(cols/128)]."""
    failures = []
    for key, t in tensors.items():
        if t.dtype != "F8_E4M3":
            continue
        if not key.endswith(".weight") or len(t.shape) != 2:
            failures.append(f"unexpected FP8 tensor without 2-D weight semantics: {key}")
            continue
        scale = tensors.get(key + "_scale_inv")
        if scale is None:
            failures.append(f"missing FP8 scale tensor: {key}_scale_inv")
            continue
        want = (math.ceil(t.shape[0] / BLOCK), math.ceil(t.shape[1] / BLOCK))
        if scale.dtype != "F32" or scale.shape != want:
            failures.append(f"invalid FP8 scale {key}_scale_inv: {scale.dtype}{scale.shape}, expected F32{want}")
    return failures


def moe_layer_keys(tensors: dict[str, TensorHeader], layer: int) -> SimpleNamespace:
    """Names of one layer's routed experts (ascending id, 0..E-1), shared
    expert (or None) and router."""
    experts: dict[int, dict[str, str]] = {}
    prefix = None
    for key in tensors:
        m = _EXPERT_KEY.match(key)
        if m is None or int(m["layer"]) != layer:
            continue
        if prefix is not None and m["prefix"] != prefix:
            raise CheckpointError(f"layer {layer} experts under two prefixes: {prefix!r}, {m['prefix']!r}")
        prefix = m["prefix"]
        experts.setdefault(int(m["expert"]), {})[m["proj"]] = key
    if not experts:
        raise CheckpointError(f"no routed experts for layer {layer}")
    ids = sorted(experts)
    if ids != list(range(len(ids))):
        raise CheckpointError(f"layer {layer} expert ids are not 0..{len(ids) - 1}")
    for e in ids:
        if set(experts[e]) != {"gate", "up", "down"}:
            raise CheckpointError(f"layer {layer} expert {e} lacks a projection: has {sorted(experts[e])}")
    mlp = f"{prefix}layers.{layer}.mlp."
    shared = {p: f"{mlp}shared_experts.{p}_proj.weight" for p in ("gate", "up", "down")}
    has_shared = [k in tensors for k in shared.values()]
    if any(has_shared) and not all(has_shared):
        raise CheckpointError(f"layer {layer} shared expert is incomplete")
    router, bias = f"{mlp}gate.weight", f"{mlp}gate.e_score_correction_bias"
    for k in (router, bias):
        if k not in tensors:
            raise CheckpointError(f"missing router tensor {k}")
    return SimpleNamespace(experts=[experts[e] for e in ids], shared=shared if all(has_shared) else None,
                           router=router, bias=bias)


def read_array(root, header: TensorHeader) -> np.ndarray:
    """Read-only memory map of one tensor (FP8 as uint8, BF16 as uint16)."""
    kinds = {"F8_E4M3": np.uint8, "U8": np.uint8, "BF16": np.uint16, "F16": np.float16, "F32": np.float32,
             "I32": np.int32, "I64": np.int64}
    if header.dtype not in kinds:
        raise CheckpointError(f"cannot read dtype {header.dtype}")
    flat = np.memmap(Path(root) / header.shard, dtype=np.uint8, mode="r", offset=header.start,
                     shape=(header.end - header.start,))
    return flat.view(kinds[header.dtype]).reshape(header.shape)


def _float32(root, header: TensorHeader) -> np.ndarray:
    a = read_array(root, header)
    if header.dtype == "BF16":
        return (a.astype(np.uint32) << 16).view(np.float32)
    return np.asarray(a, dtype=np.float32)


def layer_config(root) -> SimpleNamespace:
    """The MoE fields of config.json (text_config when present)."""
    cfg = json.loads((Path(root) / "config.json").read_text())
    text = cfg.get("text_config") or cfg
    return SimpleNamespace(hidden_size=int(text["hidden_size"]), moe_intermediate_size=int(text["moe_intermediate_size"]),
                           swiglu_limit=float(text.get("swiglu_limit", 10.0)),
                           n_routed_experts=int(text["n_routed_experts"]),
                           num_experts_per_tok=int(text["num_experts_per_tok"]),
                           n_shared_experts=int(text.get("n_shared_experts") or 0),
                           routed_scaling_factor=float(text.get("routed_scaling_factor", 1.0)),
                           norm_topk_prob=bool(text.get("norm_topk_prob", True)))


def load_moe_layer(root, layer: int, device, config: SimpleNamespace | None = None):
    """(bank, shared expert or None, gate) of one layer on `device`, after
    header, FP8-pair and shape validation (CheckpointError lists failures)."""
    N.require_device(torch.empty(0, device=device))
    root = Path(root)
    config = config or layer_config(root)
    tensors, failures = read_headers(root)
    keys = moe_layer_keys(tensors, layer)
    named = [k for e in keys.experts for k in e.values()] + (list(keys.shared.values()) if keys.shared else [])
    subset = {k: tensors[k] for k in named}
    subset.update({k + "_scale_inv": tensors[k + "_scale_inv"] for k in named if k + "_scale_inv" in tensors})
    failures = failures + validate_fp8_pairs(subset)
    failures += [f"{k} is {tensors[k].dtype}, expected F8_E4M3" for k in named if tensors[k].dtype != "F8_E4M3"]
    E, H, I = len(keys.experts), config.hidden_size, config.moe_intermediate_size
    if E != config.n_routed_experts:
        failures.append(f"layer {layer} holds {E} experts, config says {config.n_routed_experts}")
    for e, proj in enumerate(keys.experts):
        for p, want in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            if tensors[proj[p]].shape != want:
                failures.append(f"expert {e} {p}_proj is {tensors[proj[p]].shape}, expected {want}")
    if keys.shared is not None:
        Is = tensors[keys.shared["gate"]].shape[0]
        for p, want in (("gate", (Is, H)), ("up", (Is, H)), ("down", (H, Is))):
            if tensors[keys.shared[p]].shape != want:
                failures.append(f"shared {p}_proj is {tensors[keys.shared[p]].shape}, expected {want}")
    if tensors[keys.router].shape != (E, H) or tensors[keys.router].dtype not in ("BF16", "F32"):
        failures.append(f"router weight is {tensors[keys.router].dtype}{tensors[keys.router].shape}, expected "
                        f"BF16/F32{(E, H)}")
    if tensors[keys.bias].shape != (E,) or tensors[keys.bias].dtype not in ("BF16", "F32"):
        failures.append(f"router bias is {tensors[keys.bias].dtype}{tensors[keys.bias].shape}, expected F32{(E,)}")
    if failures:
        raise CheckpointError("; ".join(failures[:8]) + (f" (+{len(failures) - 8} more)" if len(failures) > 8 else ""))
    sr, sh = math.ceil(I / BLOCK), math.ceil(H / BLOCK)
    gate_up = torch.empty((E, 2 * I, H), dtype=torch.uint8, device=device)
    gate_up_s = torch.empty((E, 2 * sr, sh), dtype=torch.float32, device=device)
    down = torch.empty((E, H, I), dtype=torch.uint8, device=device)
    down_s = torch.empty((E, sh, sr), dtype=torch.float32, device=device)

    def put(dst, key):
        dst.copy_(torch.from_numpy(np.array(read_array(root, tensors[key]))))  # a writable host copy

    for e, proj in enumerate(keys.experts):  # packed.py:782-850 order: gate rows, then up rows
        put(gate_up[e, :I], proj["gate"])
        put(gate_up[e, I:], proj["up"])
        put(gate_up_s[e, :sr], proj["gate"] + "_scale_inv")
        put(gate_up_s[e, sr:], proj["up"] + "_scale_inv")
        put(down[e], proj["down"])
        put(down_s[e], proj["down"] + "_scale_inv")
    rm = TensorLayout.ROW_MAJOR_CONTIGUOUS
    bank = PackedFP8ExpertBank(owned_tensor(gate_up, layout=rm), owned_tensor(gate_up_s, layout=rm),
                               owned_tensor(down, layout=rm), owned_tensor(down_s, layout=rm), intermediate_size=I)
    shared = None
    if keys.shared is not None:
        Is = tensors[keys.shared["gate"]].shape[0]
        shared = ClampedMLP(H, Is, config.swiglu_limit, device=device)
        for p in ("gate", "up", "down"):
            lin = getattr(shared, f"{p}_proj")
            put(lin.weight, keys.shared[p])
            put(lin.weight_scale_inv, keys.shared[p] + "_scale_inv")
    weight = torch.from_numpy(np.array(_float32(root, tensors[keys.router]))).to(device)
    bias = torch.from_numpy(np.array(_float32(root, tensors[keys.bias]))).to(device)
    gate = Float32Gate(weight, bias, top_k=config.num_experts_per_tok,
                       routed_scaling_factor=config.routed_scaling_factor, norm_topk_prob=config.norm_topk_prob)
    return bank, shared, gate
