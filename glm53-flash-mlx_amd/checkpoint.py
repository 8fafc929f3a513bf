"""Import one MoE layer of a block-FP8 safetensors checkpoint.

The reference validates a checkpoint's tensor headers and its FP8 pairs
(manifest.py:300-374: every ``F8_E4M3`` tensor is a 2-D ``.weight`` with an
FP32 ``.weight_scale_inv`` of shape [ceil(rows/128), ceil(cols/128)]) and
packs a layer's routed experts into the four bank buffers
(packed.py:782-850: gate rows then up rows per expert, scales likewise).
This module does the same from the files themselves: shard headers are
parsed as JSON and tensor bytes are memory-mapped (nothing in a file is
executed), checked, and copied expert by expert into device buffers of the
reference layout, so host memory holds one expert at a time; the bank is
then re-laid on the device when another layout is asked for.

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
from .packed import DEFAULT_LAYOUT, PackedFP8ExpertBank
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


def _shard_list(root: Path) -> tuple[dict[str, str] | None, list[str]]:
    """The index's weight map (None for a single-file checkpoint) and the
    shard files to read."""
    index_path = root / "model.safetensors.index.json"
    if index_path.is_file():
        weight_map = json.loads(index_path.read_text())["weight_map"]
        return weight_map, sorted(set(weight_map.values()))
    if (root / "model.safetensors").is_file():
        return None, ["model.safetensors"]
    raise CheckpointError(f"{root} holds neither model.safetensors.index.json nor model.safetensors")


def _decode_entry(shard: str, key: str, meta, base: int) -> tuple[TensorHeader | None, list[str]]:
    """One JSON header entry as a TensorHeader (absolute offsets), or None
    and why it cannot be used."""
    try:
        dtype, shape = str(meta["dtype"]), tuple(int(d) for d in meta["shape"])
        lo, hi = (int(v) for v in meta["data_offsets"])
    except (KeyError, TypeError, ValueError):
        return None, [f"{shard}: header entry {key} has no usable dtype / shape / data_offsets"]
    if dtype not in _DTYPE_BYTES:
        return None, [f"{key}: dtype {dtype} is not one this loader reads"]
    need = math.prod(shape) * _DTYPE_BYTES[dtype]
    problems = [] if 0 <= lo <= hi and hi - lo == need else [
        f"{key}: data_offsets [{lo}, {hi}) do not hold the {need} bytes of {dtype}{list(shape)}"]
    return TensorHeader(shard, dtype, shape, base + lo, base + hi), problems


def _byte_accounting(shard: str, entries: list[TensorHeader], names: list[str], data_start: int,
                     file_size: int) -> list[str]:
    """Tensors of one shard must not share bytes, and the data section must
    end where the file does."""
    problems = []
    order = sorted(range(len(entries)), key=lambda i: (entries[i].start, entries[i].end))
    reach, holder = data_start, None  # end of the bytes claimed so far, and who claimed the last of them
    for i in order:
        if entries[i].start < reach and holder is not None:
            problems.append(f"{shard}: tensors {names[holder]} and {names[i]} claim overlapping bytes")
        if entries[i].end >= reach:
            reach, holder = entries[i].end, i
    if reach != file_size:
        problems.append(f"{shard}: the header accounts for {reach} bytes but the file has {file_size}")
    return problems


def read_headers(root) -> tuple[dict[str, TensorHeader], list[str]]:
    """Every tensor header of the checkpoint, and what is wrong with them:
    the rules of the reference's header audit (manifest.py:300-350) -- a
    known dtype, a byte range of exactly shape x element size, no two
    tensors sharing bytes, a shard's data ending at its file's end, and
    the index naming exactly the tensors the shards hold."""
    root = Path(root)
    weight_map, shards = _shard_list(root)
    tensors: dict[str, TensorHeader] = {}
    problems: list[str] = []
    for shard in shards:
        header, length, size = _shard_header(root / shard)
        names = sorted(k for k in header if k != "__metadata__")
        kept, kept_names = [], []
        for key in names:
            entry, why = _decode_entry(shard, key, header[key], 8 + length)
            problems += why
            if entry is None:
                continue
            if key in tensors:
                problems.append(f"{key}: declared in two headers ({tensors[key].shard}, {shard})")
            tensors[key] = entry
            kept.append(entry)
            kept_names.append(key)
        problems += _byte_accounting(shard, kept, kept_names, 8 + length, size)
    if weight_map is not None:
        for label, names in (("the index names {} tensor(s) no shard header holds", set(weight_map) - set(tensors)),
                             ("shard headers hold {} tensor(s) the index does not name", set(tensors) - set(weight_map))):
            if names:
                problems.append(label.format(len(names)) + f", first {min(names)}")
    return tensors, problems


def validate_fp8_pairs(tensors: dict[str, TensorHeader]) -> list[str]:
    """The FP8 pair rule of the reference's audit (manifest.py:352-374):
    each F8_E4M3 tensor is a 2-D ``.weight`` with an F32 ``.weight_scale_inv``
    of shape [ceil(rows/128), ceil(cols/128)].  The wrong-scale message keeps
    the reference's wording, which its test asserts
    (tests/test_manifest.py:230-244)."""
    problems = []
    for key in (k for k, t in tensors.items() if t.dtype == "F8_E4M3"):
        shape = tensors[key].shape
        if len(shape) != 2 or not key.endswith(".weight"):
            problems.append(f"{key}: an F8_E4M3 tensor must be a 2-D '.weight', got shape {list(shape)}")
            continue
        scale_key = key + "_scale_inv"
        scale = tensors.get(scale_key)
        want = (math.ceil(shape[0] / BLOCK), math.ceil(shape[1] / BLOCK))
        if scale is None:
            problems.append(f"{key}: its block scales {scale_key} are missing")
        elif (scale.dtype, scale.shape) != ("F32", want):
            problems.append(f"invalid FP8 scale {scale_key}: {scale.dtype}{scale.shape}, expected F32{want}")
    return problems


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
                           norm_topk_prob=bool(text.get("norm_topk_prob", True)),
                           n_group=int(text.get("n_group") or 1), topk_group=int(text.get("topk_group") or 1))


def load_moe_layer(root, layer: int, device, config: SimpleNamespace | None = None, *, layout=None):
    """(bank, shared expert or None, gate) of one layer on `device`, after
    header, FP8-pair and shape validation (CheckpointError lists failures).
    The bank is re-laid into `layout` (the package's DEFAULT_LAYOUT when
    None; "rows" keeps the checkpoint's row-major layout) once its bytes are
    on the device."""
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
    layout = DEFAULT_LAYOUT if layout is None else layout
    if layout != "rows" and H % BLOCK == 0 and I % BLOCK == 0:
        bank.relayout_(layout)
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
                       routed_scaling_factor=config.routed_scaling_factor, norm_topk_prob=config.norm_topk_prob,
                       n_group=int(getattr(config, "n_group", 1) or 1),
                       topk_group=int(getattr(config, "topk_group", 1) or 1))
    return bank, shared, gate
