"""Installing the bank-backed MoE modules into a model, layer by layer.

Counterpart of ``install_packed_moe`` / ``install_packed_grouped_moe`` /
``install_packed_decode_moe`` (reference loader.py:167-254).  The model
shape it walks is the reference's (``model.language_model.model.layers``,
each layer with an ``mlp`` and a ``compile_ffn`` flag), and the report keys
are the ones the reference's tests assert (tests/test_fp8_metal.py:274-284,
319-329).

Memory discipline: a layer's separate expert modules are released (and the
caching allocator's blocks returned) before the next layer is packed, so
at most one layer's experts are ever held twice -- at the BASELINE shapes a
layer's bank is 5.4 GB, the whole model 229 GB of the 288 GB of HBM.
"""

from __future__ import annotations

import gc
import logging
from dataclasses import dataclass

import torch

from .fp8 import DirectFP8MoE
from .grouped_fp8 import SortedGroupedFP8MoE
from .packed import PackedFP8ExpertBank, PackedFP8MoE

_log = logging.getLogger(__name__)


@dataclass(frozen=True)
class _Policy:
    """Which module a layer should end up as."""

    target: type
    backend: str
    grouped: bool

    @classmethod
    def of(cls, grouped: bool) -> "_Policy":
        if grouped:
            return cls(SortedGroupedFP8MoE, "packed-grouped", True)
        return cls(PackedFP8MoE, "packed-decode", False)

    def action(self, mlp) -> str:
        """'keep' (already this policy), 'convert' (a Direct layer), 'skip'
        (not a MoE layer this installer handles); raises for a packed layer
        of the other policy, which cannot be re-packed in place."""
        if isinstance(mlp, PackedFP8MoE):
            installed_grouped = isinstance(mlp, SortedGroupedFP8MoE)
            if installed_grouped == self.grouped:
                return "keep"
            raise ValueError(f"cannot convert existing {type(mlp).__name__} to {self.backend} in place")
        return "convert" if isinstance(mlp, DirectFP8MoE) else "skip"


class _DeviceMemory:
    """Allocated-bytes readings of the device holding a layer's experts
    (zeros for a host-resident layer)."""

    def __init__(self, direct: DirectFP8MoE):
        dev = direct.experts[0].gate_proj.weight.device if len(direct.experts) else torch.device("cpu")
        self.device = dev if dev.type == "cuda" else None

    def allocated(self) -> int:
        return int(torch.cuda.memory_allocated(self.device)) if self.device is not None else 0

    def peak(self) -> int:
        return int(torch.cuda.max_memory_allocated(self.device)) if self.device is not None else 0

    def release(self) -> None:
        gc.collect()
        if self.device is not None:
            torch.cuda.synchronize(self.device)
            torch.cuda.empty_cache()


def _swap(index: int, layer, policy: _Policy) -> dict:
    direct = layer.mlp
    memory = _DeviceMemory(direct)
    before = memory.allocated()
    bank = PackedFP8ExpertBank.pack(direct.experts)
    with_bank = memory.allocated()
    layer.mlp = policy.target(bank, direct.config, direct.gate, direct.shared_experts)
    layer.compile_ffn = False
    expert_count = len(direct.experts)
    del direct  # the only remaining reference to the separate experts
    memory.release()
    row = {
        "layer": index,
        "old_expert_count": expert_count,
        "bank_bytes": bank.nbytes,
        "active_before_bytes": before,
        "active_materialized_bytes": with_bank,
        "active_after_clear_bytes": memory.allocated(),
        "peak_bytes": memory.peak(),
        "old_expert_modules_detached": not hasattr(layer.mlp, "experts"),
    }
    _log.info("%s MoE layer=%d bank=%.3f GB active=%.3f GB", policy.backend, index, bank.nbytes / 1e9,
              row["active_after_clear_bytes"] / 1e9)
    return row


def install_packed_moe(model, *, grouped: bool) -> dict:
    """Give every Direct MoE layer a packed bank and the requested execution
    policy; layers already on that policy are left alone.  Returns the
    conversion report, also stored on the model."""
    policy = _Policy.of(grouped)
    layers = model.language_model.model.layers
    rows = [_swap(i, layer, policy) for i, layer in enumerate(layers) if policy.action(layer.mlp) == "convert"]
    still_direct = [i for i, layer in enumerate(layers)
                    if isinstance(layer.mlp, DirectFP8MoE) and not isinstance(layer.mlp, PackedFP8MoE)]
    report = {
        "backend": policy.backend,
        "grouped_enabled": policy.grouped,
        "converted_layers": [row["layer"] for row in rows],
        "converted_count": len(rows),
        "remaining_direct_layers": still_direct,
        "all_old_expert_modules_detached": all(row["old_expert_modules_detached"] for row in rows),
        "layers": rows,
    }
    model._glm53_moe_backend = policy.backend
    setattr(model, "_glm53_" + policy.backend.replace("-", "_") + "_report", report)
    return report


def install_packed_grouped_moe(model) -> dict:
    """Grouped prefill above the route threshold, packed decode below it."""
    return install_packed_moe(model, grouped=True)


def install_packed_decode_moe(model) -> dict:
    """Packed batch-1 decode; prefill keeps the Direct semantics."""
    return install_packed_moe(model, grouped=False)
