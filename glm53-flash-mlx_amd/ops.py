"""The path's entry points as torch.library custom ops.

The native library is called through ctypes, which torch.compile cannot
trace: every MoE call would break the graph.  Registered as custom ops
(namespace ``glm53``) with shape functions, each call is one opaque node --
``torch.compile(..., fullgraph=True)`` traces a model through the MoE layers,
and FakeTensor / meta propagation gets the output shapes without a device.

* ``glm53::block_fp8_linear(x, weight, scale_inv, code_flags?)`` -- fp8.py
  ``block_fp8_linear``;
* ``glm53::router_topk(x, weight, bias, top_k, routed_scaling_factor,
  norm_topk_prob, n_group, topk_group)`` -- ``Float32Gate``;
* ``glm53::moe_decode(x, owner, expert_ids?, scores?)`` -- one token through
  a ``PackedFP8MoE`` (router + routed + shared, or caller routing);
* ``glm53::moe_prefill(x, owner, expert_ids?, scores?)`` -- the grouped
  prefill of a ``SortedGroupedFP8MoE``.

The two MoE ops take the module by an integer key (``register_owner``): the
module keeps its weights, its per-(device, stream) native plans and its
cached 0x7F/0xFF code flags, as an ``nn.Module`` does for its parameters,
and the op reads them from there.  Outputs are always new tensors.
"""

from __future__ import annotations

import itertools
import weakref
from typing import Optional

import torch

_OWNERS: dict[int, weakref.ref] = {}
_KEYS = itertools.count(1)


def register_owner(module) -> int:
    """A key under which the MoE ops find `module` (held weakly)."""
    key = next(_KEYS)
    _OWNERS[key] = weakref.ref(module)
    return key


def _owner(key: int):
    ref = _OWNERS.get(int(key))
    module = ref() if ref is not None else None
    if module is None:
        raise RuntimeError(f"MoE module {key} no longer exists")
    return module


@torch.library.custom_op("glm53::block_fp8_linear", mutates_args=())
def block_fp8_linear(x: torch.Tensor, weight: torch.Tensor, scale_inv: torch.Tensor,
                     code_flags: Optional[torch.Tensor]) -> torch.Tensor:
    from .fp8 import native_block_fp8_linear

    return native_block_fp8_linear(x, weight, scale_inv, code_flags)


@block_fp8_linear.register_fake
def _(x, weight, scale_inv, code_flags):
    return x.new_empty((*x.shape[:-1], weight.shape[0]))


@torch.library.custom_op("glm53::router_topk", mutates_args=())
def router_topk(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, top_k: int, routed_scaling_factor: float,
                norm_topk_prob: bool, n_group: int = 1, topk_group: int = 1) -> tuple[torch.Tensor, torch.Tensor]:
    from .router import native_router_topk

    return native_router_topk(x, weight, bias, top_k, routed_scaling_factor, norm_topk_prob, n_group, topk_group)


@router_topk.register_fake
def _(x, weight, bias, top_k, routed_scaling_factor, norm_topk_prob, n_group=1, topk_group=1):
    lead = x.shape[:-1]
    return (x.new_empty((*lead, top_k), dtype=torch.int32), x.new_empty((*lead, top_k), dtype=torch.float32))


@torch.library.custom_op("glm53::moe_decode", mutates_args=())
def moe_decode(x: torch.Tensor, owner: int, expert_ids: Optional[torch.Tensor],
               scores: Optional[torch.Tensor]) -> torch.Tensor:
    return _owner(owner).native_decode(x, expert_ids, scores)


@moe_decode.register_fake
def _(x, owner, expert_ids, scores):
    return torch.empty_like(x)


@torch.library.custom_op("glm53::moe_prefill", mutates_args=())
def moe_prefill(x: torch.Tensor, owner: int, expert_ids: Optional[torch.Tensor],
                scores: Optional[torch.Tensor]) -> torch.Tensor:
    return _owner(owner).native_prefill(x, expert_ids, scores)


@moe_prefill.register_fake
def _(x, owner, expert_ids, scores):
    return torch.empty_like(x)
