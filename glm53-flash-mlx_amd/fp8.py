"""Block-FP8 (E4M3, 128x128 FP32 scales) operators on MI355X.

Drop-in counterparts of the reference's glm53_flash_mlx/fp8.py:
``block_fp8_linear`` (fp8.py:254-299), ``BlockFP8Linear`` (302-326),
``DirectFP8Expert`` (329-340), ``DirectFP8MoE`` (343-400), plus the
shared-expert ``ClampedMLP`` of patch.py:114-129.  Weights stay uint8 E4M3
[out, in] with ``weight_scale_inv`` FP32 [ceil(out/128), ceil(in/128)]; they
are decoded only in registers by the HIP kernels of libglm53_moe.so.
Activations are BF16.
"""

from __future__ import annotations

import math

import torch

from . import _native as N
from . import ops as _ops  # noqa: F401  (registers the glm53 custom ops)

BLOCK_SIZE = 128
DECODE_TOP_K = 8
PREFILL_TILE_ROWS = 8


def _scale_shape(out_features: int, in_features: int) -> tuple[int, int]:
    return (math.ceil(out_features / BLOCK_SIZE), math.ceil(in_features / BLOCK_SIZE))


def block_fp8_linear(x: torch.Tensor, weight: torch.Tensor, scale_inv: torch.Tensor,
                     code_flags: torch.Tensor | None = None) -> torch.Tensor:
    """Compute ``x @ dequant(weight, scale_inv).T`` without expanding weight.

    code_flags: optional device int32 from a scan of `weight` for the E4M3
    codes 0x7F / 0xFF (``_native.scan_codes``); when given and clear, the
    kernels use the hardware E4M3 decode."""
    N.require_device(x, weight, scale_inv)
    if weight.dtype != torch.uint8 or weight.dim() != 2:
        raise ValueError(f"expected 2-D uint8 E4M3 weight, got {tuple(weight.shape)} {weight.dtype}")
    if scale_inv.dtype != torch.float32 or scale_inv.dim() != 2:
        raise ValueError("weight_scale_inv must be a 2-D float32 block table")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"activations must be bfloat16, got {x.dtype}")
    out_features, in_features = weight.shape
    if x.shape[-1] != in_features:
        raise ValueError(f"input width {x.shape[-1]} != weight width {in_features}")
    expected = _scale_shape(out_features, in_features)
    if tuple(scale_inv.shape) != expected:
        raise ValueError(f"scale shape {tuple(scale_inv.shape)} != block128 shape {expected}")
    return torch.ops.glm53.block_fp8_linear(x, weight, scale_inv, code_flags)


def native_block_fp8_linear(x, weight, scale_inv, code_flags):
    """The native call behind the glm53::block_fp8_linear op (arguments
    validated by ``block_fp8_linear``)."""
    out_features, in_features = weight.shape
    flat = x.reshape(-1, in_features).contiguous()
    weight = weight.contiguous()
    scale_inv = scale_inv.contiguous()
    rows = flat.shape[0]
    y = torch.empty((rows, out_features), dtype=torch.bfloat16, device=x.device)
    lib = N.lib()
    ws_bytes = lib.glm53_fp8_linear_workspace_bytes(rows, out_features, in_features)
    ws = N.workspace(ws_bytes, x.device)
    N.check(lib.glm53_fp8_linear(N.ptr(flat), rows, in_features, N.ptr(weight), out_features, N.ptr(scale_inv),
                                 N.ptr(code_flags), N.ptr(y), N.ptr(ws), ws_bytes, N.stream_handle(x.device)))
    return y.reshape(*x.shape[:-1], out_features)


def swiglu(gate: torch.Tensor, up: torch.Tensor, limit: float) -> torch.Tensor:
    """silu(min(gate, L)) * clip(up, -L, L) with MLX's BF16 rounding sequence
    (patch.py:104-112; packed.py:146-163)."""
    N.require_device(gate, up)
    if gate.shape != up.shape or gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise ValueError("gate and up must be bfloat16 tensors of one shape")
    width = gate.shape[-1]
    joined = torch.cat([gate.reshape(-1, width), up.reshape(-1, width)], dim=1).contiguous()
    out = torch.empty((joined.shape[0], width), dtype=torch.bfloat16, device=gate.device)
    lib = N.lib()
    N.check(lib.glm53_activate_gate_up(N.ptr(joined), joined.shape[0], width, float(limit), N.ptr(out),
                                       N.stream_handle(gate.device)))
    return out.reshape(gate.shape)


class BlockFP8Linear(torch.nn.Module):
    """``nn.Linear`` ABI backed by canonical block-128 E4M3 tensors."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False, device=None):
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.register_buffer("weight", torch.zeros((out_features, in_features), dtype=torch.uint8, device=device))
        self.register_buffer("weight_scale_inv",
                             torch.ones(_scale_shape(out_features, in_features), dtype=torch.float32, device=device))
        self.bias = torch.zeros((out_features,), dtype=torch.float32, device=device) if bias else None

    @classmethod
    def from_linear(cls, linear) -> "BlockFP8Linear":
        out_features, in_features = linear.weight.shape
        return cls(in_features, out_features, bias=getattr(linear, "bias", None) is not None)

    def code_flags(self) -> torch.Tensor:
        """Cached device flag of the weight's 0x7F/0xFF codes (rescanned when
        the weight tensor is replaced or modified in place)."""
        stamp = (self.weight.data_ptr(), self.weight._version)
        cached = getattr(self, "_code_flags", None)
        if cached is None or cached[0] != stamp:
            self._code_flags = (stamp, N.scan_codes(self.weight))
        return self._code_flags[1]

    def as_c_struct(self) -> N.Linear:
        return N.Linear(self.weight.data_ptr(), self.weight_scale_inv.data_ptr(), self.out_features, self.in_features,
                        self.code_flags().data_ptr())

    def forward(self, x):
        y = block_fp8_linear(x, self.weight, self.weight_scale_inv, self.code_flags())
        return y + self.bias if self.bias is not None else y


class ClampedMLP(torch.nn.Module):
    """Shared expert: down(silu(min(gate(x), L)) * clip(up(x), L)) (patch.py:114-129)."""

    def __init__(self, hidden_size: int, intermediate_size: int, limit: float, device=None):
        super().__init__()
        self.gate_proj = BlockFP8Linear(hidden_size, intermediate_size, device=device)
        self.up_proj = BlockFP8Linear(hidden_size, intermediate_size, device=device)
        self.down_proj = BlockFP8Linear(intermediate_size, hidden_size, device=device)
        self.limit = float(limit)

    def as_c_struct(self) -> N.SharedExpert:
        return N.SharedExpert(self.gate_proj.as_c_struct(), self.up_proj.as_c_struct(), self.down_proj.as_c_struct())

    def forward(self, x):
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x), self.limit))


class DirectFP8Expert(torch.nn.Module):
    def __init__(self, hidden_size: int, intermediate_size: int, limit: float, device=None):
        super().__init__()
        self.gate_proj = BlockFP8Linear(hidden_size, intermediate_size, device=device)
        self.up_proj = BlockFP8Linear(hidden_size, intermediate_size, device=device)
        self.down_proj = BlockFP8Linear(intermediate_size, hidden_size, device=device)
        self.limit = float(limit)

    def forward(self, x):
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x), self.limit))


def _restore_and_reduce_rows(route_out: torch.Tensor, scores: torch.Tensor, tokens: int, top_k: int,
                             shared: torch.Tensor | None, direct_ids: torch.Tensor | None) -> torch.Tensor:
    """Combine per-route outputs laid out in flat route order (token-major).

    direct_ids None: FP32 slot-order weighted sum (packed.py:168-179);
    otherwise the Direct ascending-expert BF16 accumulation (fp8.py:384-397).
    """
    hidden = route_out.shape[-1]
    dev = route_out.device
    inverse = torch.arange(tokens * top_k, dtype=torch.int32, device=dev)
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=dev)
    scores = scores.reshape(-1).to(torch.float32).contiguous()
    lib = N.lib()
    if direct_ids is None:
        N.check(lib.glm53_restore_and_reduce(N.ptr(route_out), N.ptr(scores), N.ptr(inverse), tokens, top_k, hidden,
                                             N.ptr(shared), N.ptr(out), N.stream_handle(dev)))
    else:
        ids = direct_ids.reshape(-1).to(torch.int32).contiguous()
        N.check(lib.glm53_direct_order_reduce(N.ptr(route_out), N.ptr(inverse), N.ptr(ids), N.ptr(scores), tokens,
                                              top_k, hidden, N.ptr(shared), N.ptr(out), N.stream_handle(dev)))
    return out


def _bucket_forward(expert, rows: torch.Tensor) -> torch.Tensor:
    """One expert over a prefill bucket of token rows on the FP8 MFMA
    contraction tree, whatever the bucket size: a one-row bucket runs as a
    two-row problem (its row twice; rows never mix), so every route of a
    prefill -- here and in the grouped plan -- takes the same per-row
    arithmetic and the Direct-order grouped prefill equals this loop bit
    for bit."""
    n = rows.shape[0]
    x = rows if n > 1 else rows.expand(2, rows.shape[-1])
    h = swiglu(expert.gate_proj(x), expert.up_proj(x), expert.limit)
    return expert.down_proj(h)[:n]


class DirectFP8MoE(torch.nn.Module):
    """Bucketed top-k MoE over separate canonical expert tensors.

    Direct semantics (fp8.py:343-400): routing is a phase boundary with one
    host readback of the expert ids.  Decode (one row, k = 8) evaluates the
    selected experts and the ordered FP32 slot reduction; prefill visits
    experts in ascending id, runs each bucket on the FP8 MFMA contraction
    tree (one-row buckets included) and accumulates T(out * weight) in BF16,
    which SortedGroupedFP8MoE(reduction="direct") reproduces bit for bit.
    """

    def __init__(self, config, gate, shared_experts, device=None):
        super().__init__()
        self.config = config
        self.gate = gate
        self.shared_experts = shared_experts
        self.experts = torch.nn.ModuleList([
            DirectFP8Expert(config.hidden_size, config.moe_intermediate_size, config.swiglu_limit, device=device)
            for _ in range(config.n_routed_experts)
        ])

    def _expert(self, expert_id: int):
        return self.experts[expert_id]

    def forward(self, x):
        indices, scores = self.gate(x)
        k = self.config.num_experts_per_tok
        routes = indices.reshape(-1, k).to("cpu", torch.int64).numpy()
        flat_x = x.reshape(-1, x.shape[-1])
        flat_scores = scores.reshape(-1, k).to(torch.float32)
        tokens = flat_x.shape[0]
        hidden = flat_x.shape[1]
        shared = None
        if self.shared_experts is not None:
            shared = self.shared_experts(x).reshape(tokens, hidden).contiguous()
        route_out = torch.empty((tokens * k, hidden), dtype=torch.bfloat16, device=x.device)
        if tokens == 1 and routes.shape == (1, DECODE_TOP_K):
            for slot, expert_id in enumerate(routes[0]):
                route_out[slot] = self._expert(int(expert_id))(flat_x)[0]
            result = _restore_and_reduce_rows(route_out, flat_scores, 1, k, shared, None)
        else:
            import numpy as np

            for expert_id in np.unique(routes):
                rows_np, slots_np = np.nonzero(routes == expert_id)
                rows = torch.as_tensor(rows_np, device=x.device)
                flat_pos = torch.as_tensor(rows_np * k + slots_np, device=x.device)
                route_out[flat_pos] = _bucket_forward(self._expert(int(expert_id)), flat_x[rows])
            result = _restore_and_reduce_rows(route_out, flat_scores, tokens, k, shared, indices)
        # result = T(T(routed) + shared) (packed.py:922): the add is fused
        # into the reduction kernel.
        return result.reshape(x.shape)
