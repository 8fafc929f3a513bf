"""Seeded synthetic MoE layers generated on the device.

Weights ~ N(0, 0.02) quantised per 128x128 block (scale_inv = amax / 448,
E4M3 RNE, saturated at +-448), router weight ~ N(0, 0.02) FP32, router bias
~ U(-0.01, 0.01), activations ~ N(0, 1) in BF16.  Every tensor has its own
64-bit key derived from (seed, layer, expert, matrix), so any expert can be
regenerated alone; the 229 GB 42-layer bank never touches the host.
"""

from __future__ import annotations

import math
from types import SimpleNamespace

import torch

from . import _native as N
from .fp8 import BLOCK_SIZE, ClampedMLP
from .ownership import TensorLayout, owned_tensor
from .packed import DEFAULT_LAYOUT, PackedFP8ExpertBank
from .router import Float32Gate

_MASK = (1 << 64) - 1


def _mix(z: int) -> int:
    z = (z + 0x9E3779B97F4A7C15) & _MASK
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK
    return z ^ (z >> 31)


def key(*parts) -> int:
    """64-bit stream key of a tuple of ints / strings."""
    h = 0x243F6A8885A308D3
    for p in parts:
        if isinstance(p, str):
            p = int.from_bytes(p.encode()[:8].ljust(8, b"\0"), "little")
        h = _mix(h ^ (int(p) & _MASK))
    return h


def fill_fp8(codes: torch.Tensor, scale: torch.Tensor, seed: int, std: float = 0.02) -> None:
    rows, cols = codes.shape
    if scale.shape != (math.ceil(rows / BLOCK_SIZE), math.ceil(cols / BLOCK_SIZE)):
        raise ValueError("scale shape does not match codes")
    if not (codes.is_contiguous() and scale.is_contiguous()):
        raise ValueError("synthetic targets must be contiguous")
    N.check(N.lib().glm53_synth_fp8(N.ptr(codes), N.ptr(scale), rows, cols, seed, float(std),
                                    N.stream_handle(codes.device)))


def normal_f32(n: int, seed: int, std: float, device) -> torch.Tensor:
    out = torch.empty(n, dtype=torch.float32, device=device)
    N.check(N.lib().glm53_synth_f32(N.ptr(out), n, seed, float(std), 0.0, 0.0, 0, N.stream_handle(out.device)))
    return out


def uniform_f32(n: int, seed: int, lo: float, hi: float, device) -> torch.Tensor:
    out = torch.empty(n, dtype=torch.float32, device=device)
    N.check(N.lib().glm53_synth_f32(N.ptr(out), n, seed, 0.0, float(lo), float(hi), 1, N.stream_handle(out.device)))
    return out


def normal_bf16(shape, seed: int, std: float = 1.0, device="cuda") -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
    N.check(N.lib().glm53_synth_bf16(N.ptr(out), out.numel(), seed, float(std), N.stream_handle(out.device)))
    return out


def synth_bank(experts: int, hidden: int, intermediate: int, seed: int, layer: int = 0,
               device="cuda", std: float = 0.02, layout=None) -> PackedFP8ExpertBank:
    """A seeded bank written straight into `layout` (the package's
    DEFAULT_LAYOUT when None, "rows", "tiled" or a row-group exponent;
    shapes whose widths are not multiples of 128 are always row-major).  The
    expert values do not depend on the layout."""
    layout = DEFAULT_LAYOUT if layout is None else layout
    if hidden % BLOCK_SIZE or intermediate % BLOCK_SIZE:
        layout = "rows"
    g = {"rows": N.ROWS_LAYOUT, "tiled": N.TILED_LAYOUT}.get(layout, layout)
    sr, sh = math.ceil(intermediate / BLOCK_SIZE), math.ceil(hidden / BLOCK_SIZE)
    gu = torch.empty((experts, 2 * intermediate, hidden), dtype=torch.uint8, device=device)
    gus = torch.empty((experts, 2 * sr, sh), dtype=torch.float32, device=device)
    dw = torch.empty((experts, hidden, intermediate), dtype=torch.uint8, device=device)
    dws = torch.empty((experts, sh, sr), dtype=torch.float32, device=device)
    lib = N.lib()
    stream = N.stream_handle(gu.device)
    # one launch per projection over all experts; expert e of a projection
    # draws from the key derived from (projection key, e)
    # (the up rows start at row I, a whole number of row groups, so the up
    # matrix is written at byte offset I * H in either layout)
    N.check(lib.glm53_synth_fp8_batched(N.ptr(gu), N.ptr(gus), intermediate, hidden, experts,
                                        2 * intermediate * hidden, 2 * sr * sh, key(seed, layer, "gate"), std, g,
                                        stream))
    N.check(lib.glm53_synth_fp8_batched(N.ctypes.c_void_p(gu.data_ptr() + intermediate * hidden),
                                        N.ctypes.c_void_p(gus.data_ptr() + 4 * sr * sh), intermediate, hidden, experts,
                                        2 * intermediate * hidden, 2 * sr * sh, key(seed, layer, "up"), std, g, stream))
    N.check(lib.glm53_synth_fp8_batched(N.ptr(dw), N.ptr(dws), hidden, intermediate, experts, hidden * intermediate,
                                        sh * sr, key(seed, layer, "down"), std, g, stream))
    rm = TensorLayout.ROW_MAJOR_CONTIGUOUS
    return PackedFP8ExpertBank(owned_tensor(gu, layout=rm), owned_tensor(gus, layout=rm), owned_tensor(dw, layout=rm),
                               owned_tensor(dws, layout=rm), intermediate_size=intermediate, layout=g)


def synth_shared(hidden: int, intermediate: int, limit: float, seed: int, layer: int = 0, device="cuda",
                 std: float = 0.02) -> ClampedMLP:
    mlp = ClampedMLP(hidden, intermediate, limit, device=device)
    fill_fp8(mlp.gate_proj.weight, mlp.gate_proj.weight_scale_inv, key(seed, layer, "shared", "gate"), std)
    fill_fp8(mlp.up_proj.weight, mlp.up_proj.weight_scale_inv, key(seed, layer, "shared", "up"), std)
    fill_fp8(mlp.down_proj.weight, mlp.down_proj.weight_scale_inv, key(seed, layer, "shared", "down"), std)
    return mlp


def synth_gate(experts: int, hidden: int, seed: int, layer: int = 0, device="cuda", top_k: int = 8,
               routed_scaling_factor: float = 1.0, bias: torch.Tensor | None = None) -> Float32Gate:
    w = normal_f32(experts * hidden, key(seed, layer, "router", "w"), 0.02, device).reshape(experts, hidden)
    if bias is None:
        bias = uniform_f32(experts, key(seed, layer, "router", "b"), -0.01, 0.01, device)
    return Float32Gate(w, bias.to(device=device, dtype=torch.float32), top_k=top_k,
                       routed_scaling_factor=routed_scaling_factor, norm_topk_prob=True)


def layer_config(hidden=4096, intermediate=1536, experts=288, top_k=8, limit=10.0, shared=1):
    return SimpleNamespace(hidden_size=hidden, moe_intermediate_size=intermediate, swiglu_limit=float(limit),
                           n_routed_experts=experts, num_experts_per_tok=top_k, n_shared_experts=shared)


def synth_layer(config, seed: int, layer: int = 0, device="cuda", bias: torch.Tensor | None = None,
                layout=None):
    """(bank, shared expert, gate) of one synthetic MoE layer."""
    bank = synth_bank(config.n_routed_experts, config.hidden_size, config.moe_intermediate_size, seed, layer, device,
                      layout=layout)
    shared = None
    if config.n_shared_experts:
        shared = synth_shared(config.hidden_size, config.moe_intermediate_size * config.n_shared_experts,
                              config.swiglu_limit, seed, layer, device)
    gate = synth_gate(config.n_routed_experts, config.hidden_size, seed, layer, device,
                      top_k=config.num_experts_per_tok, bias=bias)
    return bank, shared, gate


def zipf_bias(experts: int, s: float = 1.1, strength: float = 0.12, seed: int = 0) -> torch.Tensor:
    """Router bias that skews selection toward a Zipf(s) popularity order:
    bias_e = -strength * s * ln(1 + rank_e), ranks a seeded permutation."""
    g = torch.Generator().manual_seed(seed)
    rank = torch.randperm(experts, generator=g).to(torch.float64)
    return (-strength * s * torch.log1p(rank)).to(torch.float32)
