"""Sorted grouped-expert FP8 prefill on MI355X.

Counterparts of the reference's glm53_flash_mlx/grouped_fp8.py:
``build_route_plan`` (157-170), ``build_grouped_tile_plan`` (173-203),
``grouped_fp8_linear`` (206-262), ``activate_gate_up`` (265-270),
``restore_and_reduce`` (273-276) and ``SortedGroupedFP8MoE`` (279-328).
The fused path (``grouped_from_routes``) runs one prefill plan: exact hi/lo
E4M3 split of the activations, device route sort, gfx950 FP8 MFMA grouped
gate/up with a SwiGLU epilogue, grouped down, the shared expert as a dense
GEMM pair and a deterministic gather-reduce -- no host synchronisation and no
sorted-activation copy.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _native as N
from .abi import GROUPED_MIN_ROUTES
from .fp8 import BLOCK_SIZE
from .packed import PackedFP8MoE, _c_shared
from .router import Float32Gate

GROUPED_TILE_ROWS = 32
PLAN_MAX_EXPERTS = 1024  # the route plan's expert bound (kPlanMaxExperts)
GROUPED_OUTPUT_COLS = 16
GROUPED_K_TILE = 128


def _route_plan(expert_ids: torch.Tensor, scores: torch.Tensor | None, top_k: int, expert_count: int,
                tile_rows: int = GROUPED_TILE_ROWS):
    dev = expert_ids.device
    ids = expert_ids.reshape(-1).to(torch.int32).contiguous()
    routes = ids.numel()
    sc = scores.reshape(-1).to(torch.float32).contiguous() if scores is not None else None
    capacity = (routes + tile_rows - 1) // tile_rows + expert_count
    i32 = dict(dtype=torch.int32, device=dev)
    # sorted positions past the valid routes are never written: zeros keep
    # them in range for gathers
    out = {
        "order": torch.zeros(routes, **i32),
        "inverse": torch.empty(routes, **i32),
        "sorted_experts": torch.zeros(routes, **i32),
        "token_ids": torch.zeros(routes, **i32),
        "sorted_scores": torch.zeros(routes, dtype=torch.float32, device=dev),
        "route_offsets": torch.empty(expert_count + 1, **i32),
        "tile_offsets": torch.empty(expert_count + 1, **i32),
        "tile_experts": torch.empty(capacity, **i32),
        "tile_starts": torch.empty(capacity, **i32),
        "tile_lengths": torch.empty(capacity, **i32),
        "status": torch.zeros(2, **i32),
    }
    lib = N.lib()
    ws_bytes = lib.glm53_route_plan_workspace_bytes(routes, expert_count)
    ws = N.workspace(ws_bytes, dev)
    N.check(lib.glm53_route_plan(N.ptr(ids), N.ptr(sc), routes, top_k, expert_count, tile_rows, N.ptr(out["order"]),
                                 N.ptr(out["inverse"]), N.ptr(out["sorted_experts"]), N.ptr(out["token_ids"]),
                                 N.ptr(out["sorted_scores"]), N.ptr(out["route_offsets"]),
                                 N.ptr(out["tile_offsets"]), N.ptr(out["tile_experts"]), N.ptr(out["tile_starts"]),
                                 N.ptr(out["tile_lengths"]), capacity, N.ptr(out["status"]), N.ptr(ws), ws_bytes,
                                 N.stream_handle(dev)))
    return out


def build_route_plan(x, topk_indices, topk_scores, *, expert_count: int | None = None):
    """Return the expert-sorted route plan (grouped_fp8.py:157-170):
    (sorted_x, sorted expert ids, sorted scores, inverse order).

    The order is a stable sort of the flat (token-major) routes by expert,
    computed on the device with no host synchronisation.  Expert ids are
    histogrammed over ``expert_count`` bins (default: the plan bound of
    1024); a route outside that range is counted as invalid by the device
    plan, gets inverse -1 and no sorted position (the sorted arrays end with
    one zero entry per invalid route).  ``sorted_x`` is materialised
    here only for API parity; the fused prefill gathers token rows in the
    GEMM instead.
    """
    N.require_device(x, topk_indices, topk_scores)
    flat_x = x.reshape(-1, x.shape[-1])
    top_k = topk_indices.shape[-1]
    experts = int(expert_count) if expert_count is not None else PLAN_MAX_EXPERTS
    plan = _route_plan(topk_indices, topk_scores, top_k, experts)
    sorted_x = flat_x.index_select(0, plan["token_ids"].long())
    return sorted_x, plan["sorted_experts"], plan["sorted_scores"], plan["inverse"]


def build_grouped_tile_plan(sorted_experts, expert_count: int, *, check: bool = False):
    """Expert-aligned fixed-capacity tile descriptors (grouped_fp8.py:173-203):
    (tile_experts, tile_starts, tile_lengths, route_offsets, tile_offsets);
    capacity ceil(R/32) + E, unused slots start at R with length 0.  No host
    synchronisation unless ``check`` asks for a ValueError on ids outside
    [0, expert_count)."""
    N.require_device(sorted_experts)
    plan = _route_plan(sorted_experts, None, 1, int(expert_count))
    if check and int(plan["status"][0].item()) != 0:
        raise ValueError(f"expert ids must lie in [0, {expert_count})")
    return (plan["tile_experts"], plan["tile_starts"], plan["tile_lengths"], plan["route_offsets"],
            plan["tile_offsets"])


def grouped_fp8_linear(x, tile_plan, weight, scale_inv):
    """Project sorted route rows from a packed block-FP8 expert bank."""
    N.require_device(x, weight, scale_inv)
    if weight.dtype != torch.uint8 or weight.dim() != 3:
        raise ValueError("grouped weight must be [experts, out, in] uint8 E4M3")
    if scale_inv.dtype != torch.float32 or scale_inv.dim() != 3:
        raise ValueError("grouped scale must be [experts, out_blocks, in_blocks] FP32")
    routes, in_features = x.shape
    experts, out_features, weight_in = weight.shape
    if out_features % BLOCK_SIZE != 0 or in_features % BLOCK_SIZE != 0 or out_features % GROUPED_OUTPUT_COLS != 0:
        raise ValueError("grouped probe requires block-aligned projection dimensions; "
                         f"got out={out_features}, in={in_features}")
    expected_scales = (experts, math.ceil(out_features / BLOCK_SIZE), math.ceil(in_features / BLOCK_SIZE))
    if weight_in != in_features or tuple(scale_inv.shape) != expected_scales:
        raise ValueError(f"incompatible grouped shapes x={tuple(x.shape)}, weight={tuple(weight.shape)}, "
                         f"scale={tuple(scale_inv.shape)}, expected_scale={expected_scales}")
    if x.dtype != torch.bfloat16:
        raise ValueError("grouped activations must be bfloat16")
    tile_experts, tile_starts, tile_lengths = (t.to(torch.int32).contiguous() for t in tile_plan[:3])
    x = x.contiguous()
    y = torch.empty((routes, out_features), dtype=torch.bfloat16, device=x.device)
    lib = N.lib()
    ws_bytes = lib.glm53_grouped_linear_workspace_bytes(routes, in_features)
    ws = N.workspace(ws_bytes, x.device)
    N.check(lib.glm53_grouped_linear(N.ptr(x), routes, None, routes, in_features, N.ptr(tile_experts),
                                     N.ptr(tile_starts), N.ptr(tile_lengths), tile_experts.numel(),
                                     N.ptr(weight.contiguous()), N.ptr(scale_inv.contiguous()), None, experts,
                                     out_features, N.ptr(y), N.ptr(ws), ws_bytes, N.stream_handle(x.device)))
    return y


def activate_gate_up(gate_up, intermediate_size: int, limit: float):
    """h = silu(min(g, L)) * clip(u, -L, L) in MLX BF16 rounding (grouped_fp8.py:265-270)."""
    if intermediate_size % BLOCK_SIZE != 0:
        raise ValueError("gate/up split must align to the block-128 scale boundary")
    N.require_device(gate_up)
    rows = gate_up.shape[0]
    if gate_up.shape[-1] != 2 * intermediate_size or gate_up.dtype != torch.bfloat16:
        raise ValueError("gate_up must be bfloat16 [rows, 2 * intermediate]")
    out = torch.empty((rows, intermediate_size), dtype=torch.bfloat16, device=gate_up.device)
    lib = N.lib()
    N.check(lib.glm53_activate_gate_up(N.ptr(gate_up.contiguous()), rows, intermediate_size, float(limit),
                                       N.ptr(out), N.stream_handle(gate_up.device)))
    return out


def restore_and_reduce(sorted_output, sorted_scores, inverse_order, shape, top_k):
    """y[t] = T(sum_slot sorted_output[inverse[t*k+slot]] * score), FP32 (grouped_fp8.py:273-276)."""
    N.require_device(sorted_output, sorted_scores, inverse_order)
    hidden = sorted_output.shape[-1]
    tokens = sorted_output.shape[0] // top_k
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=sorted_output.device)
    lib = N.lib()
    N.check(lib.glm53_restore_and_reduce(N.ptr(sorted_output.contiguous()),
                                         N.ptr(sorted_scores.to(torch.float32).contiguous()),
                                         N.ptr(inverse_order.to(torch.int32).contiguous()), tokens, top_k, hidden,
                                         None, N.ptr(out), N.stream_handle(sorted_output.device)))
    return out.reshape(shape)


class PrefillPlan:
    """Fixed-scratch prefill plan (native_prefill_moe_plan.h:18-96 counterpart)."""

    def __init__(self, hidden: int, intermediate: int, shared_intermediate: int, experts: int, top_k: int,
                 max_tokens: int, limit: float):
        self._lib = N.lib()
        handle = ctypes.c_void_p()
        N.check(self._lib.glm53_prefill_plan_create(hidden, intermediate, shared_intermediate, experts, top_k,
                                                    max_tokens, float(limit), ctypes.byref(handle)))
        self.handle = handle
        self.max_tokens = max_tokens

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value:
            self._lib.glm53_prefill_plan_destroy(handle)
            self.handle = None

    def run(self, bank, shared, router, x, tokens, ids, scores, reduction, out, device):
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        r = router.as_c_struct() if router is not None else None
        N.check(self._lib.glm53_prefill_moe(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                            ctypes.byref(r) if r else None, N.ptr(x), tokens, N.ptr(ids),
                                            N.ptr(scores), reduction, N.ptr(out), N.stream_handle(device)))

    def run_hc(self, bank, shared, router, x, tokens, ids, scores, reduction, residual, post, comb, out, device):
        """execute_indirect_hc (native_prefill_moe_plan.cpp:101-119): the MoE
        of `run` followed by the hyper-connection expand, fused into the
        reduction: out bf16 [tokens, 4, H] from residual bf16 [tokens, 4, H],
        post f32 [tokens, 4] and comb f32 [tokens, 4, 4]."""
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        r = router.as_c_struct() if router is not None else None
        N.check(self._lib.glm53_prefill_moe_hc(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                               ctypes.byref(r) if r else None, N.ptr(x), tokens, N.ptr(ids),
                                               N.ptr(scores), reduction, N.ptr(residual), N.ptr(post), N.ptr(comb),
                                               N.ptr(out), N.stream_handle(device)))

    def invalid_routes(self) -> int:
        """Synchronous: routes of the last call whose expert id was out of range."""
        value = ctypes.c_uint32()
        N.check(self._lib.glm53_prefill_plan_status(self.handle, ctypes.byref(value)))
        return int(value.value)

    # ---- read-only state of the reference plan (bindings.cpp:389-407)
    def _counters(self) -> N.PlanCounters:
        c = N.PlanCounters()
        N.check(self._lib.glm53_prefill_plan_counters(self.handle, ctypes.byref(c)))
        return c

    @property
    def execution_count(self) -> int:
        return int(self._counters().execution_count)

    @property
    def dynamic_allocation_count(self) -> int:
        return int(self._counters().dynamic_allocation_count)

    @property
    def host_synchronization_count(self) -> int:
        return int(self._counters().host_synchronization_count)

    @property
    def static_input_validation_count(self) -> int:
        return int(self._counters().static_input_validation_count)

    @property
    def dynamic_input_validation_count(self) -> int:
        return int(self._counters().dynamic_input_validation_count)

    @property
    def scratch_bytes(self) -> int:
        return int(self._counters().scratch_bytes)

    @property
    def buffer_identities(self) -> list[int]:
        """Device addresses of the plan's scratch buffers: fixed at creation."""
        cap = 32
        buf = (ctypes.c_uint64 * cap)()
        count = ctypes.c_int32()
        N.check(self._lib.glm53_prefill_plan_identities(self.handle, buf, cap, ctypes.byref(count)))
        return [int(buf[i]) for i in range(count.value)]


class SortedGroupedFP8MoE(PackedFP8MoE):
    """Prefill-only grouped path with the packed decode fallback.

    reduction="grouped" keeps the reference's FP32 slot-order combine;
    reduction="direct" combines in the exact Direct order (ascending expert,
    BF16 accumulation), the parity anchor of native_indexer_plan.metal:
    2174-2207.
    """

    def __init__(self, bank, config, gate, shared_experts, *, min_routes: int = GROUPED_MIN_ROUTES,
                 reduction: str = "grouped"):
        super().__init__(bank, config, gate, shared_experts)
        if reduction not in ("grouped", "direct"):
            raise ValueError("reduction must be 'grouped' or 'direct'")
        self.min_routes = int(min_routes)
        self.reduction = reduction
        self._prefill_plans: dict = {}
        # Plans replaced by a larger one stay alive with the module: a HIP
        # graph captured with an older plan keeps pointing at its arena.
        self._retired_prefill_plans: list = []

    def _prefill_plan(self, device, tokens: int) -> PrefillPlan:
        key = (device.index, torch.cuda.current_stream(device).cuda_stream)
        plan = self._prefill_plans.get(key)
        if plan is None or plan.max_tokens < tokens:
            shared_inter = 0
            if self.shared_experts is not None:
                shared_inter = int(self.shared_experts.gate_proj.weight.shape[0])
            capacity = max(tokens, plan.max_tokens * 2 if plan is not None else 256)
            if plan is not None:
                self._retired_prefill_plans.append(plan)
            plan = PrefillPlan(self.bank.hidden_size, self.bank.intermediate_size, shared_inter,
                               self.bank.expert_count, self.config.num_experts_per_tok, capacity,
                               self.config.swiglu_limit)
            self._prefill_plans[key] = plan
        return plan

    def native_prefill(self, x, expert_ids=None, scores=None):
        """The native call behind glm53::moe_prefill: the fused prefill plan
        with the module's Float32Gate (expert_ids None) or the caller's
        routing."""
        flat = x.reshape(-1, x.shape[-1]).contiguous()
        tokens = flat.shape[0]
        out = torch.empty_like(flat)
        reduction = N.REDUCE_DIRECT if self.reduction == "direct" else N.REDUCE_GROUPED
        plan = self._prefill_plan(x.device, tokens)
        ids = sc = None
        router = self.gate if expert_ids is None else None
        if expert_ids is not None:
            ids = expert_ids.reshape(tokens, -1).to(torch.int32).contiguous()
            sc = scores.reshape(tokens, -1).to(torch.float32).contiguous()
        plan.run(self.bank, _c_shared(self.shared_experts), router, flat, tokens, ids, sc, reduction, out, x.device)
        return out.reshape(x.shape)

    def _last_plan(self, device) -> PrefillPlan:
        return self._prefill_plans[(device.index, torch.cuda.current_stream(device).cuda_stream)]

    def grouped_from_routes(self, x, indices, scores, *, check: bool = True):
        """The grouped prefill on caller-chosen routes (grouped_fp8.py:
        300-321).  check=True reads the plan's invalid-route count back (one
        host synchronisation) and raises ValueError for ids out of range."""
        N.require_device(x, indices, scores)
        if indices.shape[-1] != self.config.num_experts_per_tok:
            raise ValueError("indices do not match num_experts_per_tok")
        result = torch.ops.glm53.moe_prefill(x, self._op_key, indices, scores)
        if check and self._last_plan(x.device).invalid_routes() != 0:
            raise ValueError(f"expert ids must lie in [0, {self.bank.expert_count})")
        return result

    def forward(self, x):
        routes = x.reshape(-1, x.shape[-1]).shape[0] * self.config.num_experts_per_tok
        if routes < self.min_routes:
            return super().forward(x)
        if isinstance(self.gate, Float32Gate):
            N.require_device(x)
            return torch.ops.glm53.moe_prefill(x, self._op_key, None, None)
        indices, scores = self.gate(x)
        return self.grouped_from_routes(x, indices, scores)
