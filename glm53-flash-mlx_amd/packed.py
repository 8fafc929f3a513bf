"""Packed per-layer FP8 expert bank and exact batch-1 decode on MI355X.

Counterparts of the reference's glm53_flash_mlx/packed.py:
``PackedFP8ExpertBank`` (packed.py:747-876) with the same four-buffer layout
contract, per-expert views (658-744), and ``PackedFP8MoE`` (879-923).  The
decode of one token runs in three HIP launches on the caller's stream
(router, fused routed+shared gate/up/SwiGLU, fused down + ordered weighted
reduction + shared add) through a fixed-scratch plan owned by the module,
the MI355X counterpart of ``NativePackedMoEDecodePlan``
(native_packed_moe_plan.h:22-146).
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _native as N
from .fp8 import BLOCK_SIZE, DECODE_TOP_K, DirectFP8MoE, block_fp8_linear, swiglu
from .router import Float32Gate


class _PackedLinearView:
    """One projection of one bank expert; row slices of a contiguous bank are
    themselves contiguous, so no copy is made."""

    def __init__(self, weight, scale_inv, *, expert_id: int, row_offset: int, scale_row_offset: int,
                 out_features: int, bank=None):
        self._bank = bank
        self._bank_weight = weight
        self._bank_scale_inv = scale_inv
        self.expert_id = int(expert_id)
        self.row_offset = int(row_offset)
        self.scale_row_offset = int(scale_row_offset)
        self.out_features = int(out_features)

    @property
    def weight(self):
        return self._bank_weight[self.expert_id, self.row_offset:self.row_offset + self.out_features]

    @property
    def weight_scale_inv(self):
        rows = math.ceil(self.out_features / BLOCK_SIZE)
        return self._bank_scale_inv[self.expert_id, self.scale_row_offset:self.scale_row_offset + rows]

    def __call__(self, x):
        flags = self._bank.code_flags() if self._bank is not None else None
        return block_fp8_linear(x, self.weight, self.weight_scale_inv, flags)


class _PackedExpertView:
    def __init__(self, bank: "PackedFP8ExpertBank", expert_id: int, limit: float):
        inter = bank.intermediate_size
        scale_rows = bank.intermediate_scale_rows
        self.gate_proj = _PackedLinearView(bank.gate_up_weight, bank.gate_up_scale_inv, expert_id=expert_id,
                                           row_offset=0, scale_row_offset=0, out_features=inter, bank=bank)
        self.up_proj = _PackedLinearView(bank.gate_up_weight, bank.gate_up_scale_inv, expert_id=expert_id,
                                         row_offset=inter, scale_row_offset=scale_rows, out_features=inter,
                                         bank=bank)
        self.down_proj = _PackedLinearView(bank.down_weight, bank.down_scale_inv, expert_id=expert_id,
                                           row_offset=0, scale_row_offset=0, out_features=bank.down_weight.shape[1],
                                           bank=bank)
        self.limit = float(limit)

    def __call__(self, x):
        return self.down_proj(swiglu(self.gate_proj(x), self.up_proj(x), self.limit))


class PackedFP8ExpertBank(torch.nn.Module):
    """Four contiguous canonical-FP8 buffers for one routed MoE layer.

    gate_up_weight u8 [E, 2I, H] (gate rows, then up rows), gate_up_scale_inv
    f32 [E, 2*ceil(I/128), ceil(H/128)], down_weight u8 [E, H, I],
    down_scale_inv f32 [E, ceil(H/128), ceil(I/128)].  The bank owns its
    bytes (ownership.py:42-61 of the reference).
    """

    def __init__(self, gate_up_weight, gate_up_scale_inv, down_weight, down_scale_inv, *, intermediate_size: int):
        super().__init__()
        tensors = (gate_up_weight, gate_up_scale_inv, down_weight, down_scale_inv)
        if any(not isinstance(t, torch.Tensor) for t in tensors):
            raise ValueError("bank buffers must be tensors")
        if any(not t.is_contiguous() for t in tensors):
            raise ValueError("bank buffers must be row-major contiguous")
        if gate_up_weight.dtype != torch.uint8 or down_weight.dtype != torch.uint8:
            raise ValueError("packed expert weights must remain uint8 E4M3")
        if gate_up_scale_inv.dtype != torch.float32 or down_scale_inv.dtype != torch.float32:
            raise ValueError("packed expert scales must remain float32")
        inter = int(intermediate_size)
        experts, rows, hidden = gate_up_weight.shape
        sr, sh = math.ceil(inter / BLOCK_SIZE), math.ceil(hidden / BLOCK_SIZE)
        expected = {
            "gate_up_weight": (gate_up_weight.shape, (experts, 2 * inter, hidden)),
            "gate_up_scale_inv": (gate_up_scale_inv.shape, (experts, 2 * sr, sh)),
            "down_weight": (down_weight.shape, (experts, hidden, inter)),
            "down_scale_inv": (down_scale_inv.shape, (experts, sh, sr)),
        }
        for name, (actual, wanted) in expected.items():
            if tuple(actual) != wanted:
                raise ValueError(f"{name} shape {tuple(actual)} != {wanted}")
        if len({t.device for t in tensors}) != 1:
            raise ValueError("bank buffers must live on one device")
        self.register_buffer("gate_up_weight", gate_up_weight)
        self.register_buffer("gate_up_scale_inv", gate_up_scale_inv)
        self.register_buffer("down_weight", down_weight)
        self.register_buffer("down_scale_inv", down_scale_inv)
        self.intermediate_size = inter
        self.intermediate_scale_rows = sr

    @classmethod
    def pack(cls, experts) -> "PackedFP8ExpertBank":
        experts = list(experts)
        if not experts:
            raise ValueError("cannot pack an empty expert list")
        hidden = experts[0].gate_proj.weight.shape[1]
        inter = experts[0].gate_proj.weight.shape[0]
        for expert in experts:
            expected = (
                (tuple(expert.gate_proj.weight.shape), (inter, hidden)),
                (tuple(expert.up_proj.weight.shape), (inter, hidden)),
                (tuple(expert.down_proj.weight.shape), (hidden, inter)),
            )
            if any(actual != wanted for actual, wanted in expected):
                raise ValueError("expert projection shapes are not uniform")
            for projection in (expert.gate_proj, expert.up_proj, expert.down_proj):
                if projection.weight.dtype != torch.uint8:
                    raise ValueError("packed expert weights must remain uint8 E4M3")
                if projection.weight_scale_inv.dtype != torch.float32:
                    raise ValueError("packed expert scales must remain float32")
        gate_up_weight = torch.stack([torch.cat([e.gate_proj.weight, e.up_proj.weight], 0) for e in experts])
        gate_up_scale = torch.stack([torch.cat([e.gate_proj.weight_scale_inv, e.up_proj.weight_scale_inv], 0)
                                     for e in experts])
        down_weight = torch.stack([e.down_proj.weight for e in experts])
        down_scale = torch.stack([e.down_proj.weight_scale_inv for e in experts])
        return cls(gate_up_weight.contiguous(), gate_up_scale.contiguous(), down_weight.contiguous(),
                   down_scale.contiguous(), intermediate_size=inter)

    @property
    def expert_count(self) -> int:
        return int(self.gate_up_weight.shape[0])

    @property
    def hidden_size(self) -> int:
        return int(self.gate_up_weight.shape[2])

    @property
    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in
                   (self.gate_up_weight, self.gate_up_scale_inv, self.down_weight, self.down_scale_inv))

    def expert(self, expert_id: int, *, limit: float) -> _PackedExpertView:
        if not 0 <= expert_id < self.expert_count:
            raise IndexError(expert_id)
        return _PackedExpertView(self, expert_id, limit)

    def code_flags(self) -> torch.Tensor:
        """Device int32 flag, nonzero when the bank holds E4M3 codes 0x7F/0xFF
        (+-480 in the reference table, NaN for the MFMA).  Scanned once per
        weight version and cached."""
        stamp = (self.gate_up_weight.data_ptr(), self.gate_up_weight._version, self.down_weight.data_ptr(),
                 self.down_weight._version)
        cached = getattr(self, "_code_flags", None)
        if cached is None or cached[0] != stamp:
            flags = torch.bitwise_or(N.scan_codes(self.gate_up_weight), N.scan_codes(self.down_weight))
            self._code_flags = (stamp, flags)
        return self._code_flags[1]

    def as_c_struct(self) -> N.Bank:
        return N.Bank(self.gate_up_weight.data_ptr(), self.gate_up_scale_inv.data_ptr(), self.down_weight.data_ptr(),
                      self.down_scale_inv.data_ptr(), self.expert_count, self.hidden_size, self.intermediate_size,
                      self.code_flags().data_ptr())


class BankHandle:
    """Native bank handle (glm53_bank_create): the bank's reference layout
    validated once and its 0x7F/0xFF code flag scanned once and owned by the
    handle.  `ptr` is a `glm53_bank*` for the C ABI's entry points; the bank
    object (and so its weights) stays referenced while the handle lives."""

    def __init__(self, bank: "PackedFP8ExpertBank", device: torch.device | None = None):
        self._lib = N.lib()
        self._bank = bank
        self._device = device if device is not None else bank.gate_up_weight.device
        N.require_device(bank.gate_up_weight, bank.down_weight)
        desc = bank.as_c_struct()
        self.ptr = ctypes.POINTER(N.Bank)()
        N.check(self._lib.glm53_bank_create(ctypes.byref(desc), N.stream_handle(self._device), ctypes.byref(self.ptr)))

    def close(self) -> None:
        if self.ptr:
            torch.cuda.synchronize(self._device)  # no call may still use the flag
            self._lib.glm53_bank_destroy(self.ptr)
            self.ptr = ctypes.POINTER(N.Bank)()

    def __enter__(self) -> "BankHandle":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        if getattr(self, "ptr", None):
            self.close()


class DecodePlan:
    """Fixed-scratch batch-1 decode plan (one per layer and stream)."""

    def __init__(self, hidden: int, intermediate: int, shared_intermediate: int, experts: int, top_k: int,
                 limit: float):
        self._lib = N.lib()
        handle = ctypes.c_void_p()
        N.check(self._lib.glm53_decode_plan_create(hidden, intermediate, shared_intermediate, experts, top_k,
                                                   float(limit), ctypes.byref(handle)))
        self.handle = handle
        self.top_k = top_k
        self._dims = (int(hidden), int(intermediate), int(shared_intermediate), int(experts))
        self._executions = 0

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value:
            self._lib.glm53_decode_plan_destroy(handle)
            self.handle = None

    def _execute(self, status: int) -> None:
        N.check(status)
        self._executions += 1

    # Read-only counters of the reference plan (bindings.cpp:584-632).
    @property
    def hidden_size(self) -> int:
        return self._dims[0]

    @property
    def intermediate_size(self) -> int:
        return self._dims[1]

    @property
    def shared_intermediate_size(self) -> int:
        return self._dims[2]

    @property
    def expert_count(self) -> int:
        return self._dims[3]

    @property
    def execution_count(self) -> int:
        return self._executions

    @property
    def dynamic_allocation_count(self) -> int:
        return 0  # all device scratch is one arena allocated at creation

    @property
    def host_synchronization_count(self) -> int:
        return 0  # every call only enqueues on the caller's stream

    @property
    def weights_bound(self) -> bool:
        return getattr(self, "_bound", None) is not None

    @property
    def bound_weight_identities_stable(self) -> bool:
        bound = getattr(self, "_bound", None)
        return bound is not None and [(t.data_ptr(), t._version) for t in self._bound_tensors(*bound[:3])] == \
            self._bound_identity

    @property
    def scratch_bytes(self) -> int:
        ptr, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
        N.check(self._lib.glm53_decode_plan_scratch(self.handle, 4, ctypes.byref(ptr), ctypes.byref(nbytes)))
        return int(nbytes.value)

    def routed(self, bank, shared, x, ids, scores, out, device):
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        self._execute(self._lib.glm53_decode_moe_routed(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                                        N.ptr(x), N.ptr(ids), N.ptr(scores), N.ptr(out),
                                                        N.stream_handle(device)))

    def full(self, bank, shared, router, x, out, ids_out, scores_out, device):
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        r = router.as_c_struct()
        self._execute(self._lib.glm53_decode_moe(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                                 ctypes.byref(r), N.ptr(x), N.ptr(out), N.ptr(ids_out),
                                                 N.ptr(scores_out), N.stream_handle(device)))

    def step(self, bank, shared, router, x, residual, out, stages, device):
        """Decoder-step form: out = T(residual + T(moe(x))) (residual may be
        None); stages is a mask of the router / gate-up / down launches."""
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        r = router.as_c_struct() if router is not None else None
        self._execute(self._lib.glm53_decode_moe_ex(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                                    ctypes.byref(r) if r else None, N.ptr(x), N.ptr(residual),
                                                    N.ptr(out), int(stages), N.stream_handle(device)))

    @staticmethod
    def _bound_tensors(bank, shared, router):
        tensors = [bank.gate_up_weight, bank.gate_up_scale_inv, bank.down_weight, bank.down_scale_inv]
        if shared is not None:
            for proj in (shared.gate_proj, shared.up_proj, shared.down_proj):
                tensors += [proj.weight, proj.weight_scale_inv]
        return tensors + [router.weight, router.e_score_correction_bias]

    def bind_weights(self, bank, shared, router) -> None:
        """Bind one layer's weights once (bindings.cpp:576-583,
        native_packed_moe_plan.cpp:231-258); binding again raises
        RuntimeError.  The storage identity of every bound tensor is
        recorded for execute_bound."""
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        r = router.as_c_struct()
        N.check(self._lib.glm53_decode_plan_bind(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                                 ctypes.byref(r)))
        flags = [bank.code_flags()]
        if shared is not None:
            flags += [shared.gate_proj.code_flags(), shared.up_proj.code_flags(), shared.down_proj.code_flags()]
        self._bound = (bank, shared, router, flags)  # keeps the scanned flag tensors the plan points at alive
        self._bound_identity = [(t.data_ptr(), t._version) for t in self._bound_tensors(bank, shared, router)]

    def execute_bound(self, x, out, device) -> None:
        """Decode x [H] with the bound weights into out [H]
        (native_packed_moe_plan.cpp:260-280).  Raises RuntimeError when
        nothing is bound, or when a bound tensor was replaced or modified in
        place since binding (its 0x7F/0xFF code flags were scanned then)."""
        bound = getattr(self, "_bound", None)
        if bound is None:
            raise RuntimeError("decode plan weights are not bound")
        now = [(t.data_ptr(), t._version) for t in self._bound_tensors(*bound[:3])]
        if now != self._bound_identity:
            raise RuntimeError("decode plan bound weight identity changed")
        self._execute(self._lib.glm53_decode_moe_bound(self.handle, N.ptr(x), N.ptr(out), N.stream_handle(device)))

    def tune(self, gate_up_rows_per_wave: int = 8, down_rows_per_wg: int = 16) -> None:
        N.check(self._lib.glm53_decode_plan_tune(self.handle, int(gate_up_rows_per_wave), int(down_rows_per_wg)))

    def set_mode(self, mode: int) -> None:
        """N.DECODE_THREE_LAUNCH (default) or N.DECODE_SINGLE_LAUNCH."""
        N.check(self._lib.glm53_decode_plan_set_mode(self.handle, int(mode)))

    def error_flag(self) -> int:
        value = ctypes.c_int32()
        N.check(self._lib.glm53_decode_plan_error_flag(self.handle, ctypes.byref(value)))
        return int(value.value)


def _c_shared(shared_experts):
    """Shared expert as block-FP8 linears, or None when absent."""
    if shared_experts is None:
        return None
    if not all(hasattr(shared_experts, n) for n in ("gate_proj", "up_proj", "down_proj")):
        raise ValueError("shared expert must expose gate_proj/up_proj/down_proj BlockFP8Linear projections")
    return shared_experts


class PackedFP8MoE(DirectFP8MoE):
    """Exact fused batch-1 decode and Direct semantics over a packed bank."""

    def __init__(self, bank, config, gate, shared_experts):
        torch.nn.Module.__init__(self)
        self.bank = bank
        self.config = config
        self.gate = gate
        self.shared_experts = shared_experts
        self._expert_views = tuple(bank.expert(i, limit=config.swiglu_limit) for i in range(bank.expert_count))
        self._plans: dict = {}

    def _expert(self, expert_id: int):
        return self._expert_views[expert_id]

    def _plan(self, device) -> DecodePlan:
        key = (device.index, torch.cuda.current_stream(device).cuda_stream)
        plan = self._plans.get(key)
        if plan is None:
            shared_inter = 0
            if self.shared_experts is not None:
                shared_inter = int(self.shared_experts.gate_proj.weight.shape[0])
            plan = DecodePlan(self.bank.hidden_size, self.bank.intermediate_size, shared_inter,
                              self.bank.expert_count, DECODE_TOP_K, self.config.swiglu_limit)
            self._plans[key] = plan
        return plan

    def decode_routed(self, x, expert_ids, scores):
        """Routed + shared decode for externally chosen experts (the
        reference's execute(x, ids, scores), native_packed_moe_plan.cpp:151)."""
        N.require_device(x)
        flat = x.reshape(-1).contiguous()
        ids = expert_ids.reshape(-1).to(torch.int32).contiguous()
        sc = scores.reshape(-1).to(torch.float32).contiguous()
        if ids.numel() != DECODE_TOP_K or sc.numel() != DECODE_TOP_K:
            raise ValueError(f"decode expects {DECODE_TOP_K} expert ids and scores")
        out = torch.empty_like(flat)
        self._plan(x.device).routed(self.bank, _c_shared(self.shared_experts), flat, ids, sc, out, x.device)
        return out.reshape(x.shape)

    def forward(self, x):
        flat_x = x.reshape(-1, x.shape[-1])
        if flat_x.shape[0] != 1:
            return super().forward(x)
        if isinstance(self.gate, Float32Gate) and self.gate.top_k == DECODE_TOP_K:
            N.require_device(x)
            flat = flat_x.reshape(-1).contiguous()
            out = torch.empty_like(flat)
            self._plan(x.device).full(self.bank, _c_shared(self.shared_experts), self.gate, flat, out, None, None,
                                      x.device)
            return out.reshape(x.shape)
        indices, scores = self.gate(x)
        if indices.shape[-1] != DECODE_TOP_K:
            return super().forward(x)
        return self.decode_routed(x, indices, scores)
