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
from . import ops
from .fp8 import BLOCK_SIZE, DECODE_TOP_K, DirectFP8MoE, block_fp8_linear, swiglu
from .ownership import (ResidentTensor, TensorLayout, borrowed_stable_tensor, owned_tensor, require_resident,
                        resident_concatenate, storage_descriptor)
from .router import Float32Gate


class _PackedLinearView:
    """One projection of one bank expert.  In a row-major bank its rows are a
    contiguous slice (no copy); in a row-group bank `weight` returns the
    expert's rows re-laid into the reference row-major layout (a copy)."""

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
        if self._bank is not None and self._bank.row_group_log2 != 0:
            rows = _reference_rows(self._bank_weight[self.expert_id:self.expert_id + 1], self._bank.row_group_log2)
            return rows[0, self.row_offset:self.row_offset + self.out_features]
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


def _bank_lease(value, name: str) -> ResidentTensor:
    try:
        return require_resident(value)
    except TypeError as exc:
        raise TypeError(f"PackedFP8ExpertBank {name}: {exc}") from None


LAYOUTS = {"rows": N.ROWS_LAYOUT, "tiled": N.TILED_LAYOUT}
# The layout the package's own banks are built in (pack, the synthetic and
# checkpoint loaders).  Row-major: on MI355X the batch-1 decode step, the
# headline workload, streams it 0.6-1.4 us per layer faster than any row-group
# layout (41.75 against 42.36-43.12 us at 16-row to 2-row groups), which
# outweighs the grouped prefill's 1-3% gain from 4- or 8-row groups.
DEFAULT_LAYOUT = "rows"


def _layout_log2(layout, hidden: int, intermediate: int) -> int:
    """Row-group exponent of a bank layout name ("rows", "tiled") or an
    explicit exponent 0..7 (glm53_bank.row_group_log2)."""
    g = LAYOUTS.get(layout, layout) if isinstance(layout, str) else layout
    if not isinstance(g, int) or isinstance(g, bool) or not 0 <= g <= N.MAX_ROW_GROUP_LOG2:
        raise ValueError(f"bank layout must be one of {sorted(LAYOUTS)} or a row-group exponent 0..."
                         f"{N.MAX_ROW_GROUP_LOG2}, got {layout!r}")
    if g and (hidden % BLOCK_SIZE or intermediate % BLOCK_SIZE):
        raise ValueError(f"a row-group bank layout needs hidden and intermediate multiples of {BLOCK_SIZE}, got "
                         f"hidden={hidden}, intermediate={intermediate}")
    return g


def _reference_rows(weight: torch.Tensor, g: int) -> torch.Tensor:
    """uint8 [E, rows, cols] expert matrices in row groups of 2^g rows,
    re-laid into the reference row-major layout (a new tensor)."""
    out = torch.empty_like(weight)
    N.relayout(weight.contiguous(), out, g, N.ROWS_LAYOUT)
    return out


class PackedFP8ExpertBank(torch.nn.Module):
    """Four contiguous canonical-FP8 buffers for one routed MoE layer.

    gate_up_weight u8 [E, 2I, H] (gate rows, then up rows), gate_up_scale_inv
    f32 [E, 2*ceil(I/128), ceil(H/128)], down_weight u8 [E, H, I],
    down_scale_inv f32 [E, ceil(H/128), ceil(I/128)] (packed.py:747-787).
    Each buffer arrives as a storage lease (ownership.py): owned, or
    borrowed-stable with its owner kept referenced by the bank; an
    ephemeral lease or a bare tensor is refused, because native plans and
    captured graphs keep the bank's device pointers.

    `layout` names how the two weight tensors hold each expert matrix:
    "rows" (the default) is the reference's row-major layout, the
    checkpoint's and the import / export format; "tiled" holds row groups
    of 16 rows whose K span is stored as consecutive 16-row x 128-byte
    blocks, and an integer g any row-group size 2^g (glm53_moe.h,
    glm53_bank).  Every entry point reads every layout with the same bits.
    ``pack``, the synthetic banks and the checkpoint loader build
    DEFAULT_LAYOUT banks unless told otherwise; ``relayout_`` converts an
    owned bank in place and ``reference_weights`` exports the row-major
    bytes.  The tensor shapes and block scales are the same in all layouts.
    """

    def __init__(self, gate_up_weight, gate_up_scale_inv, down_weight, down_scale_inv, *, intermediate_size: int,
                 layout="rows"):
        super().__init__()
        names = ("gate_up_weight", "gate_up_scale_inv", "down_weight", "down_scale_inv")
        resident = {n: _bank_lease(v, n) for n, v in zip(names, (gate_up_weight, gate_up_scale_inv, down_weight,
                                                                    down_scale_inv))}
        values = {n: r.value for n, r in resident.items()}
        for n in ("gate_up_weight", "down_weight"):
            if values[n].dtype != torch.uint8 or values[n].dim() != 3:
                raise ValueError(f"{n} must be a 3-D uint8 E4M3 tensor, got {values[n].dtype} "
                                 f"{tuple(values[n].shape)}")
        for n in ("gate_up_scale_inv", "down_scale_inv"):
            if values[n].dtype != torch.float32 or values[n].dim() != 3:
                raise ValueError(f"{n} must be a 3-D float32 block table, got {values[n].dtype}")
        inter = int(intermediate_size)
        n_exp, _, hidden = values["gate_up_weight"].shape
        ri, rh = math.ceil(inter / BLOCK_SIZE), math.ceil(hidden / BLOCK_SIZE)
        shapes = {"gate_up_weight": (n_exp, 2 * inter, hidden), "gate_up_scale_inv": (n_exp, 2 * ri, rh),
                  "down_weight": (n_exp, hidden, inter), "down_scale_inv": (n_exp, rh, ri)}
        wrong = [f"{n} {tuple(values[n].shape)} (want {shape})" for n, shape in shapes.items()
                 if tuple(values[n].shape) != shape]
        if wrong:
            raise ValueError("bank layout mismatch: " + "; ".join(wrong))
        if len({v.device for v in values.values()}) != 1:
            raise ValueError("bank buffers must live on one device")
        for n, v in values.items():
            self.register_buffer(n, v)
        self.storage_contracts = {n: storage_descriptor(r) for n, r in resident.items()}
        self._storage_owners = tuple(r.owner for r in resident.values() if r.owner is not None)
        self._weights_writable = all(resident[n].writable for n in ("gate_up_weight", "down_weight"))
        self.intermediate_size = inter
        self.intermediate_scale_rows = ri
        self.row_group_log2 = _layout_log2(layout, hidden, inter)

    @property
    def layout(self) -> str:
        """"rows", "tiled", or "groups<n>" for another row-group size."""
        names = {g: n for n, g in LAYOUTS.items()}
        return names.get(self.row_group_log2, f"groups{1 << self.row_group_log2}")

    def relayout_(self, layout="tiled") -> "PackedFP8ExpertBank":
        """Re-lay both weight tensors in place into `layout` ("rows",
        "tiled" or a row-group exponent).  Only owned weights are rewritten:
        a borrowed lease's storage belongs to its owner.  Runs on the current
        stream through a staging copy of at most 256 MB at a time; plans and
        graphs made with the old layout must not run afterwards (the layout
        is part of every call's bank descriptor)."""
        target = _layout_log2(layout, self.hidden_size, self.intermediate_size)
        if target == self.row_group_log2:
            return self
        if not self._weights_writable:
            raise ValueError("relayout_() rewrites the weights in place, but this bank borrows them; build it from "
                             "owned leases (or materialize_owned copies) to re-lay it")
        for name in ("gate_up_weight", "down_weight"):
            weight = getattr(self, name)
            per_expert = weight[0].numel()
            step = max(1, (256 << 20) // per_expert)
            for e0 in range(0, weight.shape[0], step):
                part = weight[e0:e0 + step]
                N.relayout(part.clone(), part, self.row_group_log2, target)
        self.row_group_log2 = target
        return self

    def reference_weights(self, expert_ids=None) -> tuple[torch.Tensor, torch.Tensor]:
        """(gate_up_weight, down_weight) of the experts `expert_ids` (all by
        default) in the reference row-major layout: the tensors themselves
        (or an index_select) for a row-major bank, a re-laid copy for a
        row-group bank."""
        gu, dw = self.gate_up_weight, self.down_weight
        if expert_ids is not None:
            idx = torch.as_tensor(expert_ids, dtype=torch.int64, device=gu.device).reshape(-1)
            gu, dw = gu.index_select(0, idx), dw.index_select(0, idx)
        if self.row_group_log2 == 0:
            return gu, dw
        return _reference_rows(gu, self.row_group_log2), _reference_rows(dw, self.row_group_log2)

    @classmethod
    def pack(cls, experts, *, layout=None) -> "PackedFP8ExpertBank":
        """Stack separate experts (each with gate_proj / up_proj / down_proj
        block-FP8 linears) into one owned bank, expert-major, gate rows
        before up rows (packed.py:782-850), then re-lay it on the device
        into `layout` (DEFAULT_LAYOUT when None; "rows" is the reference
        layout; a bank in host memory, or of a shape whose hidden or
        intermediate width is not a multiple of 128, stays row-major).
        Every projection must keep uint8 E4M3 weights and float32 block
        scales of one shape per projection kind."""
        experts = list(experts)
        if not experts:
            raise ValueError("pack() needs at least one expert")
        inter, hidden = (int(d) for d in experts[0].gate_proj.weight.shape)
        kinds = (("gate_proj", (inter, hidden)), ("up_proj", (inter, hidden)), ("down_proj", (hidden, inter)))
        for index, expert in enumerate(experts):
            for kind, shape in kinds:
                proj = getattr(expert, kind)
                if tuple(proj.weight.shape) != shape:
                    raise ValueError(f"expert {index} {kind} weight {tuple(proj.weight.shape)} breaks the uniform "
                                     f"shape {shape}")
                if proj.weight.dtype != torch.uint8 or proj.weight_scale_inv.dtype != torch.float32:
                    raise ValueError(f"expert {index} {kind}: weights must stay uint8 E4M3 with float32 scales")

        def stack(kinds_in_row_order, attr):
            parts = [borrowed_stable_tensor(getattr(getattr(e, k), attr), owner=getattr(e, k))
                     for e in experts for k in kinds_in_row_order]
            flat = resident_concatenate(parts, axis=0).value
            return owned_tensor(flat.view(len(experts), -1, flat.shape[-1]), layout=TensorLayout.ROW_MAJOR_CONTIGUOUS)

        bank = cls(stack(("gate_proj", "up_proj"), "weight"), stack(("gate_proj", "up_proj"), "weight_scale_inv"),
                   stack(("down_proj",), "weight"), stack(("down_proj",), "weight_scale_inv"),
                   intermediate_size=inter)
        layout = DEFAULT_LAYOUT if layout is None else layout
        if layout != "rows" and bank.gate_up_weight.is_cuda and hidden % BLOCK_SIZE == 0 and inter % BLOCK_SIZE == 0:
            bank.relayout_(layout)
        return bank

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
                      self.code_flags().data_ptr(), self.row_group_log2)


class BankHandle:
    """Native bank handle (glm53_bank_create): the bank's descriptor (either
    layout) validated once and its 0x7F/0xFF code flag scanned once and owned
    by the handle.  `ptr` is a `glm53_bank*` for the C ABI's entry points; the bank
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
    """Fixed-scratch batch-1 decode plan, one per layer and stream: the
    counterpart of ``NativePackedMoEDecodePlan`` (native_packed_moe_plan.h:
    22-146, bindings.cpp:562-632) over ``glm53_decode_plan``.

    Weights are borrowed (their pointers are passed per call, or recorded by
    bind_weights); scratch is one device arena allocated at creation.  The
    counters are the native plan's own (glm53_decode_plan_counters)."""

    _IDENTITY_CAPACITY = 16

    def __init__(self, hidden: int, intermediate: int, shared_intermediate: int, experts: int, top_k: int,
                 limit: float):
        self._lib = N.lib()
        handle = ctypes.c_void_p()
        N.check(self._lib.glm53_decode_plan_create(hidden, intermediate, shared_intermediate, experts, top_k,
                                                   float(limit), ctypes.byref(handle)))
        self.handle = handle
        self.top_k = top_k
        self._dims = (int(hidden), int(intermediate), int(shared_intermediate), int(experts))
        self._bound = None
        self._output = None  # plan-owned output of execute_bound (overwritten by the next call)

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value:
            self._lib.glm53_decode_plan_destroy(handle)
            self.handle = None

    # ---- read-only state of the reference plan (bindings.cpp:584-632)
    def _counters(self) -> N.PlanCounters:
        c = N.PlanCounters()
        N.check(self._lib.glm53_decode_plan_counters(self.handle, ctypes.byref(c)))
        return c

    def _identities(self, which: int) -> list[int]:
        buf = (ctypes.c_uint64 * self._IDENTITY_CAPACITY)()
        count = ctypes.c_int32()
        N.check(self._lib.glm53_decode_plan_identities(self.handle, which, buf, self._IDENTITY_CAPACITY,
                                                       ctypes.byref(count)))
        return [int(buf[i]) for i in range(count.value)]

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
    def weights_bound(self) -> bool:
        return bool(self._counters().weights_bound)

    @property
    def buffer_identities(self) -> list[int]:
        """Device addresses of the plan's scratch buffers: fixed at creation."""
        return self._identities(0)

    @property
    def bound_weight_identities(self) -> list[int]:
        """Device addresses the plan recorded at bind_weights (bank, shared
        expert, router when bound)."""
        return self._identities(1)

    @property
    def bound_weight_identities_stable(self) -> bool:
        """True while every bound tensor still has the storage and contents
        version it had at bind_weights (the reference's identity re-check,
        native_packed_moe_plan.cpp:400-411)."""
        if self._bound is None:
            return False
        tensors = self._bound_tensors(*self._bound[0][:3])  # what the weight objects hold now
        if [(t.data_ptr(), t._version) for t in tensors] != self._bound[2]:
            return False
        return [t.data_ptr() for t in tensors] == self.bound_weight_identities

    def debug_scratch(self, which: int) -> torch.Tensor:
        """A device view of plan scratch after the last call (diagnostics):
        0 SwiGLU rows bf16 [top_k + 1, I] (routed slots, then the shared
        expert: debug_routed_hidden / debug_shared_hidden), 1 ids int32
        [top_k], 2 scores f32 [top_k], 5 shared output bf16 [H]
        (debug_shared_down).  The view aliases the plan's arena."""
        ptr, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
        N.check(self._lib.glm53_decode_plan_scratch(self.handle, int(which), ctypes.byref(ptr), ctypes.byref(nbytes)))
        dtype = {0: torch.bfloat16, 1: torch.int32, 2: torch.float32, 5: torch.bfloat16}[int(which)]
        return _device_view(ptr.value, int(nbytes.value), dtype)

    # ---- execution
    def routed(self, bank, shared, x, ids, scores, out, device):
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        N.check(self._lib.glm53_decode_moe_routed(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                                  N.ptr(x), N.ptr(ids), N.ptr(scores), N.ptr(out),
                                                  N.stream_handle(device)))

    def full(self, bank, shared, router, x, out, ids_out, scores_out, device):
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        r = router.as_c_struct()
        N.check(self._lib.glm53_decode_moe(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                           ctypes.byref(r), N.ptr(x), N.ptr(out), N.ptr(ids_out),
                                           N.ptr(scores_out), N.stream_handle(device)))

    def step(self, bank, shared, router, x, residual, out, stages, device):
        """Decoder-step form: out = T(residual + T(moe(x))) (residual may be
        None); stages is a mask of the router / gate-up / down launches
        (without the router bit, router may be None and the plan's last
        selection is used)."""
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        r = router.as_c_struct() if router is not None else None
        N.check(self._lib.glm53_decode_moe_ex(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                              ctypes.byref(r) if r else None, N.ptr(x), N.ptr(residual),
                                              N.ptr(out), int(stages), N.stream_handle(device)))

    @staticmethod
    def _bound_tensors(bank, shared, router):
        tensors = [bank.gate_up_weight, bank.gate_up_scale_inv, bank.down_weight, bank.down_scale_inv]
        if shared is not None:
            for proj in (shared.gate_proj, shared.up_proj, shared.down_proj):
                tensors += [proj.weight, proj.weight_scale_inv]
        if router is not None:
            tensors += [router.weight, router.e_score_correction_bias]
        return tensors

    def bind_weights(self, bank, shared, router=None) -> None:
        """Record one layer's weights once (bindings.cpp:576-579,
        native_packed_moe_plan.cpp:231-258): the bank, the shared expert
        (None when absent) and optionally the router.  Binding again raises
        RuntimeError.  The plan keeps the weight objects referenced and
        records each tensor's storage identity for execute_bound."""
        b = bank.as_c_struct()
        s = shared.as_c_struct() if shared is not None else None
        r = router.as_c_struct() if router is not None else None
        N.check(self._lib.glm53_decode_plan_bind(self.handle, ctypes.byref(b), ctypes.byref(s) if s else None,
                                                 ctypes.byref(r) if r else None))
        flags = [bank.code_flags()]
        if shared is not None:
            flags += [shared.gate_proj.code_flags(), shared.up_proj.code_flags(), shared.down_proj.code_flags()]
        tensors = self._bound_tensors(bank, shared, router)
        # the weight objects, the bound tensors and the scanned flag tensors the plan points at stay referenced
        self._bound = ((bank, shared, router, flags), tensors, [(t.data_ptr(), t._version) for t in tensors],
                       bank.row_group_log2)

    def _check_bound(self):
        if self._bound is None:
            raise RuntimeError("decode plan weights are not bound")
        tensors = self._bound_tensors(*self._bound[0][:3])  # what the weight objects hold now
        if [(t.data_ptr(), t._version) for t in tensors] != self._bound[2]:
            raise RuntimeError("decode plan bound weight identity changed")
        if self._bound[0][0].row_group_log2 != self._bound[3]:
            raise RuntimeError("the bound bank was re-laid since binding; bind a new plan")

    def _check_x(self, x, who: str) -> None:
        """x must be BF16 on the bound weights' device (the kernels read its
        bytes as BF16 there)."""
        if x.dtype != torch.bfloat16:
            raise ValueError(f"{who}: x must be bfloat16, got {x.dtype}")
        device = self._bound[1][0].device
        if x.device != device:
            raise ValueError(f"{who}: x is on {x.device} but the bound weights are on {device}")

    def _out_for(self, x, out):
        if out is not None:
            return out
        if self._output is None or self._output.device != x.device:
            self._output = torch.empty(self.hidden_size, dtype=torch.bfloat16, device=x.device)
        return self._output

    def execute_bound(self, x, expert_ids, scores, *, out=None) -> torch.Tensor:
        """Decode x [H] (bf16) with the bound weights and caller-chosen
        routing: expert_ids [top_k] int, scores [top_k] f32
        (native_packed_moe_plan.h:48, .cpp:260-280).  Returns `out`, or the
        plan-owned output, which the next call overwrites.  Raises
        RuntimeError when nothing is bound or a bound tensor was replaced or
        modified in place since binding."""
        self._check_bound()
        N.require_device(x, expert_ids, scores)
        self._check_x(x, "execute_bound")
        flat = x.reshape(-1)
        ids = expert_ids.reshape(-1).to(torch.int32).contiguous()
        sc = scores.reshape(-1).to(torch.float32).contiguous()
        if flat.numel() != self.hidden_size or ids.numel() != self.top_k or sc.numel() != self.top_k:
            raise ValueError(f"execute_bound expects x [{self.hidden_size}], {self.top_k} ids and scores")
        dst = self._out_for(x, out)
        N.check(self._lib.glm53_decode_moe_bound_routed(self.handle, N.ptr(flat.contiguous()), N.ptr(ids), N.ptr(sc),
                                                        N.ptr(dst), N.stream_handle(x.device)))
        return dst

    def execute_bound_router(self, x, *, out=None) -> torch.Tensor:
        """Decode x [H] with the bound weights and the bound router (no
        reference counterpart: there the router stays in MLX)."""
        self._check_bound()
        if self._bound[0][2] is None:
            raise RuntimeError("decode plan was bound without a router")
        N.require_device(x)
        self._check_x(x, "execute_bound_router")
        flat = x.reshape(-1)
        if flat.numel() != self.hidden_size:
            raise ValueError(f"execute_bound_router expects x [{self.hidden_size}]")
        dst = self._out_for(x, out)
        N.check(self._lib.glm53_decode_moe_bound(self.handle, N.ptr(flat.contiguous()), N.ptr(dst),
                                                 N.stream_handle(x.device)))
        return dst

    def tune(self, gate_up_rows_per_wave: int = 8, down_rows_per_wg: int = 16) -> None:
        N.check(self._lib.glm53_decode_plan_tune(self.handle, int(gate_up_rows_per_wave), int(down_rows_per_wg)))

    def error_flag(self) -> int:
        value = ctypes.c_int32()
        N.check(self._lib.glm53_decode_plan_error_flag(self.handle, ctypes.byref(value)))
        return int(value.value)


class RoutedDiagnostic:
    """One decode's routed gate/up/SwiGLU boundary with every stage kept
    (native_packed_moe_plan.h:148-183 ``NativePackedMoERoutedDiagnostic``,
    bindings.cpp:634-649): after ``execute(x, expert_ids, gate_up_weight,
    gate_up_scale_inv)`` the properties ``gate``, ``up``, ``sigmoid``,
    ``silu`` and ``hidden`` are bf16 [top_k, I] device views of object-owned
    buffers (fixed addresses; the next execute overwrites them).  Separate
    from DecodePlan, so instrumenting never changes the decode's launches."""

    _STAGES = ("gate", "up", "sigmoid", "silu", "hidden")

    def __init__(self, expert_count: int = 288, *, hidden_size: int = 4096, intermediate_size: int = 2048,
                 top_k: int = DECODE_TOP_K, swiglu_limit: float = 10.0):
        self._lib = N.lib()
        handle = ctypes.c_void_p()
        N.check(self._lib.glm53_routed_diagnostic_create(hidden_size, intermediate_size, expert_count, top_k,
                                                         float(swiglu_limit), ctypes.byref(handle)))
        self.handle = handle
        self.hidden_size, self.intermediate_size, self.top_k = int(hidden_size), int(intermediate_size), int(top_k)

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value:
            self._lib.glm53_routed_diagnostic_destroy(handle)
            self.handle = None

    def execute(self, x, expert_ids, gate_up_weight, gate_up_scale_inv, *, layout="rows") -> torch.Tensor:
        """`layout`: that of gate_up_weight ("rows" for the reference's raw
        arrays; a bank's own ``layout`` when passing its tensors)."""
        N.require_device(x, expert_ids, gate_up_weight, gate_up_scale_inv)
        g = _layout_log2(layout, self.hidden_size, self.intermediate_size)
        flat = x.reshape(-1).contiguous()
        ids = expert_ids.reshape(-1).to(torch.int32).contiguous()
        if flat.numel() != self.hidden_size or ids.numel() != self.top_k:
            raise ValueError(f"expected x [{self.hidden_size}] and {self.top_k} expert ids")
        if gate_up_weight.dtype != torch.uint8 or gate_up_weight.shape[1:] != (2 * self.intermediate_size,
                                                                                self.hidden_size):
            raise ValueError("gate_up_weight must be uint8 [E, 2I, H]")
        N.check(self._lib.glm53_routed_diagnostic_execute(self.handle, N.ptr(flat), N.ptr(ids),
                                                          N.ptr(gate_up_weight.contiguous()),
                                                          N.ptr(gate_up_scale_inv.contiguous()), g,
                                                          N.stream_handle(x.device)))
        return self.hidden

    def _stage(self, which: int) -> torch.Tensor:
        ptr, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
        N.check(self._lib.glm53_routed_diagnostic_stage(self.handle, which, ctypes.byref(ptr), ctypes.byref(nbytes)))
        return _device_view(ptr.value, int(nbytes.value), torch.bfloat16).view(self.top_k, self.intermediate_size)

    gate = property(lambda self: self._stage(0))
    up = property(lambda self: self._stage(1))
    sigmoid = property(lambda self: self._stage(2))
    silu = property(lambda self: self._stage(3))
    hidden = property(lambda self: self._stage(4))

    def _counters(self):
        ex, sb = ctypes.c_uint64(), ctypes.c_uint64()
        N.check(self._lib.glm53_routed_diagnostic_counters(self.handle, ctypes.byref(ex), ctypes.byref(sb)))
        return int(ex.value), int(sb.value)

    @property
    def execution_count(self) -> int:
        return self._counters()[0]

    @property
    def scratch_bytes(self) -> int:
        return self._counters()[1]

    @property
    def buffer_identities(self) -> list[int]:
        return [self._stage(i).data_ptr() for i in range(len(self._STAGES))]


class _ArrayInterface:
    def __init__(self, address: int, count: int, typestr: str):
        self.__cuda_array_interface__ = {"shape": (count,), "typestr": typestr, "data": (address, False),
                                         "version": 2}


def _device_view(address: int, nbytes: int, dtype: torch.dtype) -> torch.Tensor:
    """A tensor over device memory the library owns (no copy; the plan that
    owns the memory must outlive the view)."""
    carrier = {torch.bfloat16: ("<i2", 2), torch.int32: ("<i4", 4), torch.float32: ("<f4", 4)}[dtype]
    view = torch.as_tensor(_ArrayInterface(address, nbytes // carrier[1], carrier[0]), device="cuda")
    return view.view(dtype)


def _c_shared(shared_experts):
    """Shared expert as block-FP8 linears, or None when absent."""
    if shared_experts is None:
        return None
    if not all(hasattr(shared_experts, n) for n in ("gate_proj", "up_proj", "down_proj")):
        raise ValueError("shared expert must expose gate_proj/up_proj/down_proj BlockFP8Linear projections")
    return shared_experts


class PackedFP8MoE(DirectFP8MoE):
    """Exact fused batch-1 decode and Direct semantics over a packed bank.

    One-token calls go through the ``glm53::moe_decode`` custom op (one
    opaque node under torch.compile); prefill keeps the Direct semantics
    (a host readback of the ids per call, as the reference's Direct)."""

    def __init__(self, bank, config, gate, shared_experts):
        torch.nn.Module.__init__(self)
        self.bank = bank
        self.config = config
        self.gate = gate
        self.shared_experts = shared_experts
        self._expert_views = tuple(bank.expert(i, limit=config.swiglu_limit) for i in range(bank.expert_count))
        self._plans: dict = {}
        self._op_key = ops.register_owner(self)

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

    def native_decode(self, x, expert_ids=None, scores=None):
        """The native call behind glm53::moe_decode: x holds one token;
        with expert_ids / scores the caller's routing (the reference's
        execute(x, ids, scores), native_packed_moe_plan.cpp:151), else the
        module's Float32Gate in the router launch."""
        flat = x.reshape(-1).contiguous()
        out = torch.empty_like(flat)
        plan = self._plan(x.device)
        if expert_ids is None:
            plan.full(self.bank, _c_shared(self.shared_experts), self.gate, flat, out, None, None, x.device)
        else:
            ids = expert_ids.reshape(-1).to(torch.int32).contiguous()
            sc = scores.reshape(-1).to(torch.float32).contiguous()
            plan.routed(self.bank, _c_shared(self.shared_experts), flat, ids, sc, out, x.device)
        return out.reshape(x.shape)

    def decode_routed(self, x, expert_ids, scores):
        """Routed + shared decode for externally chosen experts (the
        reference's execute(x, ids, scores), native_packed_moe_plan.cpp:151)."""
        N.require_device(x, expert_ids, scores)
        if expert_ids.numel() != DECODE_TOP_K or scores.numel() != DECODE_TOP_K:
            raise ValueError(f"decode expects {DECODE_TOP_K} expert ids and scores")
        if x.numel() != self.bank.hidden_size:
            raise ValueError(f"decode expects one token of width {self.bank.hidden_size}")
        return torch.ops.glm53.moe_decode(x, self._op_key, expert_ids, scores)

    def forward(self, x):
        flat_x = x.reshape(-1, x.shape[-1])
        if flat_x.shape[0] != 1:
            return super().forward(x)
        if isinstance(self.gate, Float32Gate) and self.gate.top_k == DECODE_TOP_K:
            N.require_device(x)
            return torch.ops.glm53.moe_decode(x, self._op_key, None, None)
        indices, scores = self.gate(x)
        if indices.shape[-1] != DECODE_TOP_K:
            return super().forward(x)
        return self.decode_routed(x, indices, scores)
