"""ctypes binding of libglm53_moe.so (C ABI in include/glm53_moe.h).

The library is the product: there is no Python or CPU fallback.  Loading
fails loudly when the shared library is missing or was not built, and every
entry point rejects tensors that are not on a ROCm device.  Status codes map
to the reference's Python error classes: invalid arguments raise ValueError,
missing backend / bad state / device failures raise RuntimeError
(fp8.py:256-273 of the reference).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("GLM53_MOE_LIB", _PKG / "libglm53_moe.so"))

ABI_VERSION = 2
OK, INVALID_ARGUMENT, BAD_STATE, DEVICE_ERROR = 0, 1, 2, 3
# Expert-matrix layouts (glm53_bank.row_group_log2): 0 = the reference's
# row-major layout, g > 0 = row groups of 2^g rows; TILED is the library's.
ROWS_LAYOUT, TILED_LAYOUT, MAX_ROW_GROUP_LOG2 = 0, 4, 7
REDUCE_GROUPED, REDUCE_DIRECT = 0, 1
STAGE_ROUTER, STAGE_GATE_UP, STAGE_DOWN, STAGE_ALL = 1, 2, 4, 7

_lib = None

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
F32 = ctypes.c_float
SZ = ctypes.c_size_t


class Bank(ctypes.Structure):
    _fields_ = [
        ("gate_up_weight", P),
        ("gate_up_scale_inv", P),
        ("down_weight", P),
        ("down_scale_inv", P),
        ("experts", I64),
        ("hidden", I64),
        ("intermediate", I64),
        ("code_flags", P),
        ("row_group_log2", I32),
    ]


class Linear(ctypes.Structure):
    _fields_ = [("weight", P), ("scale_inv", P), ("out_features", I64), ("in_features", I64), ("code_flags", P)]


class SharedExpert(ctypes.Structure):
    _fields_ = [("gate", Linear), ("up", Linear), ("down", Linear)]


class Router(ctypes.Structure):
    _fields_ = [
        ("weight", P),
        ("bias", P),
        ("experts", I64),
        ("hidden", I64),
        ("top_k", I64),
        ("routed_scaling_factor", F32),
        ("norm_topk_prob", I32),
        ("n_group", I32),
        ("topk_group", I32),
    ]


class PlanCounters(ctypes.Structure):
    _fields_ = [
        ("execution_count", ctypes.c_uint64),
        ("dynamic_allocation_count", ctypes.c_uint64),
        ("host_synchronization_count", ctypes.c_uint64),
        ("static_input_validation_count", ctypes.c_uint64),
        ("dynamic_input_validation_count", ctypes.c_uint64),
        ("scratch_bytes", ctypes.c_uint64),
        ("weights_bound", I32),
        ("router_bound", I32),
    ]


_SIGNATURES = {
    "glm53_last_error": (ctypes.c_char_p, []),
    "glm53_abi_version": (ctypes.c_int, []),
    "glm53_e4m3_scan_codes": (ctypes.c_int, [P, I64, P, P]),
    "glm53_bank_create": (ctypes.c_int, [P, P, P]),
    "glm53_bank_import": (ctypes.c_int, [P, I32, P, P]),
    "glm53_bank_destroy": (None, [P]),
    "glm53_relayout_weights": (ctypes.c_int, [P, P, I64, I64, I64, I32, I32, P]),
    "glm53_fp8_linear_workspace_bytes": (SZ, [I64, I64, I64]),
    "glm53_fp8_linear": (ctypes.c_int, [P, I64, I64, P, I64, P, P, P, P, SZ, P]),
    "glm53_router_workspace_bytes": (SZ, [I64, I64, I64]),
    "glm53_router_topk": (ctypes.c_int, [P, P, I64, P, P, P, SZ, P]),
    "glm53_decode_plan_create": (ctypes.c_int, [I64, I64, I64, I64, I64, F32, P]),
    "glm53_decode_plan_destroy": (None, [P]),
    "glm53_decode_moe_routed": (ctypes.c_int, [P, P, P, P, P, P, P, P]),
    "glm53_decode_moe": (ctypes.c_int, [P, P, P, P, P, P, P, P, P]),
    "glm53_decode_moe_ex": (ctypes.c_int, [P, P, P, P, P, P, P, I32, P]),
    "glm53_decode_plan_bind": (ctypes.c_int, [P, P, P, P]),
    "glm53_decode_moe_bound": (ctypes.c_int, [P, P, P, P]),
    "glm53_decode_moe_bound_routed": (ctypes.c_int, [P, P, P, P, P, P]),
    "glm53_decode_plan_tune": (ctypes.c_int, [P, I32, I32]),
    "glm53_decode_plan_scratch": (ctypes.c_int, [P, I32, P, P]),
    "glm53_decode_plan_error_flag": (ctypes.c_int, [P, P]),
    "glm53_decode_plan_counters": (ctypes.c_int, [P, P]),
    "glm53_decode_plan_identities": (ctypes.c_int, [P, I32, P, I32, P]),
    "glm53_decode_moe_static": (ctypes.c_int, [I64, I64, I64, I64, F32, P, P, P, P, P, P, P]),
    "glm53_routed_diagnostic_create": (ctypes.c_int, [I64, I64, I64, I64, F32, P]),
    "glm53_routed_diagnostic_destroy": (None, [P]),
    "glm53_routed_diagnostic_execute": (ctypes.c_int, [P, P, P, P, P, I32, P]),
    "glm53_routed_diagnostic_stage": (ctypes.c_int, [P, I32, P, P]),
    "glm53_routed_diagnostic_counters": (ctypes.c_int, [P, P, P]),
    "glm53_route_plan_workspace_bytes": (SZ, [I64, I64]),
    "glm53_route_plan": (ctypes.c_int, [P, P, I64, I64, I64, I64, P, P, P, P, P, P, P, P, P, P, I64, P, P, SZ, P]),
    "glm53_grouped_linear_workspace_bytes": (SZ, [I64, I64]),
    "glm53_grouped_linear": (ctypes.c_int, [P, I64, P, I64, I64, P, P, P, I64, P, P, P, I64, I64, P, P, SZ, P]),
    "glm53_activate_gate_up": (ctypes.c_int, [P, I64, I64, F32, P, P]),
    "glm53_sigmoid_bf16": (ctypes.c_int, [P, I64, P, P]),
    "glm53_restore_and_reduce": (ctypes.c_int, [P, P, P, I64, I64, I64, P, P, P]),
    "glm53_direct_order_reduce": (ctypes.c_int, [P, P, P, P, I64, I64, I64, P, P, P]),
    "glm53_split_activations": (ctypes.c_int, [P, I64, I64, I64, P, P, P, P]),
    "glm53_prefill_plan_create": (ctypes.c_int, [I64, I64, I64, I64, I64, I64, F32, P]),
    "glm53_prefill_plan_destroy": (None, [P]),
    "glm53_prefill_moe": (ctypes.c_int, [P, P, P, P, P, I64, P, P, I32, P, P]),
    "glm53_prefill_moe_hc": (ctypes.c_int, [P, P, P, P, P, I64, P, P, I32, P, P, P, P, P]),
    "glm53_prefill_plan_status": (ctypes.c_int, [P, P]),
    "glm53_prefill_plan_scratch": (ctypes.c_int, [P, I32, P, P]),
    "glm53_prefill_plan_counters": (ctypes.c_int, [P, P]),
    "glm53_prefill_plan_identities": (ctypes.c_int, [P, P, I32, P]),
    "glm53_synth_fp8": (ctypes.c_int, [P, P, I64, I64, ctypes.c_uint64, F32, P]),
    "glm53_synth_f32": (ctypes.c_int, [P, I64, ctypes.c_uint64, F32, F32, F32, I32, P]),
    "glm53_synth_bf16": (ctypes.c_int, [P, I64, ctypes.c_uint64, F32, P]),
    "glm53_synth_fp8_batched": (ctypes.c_int, [P, P, I64, I64, I64, I64, I64, ctypes.c_uint64, F32, I32, P]),
    "glm53_synth_step_input": (ctypes.c_int, [P, I64, ctypes.c_uint64, F32, P, P]),
    "glm53_probe_read": (ctypes.c_int, [P, I64, P, I32, P]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def load_library(path: Path | None = None):
    """Load and type the shared library (no device work)."""
    target = Path(path) if path is not None else LIB_PATH
    if not target.exists():
        raise RuntimeError(
            f"{target} is missing: build the HIP library first "
            "(python glm53-flash-mlx_amd/build.py or __graft_entry__.build())"
        )
    handle = ctypes.CDLL(str(target))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def lib():
    global _lib
    if _lib is None:
        _lib = load_library()
    return _lib


def check(status: int) -> None:
    if status == OK:
        return
    message = lib().glm53_last_error().decode(errors="replace")
    if status == INVALID_ARGUMENT:
        raise ValueError(message)
    raise RuntimeError(message)


def stream_handle(device: torch.device | None = None) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device(*tensors: torch.Tensor) -> None:
    if not torch.cuda.is_available():
        raise RuntimeError("the glm53 MI355X MoE path requires a ROCm GPU; no CPU fallback exists")
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("expected a tensor on the ROCm device, got one on the CPU")


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)


def relayout(src: torch.Tensor, dst: torch.Tensor, from_log2: int, to_log2: int) -> None:
    """Re-lay the expert matrices of a uint8 [E, rows, cols] tensor from one
    layout to another into `dst` (same shape, no overlap) on the current
    stream (glm53_relayout_weights)."""
    require_device(src, dst)
    if src.dtype != torch.uint8 or src.dim() != 3 or dst.shape != src.shape or dst.dtype != torch.uint8:
        raise ValueError("relayout needs two uint8 [experts, rows, cols] tensors of one shape")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("relayout needs contiguous tensors")
    experts, rows, cols = src.shape
    check(lib().glm53_relayout_weights(ptr(src), ptr(dst), experts, rows, cols, int(from_log2), int(to_log2),
                                       stream_handle(src.device)))


def scan_codes(codes: torch.Tensor) -> torch.Tensor:
    """Device int32 flag: 1 when codes hold E4M3 0x7F / 0xFF (see
    glm53_e4m3_scan_codes)."""
    flag = torch.empty(1, dtype=torch.int32, device=codes.device)
    c = codes.contiguous()
    check(lib().glm53_e4m3_scan_codes(ptr(c), c.numel(), ptr(flag), stream_handle(codes.device)))
    return flag
