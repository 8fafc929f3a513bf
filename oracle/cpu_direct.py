"""Binding of glm53_cpu_direct.c -- the benchmark's CPU comparator.

MEASUREMENT AND TEST INFRASTRUCTURE ONLY.  ``bench.py``'s cpu_baseline leg
times it on the GPU box's host cores and ``tests/`` check it against the
float64 oracle (``oracle.py``); the product package never imports it.

It evaluates the reference's Direct FP8 MoE (fp8.py:343-400, the FP32 router
of patch.py:131-142) with FP32 accumulation, OpenMP threads and AVX2 FMA:
the "MLX CPU-stream Direct" comparator of the task, restated in C because
MLX is not installable here and the reference has no CPU FP8 path.  BF16
tensors are carried as ``np.uint16`` bit patterns, banks in the reference
layout (packed.py:782-850).
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libglm53_cpu_direct.so"
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            subprocess.run(["make", "-s", "-C", str(_HERE), _LIB_PATH.name], check=True)
        L = ctypes.CDLL(str(_LIB_PATH))
        P, I64, F32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        L.glm53c_linear.argtypes = [P, I64, I64, P, I64, P, P, I64]
        L.glm53c_router.argtypes = [P, I64, I64, P, P, I64, I64, F32, ctypes.c_int, P, P]
        L.glm53c_direct_moe.argtypes = [P, I64, I64, I64, I64, P, P, P, P, P, P, P, P, P, P, P, P, I64, F32, P]
        L.glm53c_num_threads.restype = ctypes.c_int
        L.glm53c_decode_codes.argtypes = [P, I64, P]
        _lib = L
    return _lib


def _p(a):
    return ctypes.c_void_p(0 if a is None else a.ctypes.data)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def num_threads() -> int:
    return int(lib().glm53c_num_threads())


def decode_codes(codes) -> np.ndarray:
    """The comparator's E4M3 decode of each code (float32)."""
    c = _c(codes, np.uint8)
    out = np.zeros(c.shape, dtype=np.float32)
    lib().glm53c_decode_codes(_p(c), c.size, _p(out))
    return out


def linear(x_bits, weight, scale_inv):
    """block_fp8_linear (fp8.py:254-299) with FP32 accumulation: bf16 bits
    [..., K] x u8 [N, K] (f32 block scales) -> bf16 bits [..., N]."""
    x = _c(x_bits, np.uint16)
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    w, s = _c(weight, np.uint8), _c(scale_inv, np.float32)
    n = w.shape[0]
    y = np.zeros((x2.shape[0], n), dtype=np.uint16)
    lib().glm53c_linear(_p(x2), x2.shape[0], k, _p(w), n, _p(s), _p(y), n)
    return y.reshape(*x.shape[:-1], n)


def router(x_bits, weight, bias, *, top_k=8, routed_scaling_factor=1.0, norm_topk_prob=True):
    """Float32Gate (patch.py:131-142) with FP32 logits: (ids int32 [T, k],
    scores f32 [T, k])."""
    x = _c(x_bits, np.uint16)
    h = x.shape[-1]
    x2 = x.reshape(-1, h)
    w, b = _c(weight, np.float32), _c(bias, np.float32)
    t = x2.shape[0]
    ids = np.zeros((t, top_k), dtype=np.int32)
    sc = np.zeros((t, top_k), dtype=np.float32)
    lib().glm53c_router(_p(x2), t, h, _p(w), _p(b), w.shape[0], top_k, float(routed_scaling_factor),
                        int(bool(norm_topk_prob)), _p(ids), _p(sc))
    return ids, sc


def direct_moe(x_bits, bank, ids, scores, limit, shared=None):
    """DirectFP8MoE.__call__ (fp8.py:343-400) on given routes: bank with the
    reference-layout arrays gate_up_weight, gate_up_scale_inv, down_weight,
    down_scale_inv and intermediate_size; shared (or None) with (weight,
    scale) pairs gate, up, down.  One token with 8 routes takes the decode
    combine (FP32 slot order), more tokens the ascending-expert BF16 one."""
    x = _c(x_bits, np.uint16)
    h = x.shape[-1]
    x2 = x.reshape(-1, h)
    idx = _c(ids, np.int32)
    k = idx.shape[-1]
    sc = _c(scores, np.float32)
    gu, gus = _c(bank.gate_up_weight, np.uint8), _c(bank.gate_up_scale_inv, np.float32)
    dw, dws = _c(bank.down_weight, np.uint8), _c(bank.down_scale_inv, np.float32)
    if shared is not None:
        sg, sgs = (_c(shared.gate[0], np.uint8), _c(shared.gate[1], np.float32))
        su, sus = (_c(shared.up[0], np.uint8), _c(shared.up[1], np.float32))
        sd, sds = (_c(shared.down[0], np.uint8), _c(shared.down[1], np.float32))
        inter_s = sg.shape[0]
    else:
        sg = sgs = su = sus = sd = sds = None
        inter_s = 0
    out = np.zeros_like(x2)
    lib().glm53c_direct_moe(_p(x2), x2.shape[0], h, int(bank.intermediate_size), k, _p(idx), _p(sc), _p(gu), _p(gus),
                            _p(dw), _p(dws), _p(sg), _p(sgs), _p(su), _p(sus), _p(sd), _p(sds), inter_s,
                            float(limit), _p(out))
    return out.reshape(x.shape)
