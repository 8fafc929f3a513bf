"""CPU oracle for the FP8 block-scaled MoE path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker or the
timed CPU comparator.  The product package never imports it; its HIP path
fails loudly when its native library is missing.

This module restates the reference's Direct semantics (the "MLX Direct
oracle" of the task) on the CPU.  Heavy contractions run in the C
restatement ``glm53_oracle.c`` (double-precision sums rounded to FP32 and
then BF16 where the reference rounds); composition and integer plans are
NumPy.  BF16 tensors are carried as ``np.uint16`` bit patterns.

Parity pins (see tests/test_oracle_*.py):
  * E4M3 decode: all 256 codes against the reference LUT values
    (fixture tests/golden/e4m3_lut.json) and torch.float8_e4m3fn.
  * linear: float64 closed form and the reference KAT
    (tests/test_fp8_metal.py:23-39 of the reference).
  * sigmoid/SwiGLU: the SHA-256 of the reference's exhaustive BF16 sigmoid
    sweep (bench-results/m3ultra512-native-routed-sigmoid-formula-sweep-
    20260907.json).
  * router weights: the reference KAT (tests/test_grouped_divergence.py:
    181-199); selection: brute force (parity of selection against mlx-vlm is
    unpinned, see the module docstring of ``router``).
  * tile plan: the reference KAT (tests/test_fp8_metal.py:201-238) and the
    invariants of scripts/probe_grouped_fp8_moe.py:103-166.
  * Direct-order reduce: independent scatter-add formulation
    (tests/test_grouped_divergence.py:233-254).
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path
from types import SimpleNamespace

import numpy as np

BLOCK = 128
_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "libglm53_oracle.so"
_lib = None


def build(force: bool = True) -> Path:
    """Compile the C restatement with gcc (OpenMP, AVX2)."""
    if force or not _LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build(force=False)
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


def _declare(L):
    P = ctypes.c_void_p
    I64 = ctypes.c_int64
    L.glm53o_e4m3_value.restype = ctypes.c_double
    L.glm53o_e4m3_value.argtypes = [ctypes.c_uint8]
    L.glm53o_e4m3_lut.argtypes = [P]
    L.glm53o_fp8_linear.argtypes = [P, I64, I64, I64, P, I64, P, I64, P, I64]
    L.glm53o_f32_linear.argtypes = [P, I64, I64, P, I64, P]
    L.glm53o_sigmoid_bf16.restype = ctypes.c_uint16
    L.glm53o_sigmoid_bf16.argtypes = [ctypes.c_uint16]
    L.glm53o_swiglu.argtypes = [P, P, I64, ctypes.c_float, P]
    L.glm53o_router.argtypes = [P, I64, I64, P, P, I64, I64, ctypes.c_float, ctypes.c_int, I64, I64, P, P, P]
    L.glm53o_weighted_reduction.argtypes = [P, P, I64, I64, P]
    L.glm53o_add_bf16.argtypes = [P, P, I64, P]
    L.glm53o_hc_expand.argtypes = [P, P, P, P, I64, I64, P]
    L.glm53o_direct_order_reduce.argtypes = [P, P, P, I64, I64, I64, P]
    L.glm53o_restore_and_reduce.argtypes = [P, P, P, I64, I64, I64, P]
    L.glm53o_num_threads.restype = ctypes.c_int
    L.glm53o_set_num_threads.argtypes = [ctypes.c_int]


def _p(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data)


def num_threads() -> int:
    return int(lib().glm53o_num_threads())


def set_num_threads(n: int) -> None:
    lib().glm53o_set_num_threads(int(n))


# ------------------------------------------------------------------ BF16 ---

def f32_to_bf16(values) -> np.ndarray:
    """Round-to-nearest-even FP32 -> BF16 bit patterns (np.uint16)."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ E4M3 ---

def e4m3_lut() -> np.ndarray:
    """fp8.py:22-39: the 256-entry decode table (0x7F/0xFF -> +-480)."""
    out = np.zeros(256, dtype=np.float32)
    lib().glm53o_e4m3_lut(_p(out))
    return out


def quantize_e4m3_blocks(w: np.ndarray):
    """Quantise FP32 [N, K] to E4M3 codes with FP32 128x128 block scales.

    scale_inv = amax / 448 per block; codes = RNE(w / scale_inv) to the E4M3
    grid, saturated to +-448 (never the 0x7F / 0xFF codes).  This is the
    synthetic-weight recipe of the task (checkpoint-style block FP8).
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    sr, sc = math.ceil(n / BLOCK), math.ceil(k / BLOCK)
    scale = np.zeros((sr, sc), dtype=np.float32)
    codes = np.zeros((n, k), dtype=np.uint8)
    lut = e4m3_lut()
    positive = lut[:127].astype(np.float64)  # codes 0x00..0x7E, ascending
    for i in range(sr):
        for j in range(sc):
            blk = w[i * BLOCK:(i + 1) * BLOCK, j * BLOCK:(j + 1) * BLOCK]
            amax = float(np.max(np.abs(blk))) if blk.size else 0.0
            s = np.float32(amax / 448.0) if amax > 0 else np.float32(1.0)
            scale[i, j] = s
            q = blk.astype(np.float64) / np.float64(s)
            mag = np.minimum(np.abs(q), 448.0)
            idx = np.searchsorted(positive, mag)  # first >= mag
            idx = np.clip(idx, 1, 126)
            lo, hi = positive[idx - 1], positive[idx]
            pick_hi = (hi - mag < mag - lo) | ((hi - mag == mag - lo) & (idx % 2 == 0))
            code = np.where(pick_hi, idx, idx - 1)
            code = np.where(mag >= positive[126], 126, code)
            code = np.where(mag == 0, 0, code)
            code = code.astype(np.uint8) | np.where(q < 0, 0x80, 0).astype(np.uint8)
            codes[i * BLOCK:(i + 1) * BLOCK, j * BLOCK:(j + 1) * BLOCK] = code
    return codes, scale


def dequantize(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Dense float64 expansion (test-only closed form)."""
    lut = np.array([lib().glm53o_e4m3_value(c) for c in range(256)], dtype=np.float64)
    n, k = codes.shape
    s = np.repeat(np.repeat(scale.astype(np.float64), BLOCK, 0), BLOCK, 1)[:n, :k]
    return lut[codes] * s


# ---------------------------------------------------------------- linear ---

def fp8_linear(x_bits: np.ndarray, weight: np.ndarray, scale_inv: np.ndarray) -> np.ndarray:
    """fp8.py:254-299 ``block_fp8_linear`` on BF16 bit patterns."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    lead = x.shape[:-1]
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    w = np.ascontiguousarray(weight, dtype=np.uint8)
    s = np.ascontiguousarray(scale_inv, dtype=np.float32)
    n = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"input width {k} != weight width {w.shape[1]}")
    if s.shape != (math.ceil(n / BLOCK), math.ceil(k / BLOCK)):
        raise ValueError(f"scale shape {s.shape} != block128 shape")
    m = x2.shape[0]
    y = np.zeros((m, n), dtype=np.uint16)
    lib().glm53o_fp8_linear(_p(x2), m, k, k, _p(w), n, _p(s), s.shape[1], _p(y), n)
    return y.reshape(*lead, n)


# ---------------------------------------------------------------- SwiGLU ---

def sigmoid_bf16(g_bits: np.ndarray) -> np.ndarray:
    """MLX BF16 sigmoid (stepwise BF16, fast::exp midpoint at -6.84375)."""
    g = np.ascontiguousarray(g_bits, dtype=np.uint16).reshape(-1)
    out = np.array([lib().glm53o_sigmoid_bf16(int(v)) for v in g], dtype=np.uint16)
    return out.reshape(np.shape(g_bits))


def swiglu(gate_bits: np.ndarray, up_bits: np.ndarray, limit: float) -> np.ndarray:
    g = np.ascontiguousarray(gate_bits, dtype=np.uint16)
    u = np.ascontiguousarray(up_bits, dtype=np.uint16)
    if g.shape != u.shape:
        raise ValueError("gate/up shape mismatch")
    out = np.zeros_like(g)
    lib().glm53o_swiglu(_p(g), _p(u), g.size, float(limit), _p(out))
    return out


# ---------------------------------------------------------------- router ---

def router(x_bits, weight, bias, *, top_k=8, routed_scaling_factor=1.0, norm_topk_prob=True,
           return_choice=False, n_group=1, topk_group=1):
    """patch.py:131-142 FP32 router + DeepSeek-V3 aux-loss-free selection.

    Selection parity with mlx-vlm's ``group_expert_select`` is unpinned (the
    module is absent); the rule here is the published one -- with n_group > 1
    groups of consecutive experts scored by the sum of their two largest
    biased scores, all but the topk_group best zeroed -- and the tie policy
    (biased score desc, expert id asc; equal group scores: lower group kept).
    ``choice`` (return_choice) is the biased score after the group limit.
    """
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    lead = x.shape[:-1]
    h = x.shape[-1]
    x2 = x.reshape(-1, h)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    b = np.ascontiguousarray(bias, dtype=np.float32)
    e = w.shape[0]
    t = x2.shape[0]
    ids = np.zeros((t, top_k), dtype=np.int32)
    scores = np.zeros((t, top_k), dtype=np.float32)
    choice = np.zeros((t, e), dtype=np.float32)
    lib().glm53o_router(_p(x2), t, h, _p(w), _p(b), e, top_k, float(routed_scaling_factor),
                        int(bool(norm_topk_prob)), int(n_group), int(topk_group), _p(ids), _p(scores), _p(choice))
    ids = ids.reshape(*lead, top_k)
    scores = scores.reshape(*lead, top_k)
    if return_choice:
        return ids, scores, choice.reshape(*lead, e)
    return ids, scores


def router_weights_for(x_bits, weight, ids, *, routed_scaling_factor=1.0, norm_topk_prob=True):
    """Scores for given expert ids (scripts/sweep_grouped_fp8_suffix.py:84-91)."""
    x = bf16_to_f32(x_bits).astype(np.float64)
    logits = (x @ np.asarray(weight, dtype=np.float64).T).astype(np.float32)
    sig = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32)
    picked = np.take_along_axis(sig, np.asarray(ids), axis=-1)
    if picked.shape[-1] > 1 and norm_topk_prob:
        total = np.zeros(picked.shape[:-1], dtype=np.float32)
        for s in range(picked.shape[-1]):
            total = (total + picked[..., s]).astype(np.float32)
        picked = (picked / total[..., None]).astype(np.float32)
    return (picked * np.float32(routed_scaling_factor)).astype(np.float32)


# ------------------------------------------------------------------ bank ---

def bank_shapes(experts: int, hidden: int, intermediate: int):
    """packed.py:782-850 bank layout contract."""
    sr = math.ceil(intermediate / BLOCK)
    sh = math.ceil(hidden / BLOCK)
    return {
        "gate_up_weight": (experts, 2 * intermediate, hidden),
        "gate_up_scale_inv": (experts, 2 * sr, sh),
        "down_weight": (experts, hidden, intermediate),
        "down_scale_inv": (experts, sh, sr),
    }


def expert_matrices(bank, e: int):
    """Per-expert gate/up/down views of a bank (packed.py:702-744)."""
    inter = bank.intermediate_size
    sr = math.ceil(inter / BLOCK)
    return SimpleNamespace(
        gate=(bank.gate_up_weight[e, :inter], bank.gate_up_scale_inv[e, :sr]),
        up=(bank.gate_up_weight[e, inter:], bank.gate_up_scale_inv[e, sr:2 * sr]),
        down=(bank.down_weight[e], bank.down_scale_inv[e]),
    )


def expert_forward(x_bits, mats, limit):
    """fp8.py:329-340 ``DirectFP8Expert``: down(silu(min(g,L)) * clip(u,L))."""
    g = fp8_linear(x_bits, *mats.gate)
    u = fp8_linear(x_bits, *mats.up)
    hid = swiglu(g, u, limit)
    return fp8_linear(hid, *mats.down)


def shared_forward(x_bits, shared, limit):
    """patch.py:114-129 ``ClampedMLP`` over block-FP8 linears."""
    if shared is None:
        return None
    mats = SimpleNamespace(gate=shared.gate, up=shared.up, down=shared.down)
    return expert_forward(x_bits, mats, limit)


def _weighted_reduction(down_bits, scores):
    d = np.ascontiguousarray(down_bits, dtype=np.uint16)
    s = np.ascontiguousarray(scores, dtype=np.float32)
    out = np.zeros(d.shape[1], dtype=np.uint16)
    lib().glm53o_weighted_reduction(_p(d), _p(s), d.shape[0], d.shape[1], _p(out))
    return out


def hc_expand(moe, residual, post, comb):
    """native_indexer_plan.metal:2362-2388: moe bf16 [T, H], residual bf16
    [T, 4, H], post f32 [T, 4], comb f32 [T, 4, 4] -> bf16 [T, 4, H]."""
    m = np.ascontiguousarray(moe, dtype=np.uint16)
    r = np.ascontiguousarray(residual, dtype=np.uint16)
    po = np.ascontiguousarray(post, dtype=np.float32)
    co = np.ascontiguousarray(comb, dtype=np.float32)
    t, h = m.shape
    out = np.zeros((t, 4, h), dtype=np.uint16)
    lib().glm53o_hc_expand(_p(m), _p(r), _p(po), _p(co), t, h, _p(out))
    return out


def add_bf16(a, b):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.zeros_like(a)
    lib().glm53o_add_bf16(_p(a), _p(b), a.size, _p(out))
    return out


def decode_moe(x_bits, bank, ids, scores, limit, shared=None, return_stages=False):
    """Batch-1 decode: packed.py:896-923 == fp8.py:372-383 (Direct decode).

    hidden[s] = swiglu(T(gate), T(up)); down[s] = T(down_s . hidden[s]);
    routed = T(sum_s float(down[s]) * score[s]) in slot order; out =
    T(routed + shared).
    """
    x = np.ascontiguousarray(x_bits, dtype=np.uint16).reshape(-1)
    ids = np.asarray(ids).reshape(-1)
    scores = np.asarray(scores, dtype=np.float32).reshape(-1)
    hidden = []
    downs = []
    for e in ids:
        mats = expert_matrices(bank, int(e))
        g = fp8_linear(x[None], *mats.gate)
        u = fp8_linear(x[None], *mats.up)
        hid = swiglu(g, u, limit)
        hidden.append(hid[0])
        downs.append(fp8_linear(hid, *mats.down)[0])
    hidden = np.stack(hidden)
    downs = np.stack(downs)
    routed = _weighted_reduction(downs, scores)
    out = routed
    shared_out = None
    if shared is not None:
        shared_out = shared_forward(x[None], shared, limit)[0]
        out = add_bf16(routed, shared_out)
    if return_stages:
        return out, SimpleNamespace(hidden=hidden, down=downs, routed=routed, shared=shared_out)
    return out


def direct_moe(x_bits, bank, ids, scores, limit, shared=None):
    """fp8.py:364-397 ``DirectFP8MoE.__call__`` semantics over a bank.

    Decode (one row, k=8) uses the ordered FP32 slot reduction; prefill
    visits experts in ascending id and accumulates T(out * w) into a BF16
    result (native_indexer_plan.metal:2174-2207 restates the order).
    """
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    h = x.shape[-1]
    flat = x.reshape(-1, h)
    k = np.asarray(ids).shape[-1]
    routes = np.asarray(ids).reshape(-1, k)
    flat_scores = np.asarray(scores, dtype=np.float32).reshape(-1, k)
    if flat.shape[0] == 1 and k == 8:
        return decode_moe(flat[0], bank, routes[0], flat_scores[0], limit, shared).reshape(x.shape)
    t = flat.shape[0]
    route_out = np.zeros((t * k, h), dtype=np.uint16)
    for e in np.unique(routes):
        rows, slots = np.nonzero(routes == e)
        out = expert_forward(flat[rows], expert_matrices(bank, int(e)), limit)
        route_out[rows * k + slots] = out
    result = direct_order_reduce(route_out, routes, flat_scores)
    if shared is not None:
        result = add_bf16(result, shared_forward(flat, shared, limit))
    return result.reshape(x.shape)


def direct_order_reduce(route_out, ids, scores):
    r = np.ascontiguousarray(route_out, dtype=np.uint16)
    i = np.ascontiguousarray(ids, dtype=np.int32)
    s = np.ascontiguousarray(scores, dtype=np.float32)
    t, k = i.shape
    h = r.shape[1]
    out = np.zeros((t, h), dtype=np.uint16)
    lib().glm53o_direct_order_reduce(_p(r), _p(i), _p(s), t, k, h, _p(out))
    return out


# ------------------------------------------------------------ grouped path ---

def build_route_plan(ids, scores):
    """grouped_fp8.py:157-170: stable expert sort of the flat routes."""
    ids = np.asarray(ids)
    k = ids.shape[-1]
    flat_ids = ids.reshape(-1).astype(np.int64)
    order = np.argsort(flat_ids, kind="stable")
    inverse = np.argsort(order, kind="stable")
    token_ids = order // k
    return SimpleNamespace(
        order=order,
        inverse=inverse,
        token_ids=token_ids,
        sorted_experts=flat_ids[order],
        sorted_scores=np.asarray(scores, dtype=np.float32).reshape(-1)[order],
    )


def build_grouped_tile_plan(sorted_experts, expert_count: int, tile_rows: int = 32):
    """grouped_fp8.py:173-203: expert-aligned tile descriptors.

    capacity = ceil(R / tile_rows) + E; an unused slot has start = R, len 0.
    """
    se = np.asarray(sorted_experts, dtype=np.int64)
    routes = se.size
    counts = np.bincount(se, minlength=expert_count)[:expert_count].astype(np.int64)
    route_offsets = np.concatenate([[0], np.cumsum(counts)])
    tile_counts = (counts + tile_rows - 1) // tile_rows
    tile_offsets = np.concatenate([[0], np.cumsum(tile_counts)])
    slots = (routes + tile_rows - 1) // tile_rows + expert_count
    experts = np.zeros(slots, dtype=np.int64)
    starts = np.full(slots, routes, dtype=np.int64)
    lengths = np.zeros(slots, dtype=np.int64)
    d = 0
    for e in range(expert_count):
        for local in range(int(tile_counts[e])):
            start = route_offsets[e] + local * tile_rows
            experts[d] = e
            starts[d] = start
            lengths[d] = min(tile_rows, route_offsets[e + 1] - start)
            d += 1
    return SimpleNamespace(experts=experts, starts=starts, lengths=lengths,
                           route_offsets=route_offsets, tile_offsets=tile_offsets)


def grouped_linear(sorted_x, sorted_experts, weight, scale_inv):
    """grouped_fp8.py:206-262: row r uses expert sorted_experts[r]."""
    x = np.ascontiguousarray(sorted_x, dtype=np.uint16)
    se = np.asarray(sorted_experts)
    n = weight.shape[1]
    out = np.zeros((x.shape[0], n), dtype=np.uint16)
    for e in np.unique(se):
        rows = np.nonzero(se == e)[0]
        out[rows] = fp8_linear(x[rows], weight[int(e)], scale_inv[int(e)])
    return out


def activate_gate_up(gate_up_bits, intermediate_size: int, limit: float):
    """grouped_fp8.py:265-270."""
    g = np.ascontiguousarray(gate_up_bits[:, :intermediate_size])
    u = np.ascontiguousarray(gate_up_bits[:, intermediate_size:])
    return swiglu(g, u, limit)


def restore_and_reduce(sorted_out, sorted_scores, inverse, tokens, top_k):
    """grouped_fp8.py:273-276 (FP32 products, FP32 slot-order sum)."""
    so = np.ascontiguousarray(sorted_out, dtype=np.uint16)
    ss = np.ascontiguousarray(sorted_scores, dtype=np.float32)
    inv = np.ascontiguousarray(inverse, dtype=np.int64)
    h = so.shape[1]
    out = np.zeros((tokens, h), dtype=np.uint16)
    lib().glm53o_restore_and_reduce(_p(so), _p(ss), _p(inv), tokens, top_k, h, _p(out))
    return out


def grouped_moe(x_bits, bank, ids, scores, limit, shared=None, reduction="grouped"):
    """grouped_fp8.py:294-321 ``grouped_from_routes`` (+ shared expert).

    reduction="grouped": FP32 slot-order reduce (grouped_fp8.py:273-276);
    reduction="direct": ascending-expert BF16 reduce (the exact Direct order,
    native_indexer_plan.metal:2174-2207).
    """
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    h = x.shape[-1]
    flat = x.reshape(-1, h)
    ids = np.asarray(ids)
    k = ids.shape[-1]
    flat_ids = ids.reshape(-1, k)
    plan = build_route_plan(flat_ids, scores)
    sorted_x = flat[plan.token_ids]
    gate_up = grouped_linear(sorted_x, plan.sorted_experts, bank.gate_up_weight, bank.gate_up_scale_inv)
    hidden = activate_gate_up(gate_up, bank.intermediate_size, limit)
    down = grouped_linear(hidden, plan.sorted_experts, bank.down_weight, bank.down_scale_inv)
    t = flat.shape[0]
    if reduction == "grouped":
        result = restore_and_reduce(down, plan.sorted_scores, plan.inverse, t, k)
    else:
        route_out = down[plan.inverse]
        result = direct_order_reduce(route_out, flat_ids, np.asarray(scores, np.float32).reshape(-1, k))
    if shared is not None:
        result = add_bf16(result, shared_forward(flat, shared, limit))
    return result.reshape(x.shape)


def moe_reductions(x_bits, bank, ids, scores, limit, shared=None):
    """{"direct": direct_moe(...), "grouped": grouped_moe(..., "grouped")}
    from one pass over the experts: both reductions combine the same
    per-route outputs (each route's expert output is the exactly rounded
    sum in either contraction tree), Direct in ascending expert order with
    BF16 accumulation (fp8.py:384-397), grouped as the FP32 slot-order sum
    (grouped_fp8.py:273-276), then T(+ shared) (packed.py:922)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    h = x.shape[-1]
    flat = x.reshape(-1, h)
    k = np.asarray(ids).shape[-1]
    routes = np.asarray(ids).reshape(-1, k)
    flat_scores = np.asarray(scores, dtype=np.float32).reshape(-1, k)
    t = flat.shape[0]
    route_out = np.zeros((t * k, h), dtype=np.uint16)
    for e in np.unique(routes):
        rows, slots = np.nonzero(routes == e)
        route_out[rows * k + slots] = expert_forward(flat[rows], expert_matrices(bank, int(e)), limit)
    out = {"direct": direct_order_reduce(route_out, routes, flat_scores),
           "grouped": restore_and_reduce(route_out, flat_scores.reshape(-1), np.arange(t * k), t, k)}
    if shared is not None:
        sh = shared_forward(flat, shared, limit)
        out = {name: add_bf16(v, sh) for name, v in out.items()}
    return {name: v.reshape(x.shape) for name, v in out.items()}


# ------------------------------------------------------------- metrics ---

def compare(actual_bits, expected_bits):
    """Parity statistics on BF16 outputs: max-abs-rel and cosine."""
    a = bf16_to_f32(actual_bits).astype(np.float64).reshape(-1)
    e = bf16_to_f32(expected_bits).astype(np.float64).reshape(-1)
    diff = np.abs(a - e)
    scale = max(float(np.max(np.abs(e))), 1e-30)
    denom = float(np.linalg.norm(a) * np.linalg.norm(e))
    cos = float(np.dot(a, e) / denom) if denom > 0 else (1.0 if np.array_equal(a, e) else 0.0)
    return {
        "max_abs": float(diff.max()) if diff.size else 0.0,
        "max_abs_rel": float(diff.max() / scale) if diff.size else 0.0,
        "cosine": cos,
        "bit_exact_fraction": float(np.mean(np.asarray(actual_bits).reshape(-1) == np.asarray(expected_bits).reshape(-1))) if diff.size else 1.0,
        "allclose_0_02": bool(np.all(diff <= 0.02 + 0.02 * np.abs(e))),
    }
