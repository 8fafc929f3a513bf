"""CPU pins of the oracle (no GPU): golden vectors, known-answer tests of the
reference's own suite, closed forms and brute force.

Each test is chosen so that a plausible slip in the oracle (a dropped term, a
wrong sign, a transposed scale table, a different accumulation order) makes
it fail.  The oracle is the checker for the GPU parity tests, so it is pinned
here independently of the HIP library.
"""

from __future__ import annotations

import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def bf16_round_f64(values) -> np.ndarray:
    """float64 -> BF16 bits through float32 (both RNE)."""
    from oracle import oracle

    return oracle.f32_to_bf16(np.asarray(values, dtype=np.float64).astype(np.float32))


def e4m3_closed_form(code: int) -> float:
    """E4M3 value from its bit fields (bias 7, subnormal exponent -6).  0x7F
    and 0xFF are read as the finite value 480 = 1.875 * 2^8, as the
    reference's table does (fp8.py:22-39) where OCP E4M3 has NaN."""
    sign = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0:
        return sign * (m / 8.0) * 2.0 ** -6
    return sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)


# --------------------------------------------------------------- E4M3 ---

def test_e4m3_lut_equals_reference_table(O):
    golden = json.loads((GOLDEN / "e4m3_lut.json").read_text())["values"]
    lut = O.e4m3_lut()
    assert lut.shape == (256,)
    assert np.array_equal(lut, np.asarray(golden, dtype=np.float32))


def test_e4m3_lut_closed_form_and_480_codes(O):
    lut = O.e4m3_lut()
    for c in range(256):
        assert lut[c] == np.float32(e4m3_closed_form(c)), hex(c)
        assert O.lib().glm53o_e4m3_value(c) == e4m3_closed_form(c)
    assert lut[0x7F] == 480.0 and lut[0xFF] == -480.0


def test_e4m3_lut_matches_torch_float8_except_nan_codes(O):
    torch = pytest.importorskip("torch")
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    tv = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    lut = O.e4m3_lut()
    finite = np.ones(256, dtype=bool)
    finite[[0x7F, 0xFF]] = False
    assert np.array_equal(lut[finite], tv[finite])
    assert np.isnan(tv[0x7F]) and np.isnan(tv[0xFF])


# ------------------------------------------------------------ sigmoid ---

def _sweep_domain() -> np.ndarray:
    """All finite BF16 values in [-10, 10], ascending bit order."""
    from oracle import oracle

    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = oracle.bf16_to_f32(bits)
    keep = np.isfinite(vals) & (vals >= -10.0) & (vals <= 10.0)
    return bits[keep]


def _sha(bits: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(bits, dtype="<u2").tobytes()).hexdigest()


def test_sigmoid_domain_matches_reference_sweep():
    sweep = json.loads((GOLDEN / "sigmoid_sweep.json").read_text())
    dom = _sweep_domain()
    assert dom.size == sweep["domain_elements"] == 33346
    assert _sha(dom) == sweep["domain_bits_sha256"]


def test_sigmoid_matches_reference_sweep_hash(O):
    """The reference's exhaustive BF16 sweep hash of mx.sigmoid (the ordering
    its routed activation uses) pins every one of the 33,346 values."""
    sweep = json.loads((GOLDEN / "sigmoid_sweep.json").read_text())
    out = O.sigmoid_bf16(_sweep_domain())
    assert _sha(out) == sweep["reference_sigmoid_sha256"]
    assert sweep["formula_hashes"]["fast_bf16"] == sweep["reference_sigmoid_sha256"]


def test_sigmoid_differs_from_correctly_rounded_exp_at_one_point(O):
    """A float64 restatement (exp correctly rounded, every step to BF16)
    reproduces the sweep's 'precise_bf16' hash; the oracle differs from it
    at exactly the one element the sweep records."""
    sweep = json.loads((GOLDEN / "sigmoid_sweep.json").read_text())
    from oracle import oracle

    dom = _sweep_domain()
    g = oracle.bf16_to_f32(dom).astype(np.float64)
    e = oracle.bf16_to_f32(bf16_round_f64(np.exp(np.abs(g)))).astype(np.float64)
    d = oracle.bf16_to_f32(bf16_round_f64(1.0 + e)).astype(np.float64)
    tail = oracle.bf16_to_f32(bf16_round_f64(1.0 / d)).astype(np.float64)
    precise = np.where(g < 0, bf16_round_f64(tail), bf16_round_f64(1.0 - tail))
    assert _sha(precise) == sweep["formula_hashes"]["precise_bf16"]
    out = O.sigmoid_bf16(dom)
    diff = np.nonzero(out != precise)[0]
    first = sweep["formula_first_difference"]["precise_bf16"]
    assert diff.tolist() == [first["index"]]
    assert int(out[diff[0]]) == int(first["reference_bits"], 16)
    assert int(precise[diff[0]]) == int(first["actual_bits"], 16)
    assert int(dom[diff[0]]) == 0xC0DB


def test_sigmoid_close_to_float64_everywhere(O):
    from oracle import oracle

    dom = _sweep_domain()
    g = oracle.bf16_to_f32(dom).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-g))
    got = oracle.bf16_to_f32(O.sigmoid_bf16(dom)).astype(np.float64)
    # every stepwise value sits within a few BF16 ulps of the true sigmoid
    assert np.all(np.abs(got - ref) <= 4 * 2.0 ** -8 * np.maximum(ref, 2.0 ** -126) + 1e-30)


# ------------------------------------------------------------- SwiGLU ---

def test_swiglu_clamps_and_rounding(O):
    from oracle import oracle

    rng = np.random.default_rng(3)
    limit = 7.0
    g = oracle.f32_to_bf16(rng.normal(0, 6, 4096).astype(np.float32))
    u = oracle.f32_to_bf16(rng.normal(0, 6, 4096).astype(np.float32))
    h = O.swiglu(g, u, limit)
    gf = oracle.bf16_to_f32(g).astype(np.float64)
    uf = oracle.bf16_to_f32(u).astype(np.float64)
    gc = np.minimum(gf, limit)
    uc = np.clip(uf, -limit, limit)
    exact = gc / (1.0 + np.exp(-gc)) * uc
    hf = oracle.bf16_to_f32(h).astype(np.float64)
    # three BF16 roundings and the stepwise sigmoid: within 2^-6 relative
    assert np.all(np.abs(hf - exact) <= 2.0 ** -6 * np.abs(exact) + 1e-6)
    # gate above the limit is the limit; up is clipped on both sides
    big = oracle.f32_to_bf16(np.array([30.0, -30.0, 7.0], dtype=np.float32))
    lim = oracle.f32_to_bf16(np.array([7.0, -7.0, 7.0], dtype=np.float32))
    one = oracle.f32_to_bf16(np.ones(3, dtype=np.float32))
    assert np.array_equal(O.swiglu(big[:1].repeat(3), big, limit), O.swiglu(lim[:1].repeat(3), lim, limit))
    three = oracle.f32_to_bf16(np.full(3, 3.0, np.float32))
    assert np.array_equal(O.swiglu(three, big, limit), O.swiglu(three, lim, limit))
    neg = O.swiglu(oracle.f32_to_bf16(np.array([-30.0], np.float32)), one[:1], limit)
    assert abs(float(oracle.bf16_to_f32(neg)[0])) < 1e-9  # silu(-30) ~ -2.8e-12


# ------------------------------------------------------------- linear ---

def test_fp8_linear_reference_kat_129x257(O):
    """tests/test_fp8_metal.py:23-39: m=129, k=257 (crosses output and
    reduction block boundaries), codes randint(0, 247), scales U*0.02,
    error against the float32 dequantised matmul <= 0.03125."""
    from oracle import oracle

    rng = np.random.default_rng(11)
    codes = rng.integers(0, 247, size=(129, 257)).astype(np.uint8)
    scales = (rng.uniform(size=(2, 3)) * 0.02).astype(np.float32)
    x = oracle.f32_to_bf16(rng.normal(size=(2, 257)).astype(np.float32))
    y = O.fp8_linear(x, codes, scales)
    dense = O.e4m3_lut()[codes].astype(np.float32)
    expanded = np.repeat(np.repeat(scales, 128, 0), 128, 1)[:129, :257]
    expected = oracle.f32_to_bf16(oracle.bf16_to_f32(x) @ (dense * expanded).T)
    err = np.max(np.abs(oracle.bf16_to_f32(y) - oracle.bf16_to_f32(expected)))
    assert err <= 0.03125


def test_fp8_linear_closed_form_distinct_block_scales(O):
    """Every 128x128 block gets a distinct power-of-ten scale, so a transposed
    or shifted scale index changes the result by orders of magnitude."""
    from oracle import oracle

    rng = np.random.default_rng(5)
    n, k = 300, 390  # 3 x 4 scale grid, ragged edges
    codes = rng.integers(0, 256, size=(n, k)).astype(np.uint8)
    scales = np.array([[10.0 ** -(i * 4 + j) for j in range(4)] for i in range(3)], dtype=np.float32)
    x = oracle.f32_to_bf16(rng.normal(size=(5, k)).astype(np.float32))
    y = oracle.bf16_to_f32(O.fp8_linear(x, codes, scales)).astype(np.float64)
    vals = np.array([e4m3_closed_form(c) for c in range(256)])[codes]
    w = vals * np.repeat(np.repeat(scales.astype(np.float64), 128, 0), 128, 1)[:n, :k]
    exact = oracle.bf16_to_f32(x).astype(np.float64) @ w.T
    # only the final BF16 rounding separates the oracle from the exact sum
    assert np.all(np.abs(y - exact) <= 2.0 ** -8 * np.abs(exact) + 1e-38)


def test_fp8_linear_rejects_bad_scale_shape(O):
    codes = np.zeros((129, 257), np.uint8)
    with pytest.raises(ValueError):
        O.fp8_linear(np.zeros((1, 257), np.uint16), codes, np.ones((3, 2), np.float32))


# ----------------------------------------------------------- quantiser ---

def test_quantizer_grid_and_scales(O):
    rng = np.random.default_rng(9)
    w = rng.normal(0, 0.02, size=(200, 300)).astype(np.float32)
    codes, scale = O.quantize_e4m3_blocks(w)
    assert scale.shape == (2, 3)
    assert not np.any((codes & 0x7F) == 0x7F)
    for i in range(2):
        for j in range(3):
            blk = w[i * 128:(i + 1) * 128, j * 128:(j + 1) * 128]
            assert scale[i, j] == np.float32(np.max(np.abs(blk)) / 448.0)
    deq = O.dequantize(codes, scale)
    rel = np.abs(deq - w) / np.repeat(np.repeat(scale, 128, 0), 128, 1)[:200, :300]
    # half an E4M3 step: 2^-4 relative for normals, 2^-10 absolute below 2^-6
    assert np.all(rel <= np.maximum(np.abs(w) / np.repeat(np.repeat(scale, 128, 0), 128, 1)[:200, :300] * 2.0 ** -4,
                                    2.0 ** -10) + 1e-9)
    # values already on the grid are reproduced exactly
    grid = O.dequantize(codes, scale).astype(np.float32)
    codes2, scale2 = O.quantize_e4m3_blocks(grid)
    assert np.array_equal(scale2, scale) and np.array_equal(codes2, codes)


# -------------------------------------------------------------- router ---

def test_router_weights_reference_kat(O):
    """tests/test_grouped_divergence.py:181-199: W = [[1,0],[0,1],[1,1]],
    x = [1, 2], ids [2, 0], norm, scaling 2.0 ->
    sigmoid([3, 1]) / sum * 2."""
    from oracle import oracle

    w = np.array([[1.0, 0.0], [0.0, 1.0], [1.0, 1.0]], np.float32)
    x = oracle.f32_to_bf16(np.array([[1.0, 2.0]], np.float32))
    got = O.router_weights_for(x, w, np.array([[2, 0]]), routed_scaling_factor=2.0)
    raw = 1.0 / (1.0 + np.exp(-np.array([3.0, 1.0])))
    assert np.allclose(got, raw / raw.sum() * 2.0, rtol=1e-6, atol=1e-6)
    ids, scores = O.router(x, w, np.zeros(3, np.float32), top_k=2, routed_scaling_factor=2.0)
    raw = 1.0 / (1.0 + np.exp(-np.array([3.0, 2.0])))
    assert ids.tolist() == [[2, 1]]
    assert np.allclose(scores, raw / raw.sum() * 2.0, rtol=1e-6, atol=1e-6)


def test_router_brute_force_selection_bias_and_ties(O):
    """Brute force: choice = sigmoid(logit) + bias (FP32), top-k by (choice
    desc, id asc); weights from the UNbiased sigmoid, normalised and scaled."""
    from oracle import oracle

    rng = np.random.default_rng(21)
    T, H, E, k = 6, 64, 40, 8
    x = oracle.f32_to_bf16(rng.normal(size=(T, H)).astype(np.float32))
    w = (rng.normal(size=(E, H)) * 0.1).astype(np.float32)
    bias = (rng.normal(size=E) * 0.05).astype(np.float32)
    bias[5] = bias[6] = 10.0  # forced picks, and exact ties broken by id
    w[6] = w[5]
    ids, scores, choice = O.router(x, w, bias, top_k=k, routed_scaling_factor=2.5, return_choice=True)
    logits = (oracle.bf16_to_f32(x).astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32)
    sig = (1.0 / (1.0 + np.exp(-logits.astype(np.float64)))).astype(np.float32)
    ch = (sig + bias).astype(np.float32)
    assert np.allclose(choice, ch, rtol=0, atol=2e-7)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(choice[t, e]), e))[:k]
        assert ids[t].tolist() == order
        assert ids[t, 0] == 5 and ids[t, 1] == 6
    expect = O.router_weights_for(x, w, ids, routed_scaling_factor=2.5)
    assert np.allclose(scores, expect, rtol=1e-6, atol=0)
    assert np.allclose(scores.sum(-1), 2.5, rtol=1e-5)


def _biased_router(bias_rows):
    """A router whose biased scores are 0.5 + bias exactly: zero weights make
    every logit 0 and every sigmoid 0.5, for one token per bias row."""
    from oracle import oracle

    bias_rows = np.asarray(bias_rows, dtype=np.float32)
    e = bias_rows.shape[-1]
    x = oracle.f32_to_bf16(np.ones((1, 8), dtype=np.float32))
    return x, np.zeros((e, 8), dtype=np.float32), bias_rows


def test_router_group_limited_known_answers(O):
    """Group-limited selection (patch.py:134-142 passes n_group, topk_group to
    mlx-vlm's group_expert_select; the published DeepSeek-V3 rule): groups of
    consecutive experts scored by the sum of their two largest biased scores,
    all but the topk_group best groups zeroed, then the top-k.  Known answers
    on constructed scores (16 experts, 4 groups of 4):

    group 0: 0.90 0.89 0.20 0.20 -> 1.79   group 1: 0.95 0.30 0.30 0.30 -> 1.25
    group 2: 0.80 0.80 0.80 0.80 -> 1.60   group 3: 0.60 0.60 0.60 0.60 -> 1.20

    keeps groups 0 and 2, so the top-4 is experts 0, 1, 8, 9: expert 4 (the
    largest score, 0.95) is dropped with its group, and ungrouped selection
    (n_group = 1) picks 4, 0, 1, 8 instead.  A group's second score counts
    even when it equals the first (group 2 scores 1.60, not 0.80)."""
    b = np.array([0.40, 0.39, -0.30, -0.30, 0.45, -0.20, -0.20, -0.20,
                  0.30, 0.30, 0.30, 0.30, 0.10, 0.10, 0.10, 0.10])
    x, w, bias = _biased_router(b)
    ids, sc, choice = O.router(x, w, bias, top_k=4, n_group=4, topk_group=2, return_choice=True)
    assert ids[0].tolist() == [0, 1, 8, 9]
    assert np.allclose(sc[0], 0.25)  # equal sigmoids, normalised
    assert np.all(choice[0, 4:8] == 0.0) and np.all(choice[0, 12:] == 0.0)
    assert O.router(x, w, bias, top_k=4)[0][0].tolist() == [4, 0, 1, 8]
    # topk_group = n_group keeps every group: the ungrouped answer
    assert O.router(x, w, bias, top_k=4, n_group=4, topk_group=4)[0][0].tolist() == [4, 0, 1, 8]
    # one group kept: group 0 alone
    assert O.router(x, w, bias, top_k=4, n_group=4, topk_group=1)[0][0].tolist() == [0, 1, 2, 3]
    # equal group scores: the lower group index is kept
    b2 = np.array([0.2, 0.1, 0.0, 0.0, 0.1, 0.2, 0.3, -0.4])  # groups of 4: 0.7+0.6 = 1.3 against 0.8+0.7 = 1.5
    x, w, bias = _biased_router(b2)
    assert O.router(x, w, bias, top_k=2, n_group=2, topk_group=1)[0][0].tolist() == [6, 5]
    b3 = np.array([0.3, 0.2, 0.0, 0.0, 0.2, 0.3, 0.0, 0.0])  # both groups 0.8 + 0.7
    x, w, bias = _biased_router(b3)
    assert O.router(x, w, bias, top_k=2, n_group=2, topk_group=1)[0][0].tolist() == [0, 1]


def test_router_group_limited_equals_restricted_selection(O):
    """Property on random scores: when every kept group has at least top_k
    positive biased scores, the group-limited top-k equals the ungrouped top-k
    restricted to the experts of the kept groups, and each kept group's score
    is at least every dropped group's."""
    from oracle import oracle

    rng = np.random.default_rng(5)
    T, H, E, G, keep, k = 12, 64, 64, 8, 3, 6
    x = oracle.f32_to_bf16(rng.normal(size=(T, H)).astype(np.float32))
    w = (rng.normal(size=(E, H)) * 0.1).astype(np.float32)
    bias = (rng.normal(size=E) * 0.05).astype(np.float32)
    ids, _, _ = O.router(x, w, bias, top_k=k, n_group=G, topk_group=keep, return_choice=True)
    _, _, choice0 = O.router(x, w, bias, top_k=k, return_choice=True)
    per = E // G
    for t in range(T):
        grp = choice0[t].reshape(G, per)
        top2 = np.sort(grp, axis=1)[:, -2:]
        gscore = (top2[:, 1] + top2[:, 0]).astype(np.float32)
        kept = sorted(range(G), key=lambda g: (-float(gscore[g]), g))[:keep]
        assert min(gscore[kept]) >= max(np.delete(gscore, kept))
        allowed = [e for e in range(E) if e // per in kept]
        assert all(choice0[t, e] > 0 for e in allowed)
        order = sorted(allowed, key=lambda e: (-float(choice0[t, e]), e))[:k]
        assert ids[t].tolist() == order


# ------------------------------------------------------------ tile plan ---

def test_tile_plan_reference_kat():
    """tests/test_fp8_metal.py:201-238."""
    from oracle import oracle

    se = np.array([0] * 31 + [1] * 32 + [287] * 33)
    plan = oracle.build_grouped_tile_plan(se, 288)
    valid = plan.starts < se.size
    assert list(zip(plan.experts[valid].tolist(), plan.starts[valid].tolist(), plan.lengths[valid].tolist())) == [
        (0, 0, 31), (1, 31, 32), (287, 63, 32), (287, 95, 1)]
    counts = np.bincount(se, minlength=288)
    assert int((counts > 0).sum()) == 3 and int((counts == 0).sum()) == 285 and counts.max() == 33
    assert plan.experts.size == math.ceil(96 / 32) + 288
    assert np.all(plan.lengths[~valid] == 0)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_tile_plan_invariants(seed):
    """scripts/probe_grouped_fp8_moe.py:103-166: every route covered once,
    no tile crosses an expert boundary, tiles start expert-aligned."""
    from oracle import oracle

    rng = np.random.default_rng(seed)
    E = 37
    se = np.sort(rng.integers(0, E, size=int(rng.integers(0, 400))))
    plan = oracle.build_grouped_tile_plan(se, E)
    covered = np.zeros(se.size, np.int64)
    for e, s, n in zip(plan.experts, plan.starts, plan.lengths):
        if n == 0:
            assert s == se.size
            continue
        assert 1 <= n <= 32
        assert np.all(se[s:s + n] == e)
        assert s == plan.route_offsets[e] or (s - plan.route_offsets[e]) % 32 == 0
        covered[s:s + n] += 1
    assert np.all(covered == 1)


def test_route_plan_is_stable_sort():
    from oracle import oracle

    rng = np.random.default_rng(4)
    ids = rng.integers(0, 9, size=(13, 4))
    scores = rng.uniform(size=(13, 4)).astype(np.float32)
    plan = oracle.build_route_plan(ids, scores)
    flat = ids.reshape(-1)
    brute = sorted(range(flat.size), key=lambda r: (flat[r], r))
    assert plan.order.tolist() == brute
    assert np.array_equal(plan.order[plan.inverse], np.arange(flat.size))
    assert np.array_equal(plan.token_ids, np.array(brute) // 4)
    assert np.array_equal(plan.sorted_scores, scores.reshape(-1)[brute])


# ----------------------------------------------------------- reductions ---

def test_direct_order_reduce_matches_expert_scatter_add(O):
    """tests/test_grouped_divergence.py:233-254: visiting experts in ascending
    id and adding T(out * score) into a BF16 accumulator."""
    from oracle import oracle

    rng = np.random.default_rng(8)
    indices = np.array([[7, 0, 6, 1, 5, 2, 4, 3], [3, 4, 2, 5, 1, 6, 0, 7]], np.int32)
    scores = rng.uniform(size=(2, 8)).astype(np.float32)
    route = oracle.f32_to_bf16(rng.normal(size=(16, 128)).astype(np.float32))
    expected = np.zeros((2, 128), np.uint16)
    for expert in range(8):
        for row, slot in np.argwhere(indices == expert):
            prod = oracle.f32_to_bf16(oracle.bf16_to_f32(route[row * 8 + slot]) * scores[row, slot])
            acc = oracle.bf16_to_f32(expected[row]) + oracle.bf16_to_f32(prod)
            expected[row] = oracle.f32_to_bf16(acc)
    assert np.array_equal(O.direct_order_reduce(route, indices, scores), expected)
    # the order matters: slot order gives a different BF16 result somewhere
    slot_order = np.zeros((2, 128), np.uint16)
    for row in range(2):
        for slot in range(8):
            prod = oracle.f32_to_bf16(oracle.bf16_to_f32(route[row * 8 + slot]) * scores[row, slot])
            slot_order[row] = oracle.f32_to_bf16(oracle.bf16_to_f32(slot_order[row]) + oracle.bf16_to_f32(prod))
    assert not np.array_equal(slot_order, expected)


def test_restore_and_reduce_fp32_slot_order(O):
    """grouped_fp8.py:273-276: restore route order, FP32 products, FP32 sum in
    slot order, one BF16 rounding."""
    from oracle import oracle

    rng = np.random.default_rng(12)
    T, k, H = 5, 8, 96
    ids = rng.integers(0, 11, size=(T, k))
    scores = rng.uniform(size=(T, k)).astype(np.float32)
    plan = oracle.build_route_plan(ids, scores)
    sorted_out = oracle.f32_to_bf16(rng.normal(size=(T * k, H)).astype(np.float32))
    got = O.restore_and_reduce(sorted_out, plan.sorted_scores, plan.inverse, T, k)
    expected = np.zeros((T, H), np.uint16)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for s in range(k):
            r = plan.inverse[t * k + s]
            acc = (acc + oracle.bf16_to_f32(sorted_out[r]) * np.float32(plan.sorted_scores[r])).astype(np.float32)
        expected[t] = oracle.f32_to_bf16(acc)
    assert np.array_equal(got, expected)


# ------------------------------------------------------------- MoE level ---

def _bank(O, rng, E, H, I):
    from types import SimpleNamespace

    sh = O.bank_shapes(E, H, I)
    return SimpleNamespace(
        gate_up_weight=rng.integers(0, 247, size=sh["gate_up_weight"]).astype(np.uint8),
        gate_up_scale_inv=(rng.uniform(size=sh["gate_up_scale_inv"]) * 0.002).astype(np.float32),
        down_weight=rng.integers(0, 247, size=sh["down_weight"]).astype(np.uint8),
        down_scale_inv=(rng.uniform(size=sh["down_scale_inv"]) * 0.002).astype(np.float32),
        intermediate_size=I,
    )


def test_bank_shapes_reference_kat(O):
    """tests/test_fp8_metal.py:120-124 (E=8, H=257, I=129)."""
    assert O.bank_shapes(8, 257, 129) == {
        "gate_up_weight": (8, 258, 257), "gate_up_scale_inv": (8, 4, 3),
        "down_weight": (8, 257, 129), "down_scale_inv": (8, 3, 2)}


def test_decode_matches_explicit_routing_closed_form(O):
    """tests/test_fp8_metal.py:42-83: routes [7,1,5,0,3,6,2,4], fixed scores,
    H=257, I=129, limit 3; explicit float64 routing within rtol/atol 0.02."""
    from oracle import oracle

    rng = np.random.default_rng(17)
    E, H, I, L = 8, 257, 129, 3.0
    bank = _bank(O, rng, E, H, I)
    ids = np.array([7, 1, 5, 0, 3, 6, 2, 4])
    scores = np.array([0.24, 0.18, 0.15, 0.13, 0.11, 0.08, 0.06, 0.05], np.float32)
    x = oracle.f32_to_bf16((rng.normal(size=H) * 2).astype(np.float32))
    got = oracle.bf16_to_f32(O.direct_moe(x[None], bank, ids[None], scores[None], L)).astype(np.float64)[0]
    xf = oracle.bf16_to_f32(x).astype(np.float64)
    expected = np.zeros(H)
    for slot, e in enumerate(ids):
        # the up half's scale rows start at ceil(I / 128), not at row I / 128
        g = O.dequantize(bank.gate_up_weight[e, :I], bank.gate_up_scale_inv[e, :2]) @ xf
        u = O.dequantize(bank.gate_up_weight[e, I:], bank.gate_up_scale_inv[e, 2:]) @ xf
        gc = np.minimum(g, L)
        h = gc / (1.0 + np.exp(-gc)) * np.clip(u, -L, L)
        expected += (O.dequantize(bank.down_weight[e], bank.down_scale_inv[e]) @ h) * float(scores[slot])
    assert np.allclose(got, expected, rtol=0.02, atol=0.02)


def test_grouped_equals_direct_and_decode_fallback(O):
    """tests/test_fp8_metal.py:156-198 on the oracle: deterministic routes
    (5r + 3) mod 8, scores 1/8; grouped (Direct-order reduction) equals
    Direct exactly, the FP32 slot-order reduction within 0.02; one token
    takes the decode path either way."""
    from oracle import oracle

    rng = np.random.default_rng(23)
    E, H, I, L, T = 8, 256, 128, 3.0, 6
    bank = _bank(O, rng, E, H, I)
    routes = ((np.arange(T * 8) * 5 + 3) % 8).reshape(T, 8)
    scores = np.full((T, 8), 0.125, np.float32)
    x = oracle.f32_to_bf16(rng.normal(size=(T, H)).astype(np.float32))
    direct = O.direct_moe(x, bank, routes, scores, L)
    assert np.array_equal(O.grouped_moe(x, bank, routes, scores, L, reduction="direct"), direct)
    grouped = O.grouped_moe(x, bank, routes, scores, L, reduction="grouped")
    a, e = oracle.bf16_to_f32(grouped), oracle.bf16_to_f32(direct)
    assert np.allclose(a, e, rtol=0.02, atol=0.02)
    one = O.direct_moe(x[:1], bank, routes[:1], scores[:1], L)
    assert np.array_equal(one[0], O.decode_moe(x[0], bank, routes[0], scores[0], L))


def test_moe_reductions_equal_the_separate_compositions(O):
    """moe_reductions (one pass over the experts, both combines) equals
    direct_moe and grouped_moe(reduction="grouped") bit for bit, with a
    shared expert and uneven routes; the two reductions differ somewhere,
    so the comparison is not of one array with itself."""
    from types import SimpleNamespace

    from oracle import oracle

    rng = np.random.default_rng(29)
    E, H, I, L, T = 8, 256, 128, 3.0, 24
    bank = _bank(O, rng, E, H, I)
    shared_bank = _bank(O, rng, 1, H, I)
    mats = O.expert_matrices(shared_bank, 0)
    shared = SimpleNamespace(gate=mats.gate, up=mats.up, down=mats.down)
    routes = np.stack([rng.choice(E, size=4, replace=False) for _ in range(T)])
    scores = rng.uniform(0.05, 1.5, size=(T, 4)).astype(np.float32)
    x = oracle.f32_to_bf16((rng.normal(size=(T, H)) * 3).astype(np.float32))
    both = O.moe_reductions(x, bank, routes, scores, L, shared)
    assert np.array_equal(both["direct"], O.direct_moe(x, bank, routes, scores, L, shared))
    assert np.array_equal(both["grouped"], O.grouped_moe(x, bank, routes, scores, L, shared, reduction="grouped"))
    assert not np.array_equal(both["direct"], both["grouped"])


def test_hc_expand_special_cases_and_float64_restatement(O):
    """Hyper-connection expand (metal:2362-2388): comb = identity with post =
    0 returns the residual streams bit for bit; comb = 0 with post = 1
    returns the MoE output; random inputs match a float64 restatement that
    rounds the FMA chain and the product to FP32 where the kernel does."""
    rng = np.random.default_rng(21)
    T, H = 5, 64
    moe = O.f32_to_bf16(rng.normal(size=(T, H)).astype(np.float32))
    res = O.f32_to_bf16(rng.normal(size=(T, 4, H)).astype(np.float32))
    eye = np.broadcast_to(np.eye(4, dtype=np.float32), (T, 4, 4)).copy()
    assert np.array_equal(O.hc_expand(moe, res, np.zeros((T, 4), np.float32), eye), res)
    got = O.hc_expand(moe, res, np.ones((T, 4), np.float32), np.zeros((T, 4, 4), np.float32))
    assert np.array_equal(got, np.repeat(moe[:, None, :], 4, axis=1))
    post = rng.normal(size=(T, 4)).astype(np.float32)
    comb = rng.normal(size=(T, 4, 4)).astype(np.float32)
    m = O.bf16_to_f32(moe).astype(np.float64)
    r = O.bf16_to_f32(res).astype(np.float64)
    want = np.zeros((T, 4, H), np.uint16)
    for b in range(4):
        mixed = np.zeros((T, H), np.float32)
        for src in range(4):  # one rounding per FMA: at these magnitudes the product-sum is exact in float64
            mixed = (comb[:, src, b, None].astype(np.float64) * r[:, src] + mixed.astype(np.float64)).astype(np.float32)
        branch = (post[:, b, None].astype(np.float64) * m).astype(np.float32)
        want[:, b] = O.f32_to_bf16((branch.astype(np.float64) + mixed.astype(np.float64)).astype(np.float32))
    assert np.array_equal(O.hc_expand(moe, res, post, comb), want)


def test_cpu_comparator_matches_the_oracle(O):
    """The benchmark's CPU comparator (oracle/cpu_direct.py: Direct with FP32
    accumulation, timed as bench.py's cpu_baseline) computes the same
    function as the float64 oracle: linear within the BASELINE gates with
    most outputs bit-identical, the router's picks equal (no near-ties at
    these scales), decode and prefill MoE (with a shared expert) within the
    gates and the reference's elementwise tolerance."""
    from types import SimpleNamespace

    from oracle import cpu_direct as C
    from oracle import oracle

    from conftest import assert_parity

    codes = np.arange(256, dtype=np.uint8)
    assert np.array_equal(C.decode_codes(codes).view(np.uint32), O.e4m3_lut().view(np.uint32))
    rng = np.random.default_rng(31)
    E, H, I, L, T = 8, 256, 128, 3.0, 20
    bank = _bank(O, rng, E, H, I)
    mats = O.expert_matrices(_bank(O, rng, 1, H, I), 0)
    shared = SimpleNamespace(gate=mats.gate, up=mats.up, down=mats.down)
    x = oracle.f32_to_bf16(rng.normal(size=(T, H)).astype(np.float32))
    w, s = bank.gate_up_weight[3], bank.gate_up_scale_inv[3]
    assert_parity(C.linear(x, w, s), O.fp8_linear(x, w, s), O, exact_fraction=0.97)
    rw = (rng.normal(size=(E, H)) * 0.05).astype(np.float32)
    rb = rng.uniform(-0.01, 0.01, size=E).astype(np.float32)
    ids, sc = C.router(x, rw, rb, top_k=4)
    ids_o, sc_o = O.router(x, rw, rb, top_k=4)
    assert np.array_equal(ids, ids_o)
    np.testing.assert_allclose(sc, sc_o, rtol=2e-6)
    got = C.direct_moe(x, bank, ids, sc, L, shared)
    assert_parity(got, O.direct_moe(x, bank, ids, sc, L, shared), O, exact_fraction=0.75)
    ids8 = np.stack([rng.choice(E, size=8, replace=False)]).astype(np.int32)
    sc8 = rng.uniform(0.05, 0.3, size=(1, 8)).astype(np.float32)
    got1 = C.direct_moe(x[:1], bank, ids8, sc8, L, shared)
    assert_parity(got1, O.direct_moe(x[:1], bank, ids8, sc8, L, shared), O, exact_fraction=0.75)
    assert C.num_threads() >= 1
