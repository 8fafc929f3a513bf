"""GPU parity: route plan, grouped FP8 GEMM and sorted grouped prefill
(grouped_fp8.py:157-328)."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from conftest import assert_parity, from_bits, host_bank, host_shared, random_codes, submodule, to_bits

pytestmark = pytest.mark.gpu


def test_route_plan_is_stable_sort(O, dev):
    import torch

    grouped = submodule("grouped_fp8")
    rng = np.random.default_rng(4)
    for tokens, experts in ((256, 288), (2048, 288), (3, 8), (1000, 64), (2100, 288)):
        ids = np.stack([rng.choice(experts, size=8, replace=False) for _ in range(tokens)]).astype(np.int32)
        scores = rng.uniform(size=ids.shape).astype(np.float32)
        plan = grouped._route_plan(torch.from_numpy(ids).to(dev), torch.from_numpy(scores).to(dev), 8, experts)
        want = O.build_route_plan(ids, scores)
        np.testing.assert_array_equal(plan["order"].cpu().numpy(), want.order)
        np.testing.assert_array_equal(plan["inverse"].cpu().numpy(), want.inverse)
        np.testing.assert_array_equal(plan["token_ids"].cpu().numpy(), want.token_ids)
        np.testing.assert_array_equal(plan["sorted_experts"].cpu().numpy(), want.sorted_experts)
        np.testing.assert_array_equal(plan["sorted_scores"].cpu().numpy(), want.sorted_scores)
        tiles = O.build_grouped_tile_plan(want.sorted_experts, experts)
        np.testing.assert_array_equal(plan["tile_experts"].cpu().numpy(), tiles.experts)
        np.testing.assert_array_equal(plan["tile_starts"].cpu().numpy(), tiles.starts)
        np.testing.assert_array_equal(plan["tile_lengths"].cpu().numpy(), tiles.lengths)
        np.testing.assert_array_equal(plan["route_offsets"].cpu().numpy(), tiles.route_offsets)
        np.testing.assert_array_equal(plan["tile_offsets"].cpu().numpy(), tiles.tile_offsets)
        assert int(plan["status"][0]) == 0


def test_tile_plan_kat_sparse_edge_buckets(M, dev):
    """tests/test_fp8_metal.py:201-238 of the reference."""
    import torch

    sorted_experts = torch.tensor([0] * 31 + [1] * 32 + [287] * 33, dtype=torch.int32, device=dev)
    experts, starts, lengths, route_offsets, tile_offsets = M.build_grouped_tile_plan(sorted_experts, 288)
    experts, starts, lengths = (t.cpu().numpy() for t in (experts, starts, lengths))
    valid = starts < 96
    assert list(zip(experts[valid], starts[valid], lengths[valid])) == [(0, 0, 31), (1, 31, 32), (287, 63, 32),
                                                                        (287, 95, 1)]
    assert np.all(lengths[~valid] == 0)
    assert experts.size == 96 // 32 + 288
    counts = np.bincount(sorted_experts.cpu().numpy(), minlength=288)
    assert int(np.sum(counts == 0)) == 285
    np.testing.assert_array_equal(route_offsets.cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))


@pytest.mark.parametrize("tokens,experts,skew", [(2048, 288, False), (2049, 288, False), (2048, 16, True),
                                                 (2300, 16, True), (130, 1024, False)])
def test_route_plan_with_invalid_ids(dev, tokens, experts, skew):
    """The route plan (count / scan / scatter) on ids with ~1% out of range
    (negative or >= experts), uniform or skewed (long runs of one expert in
    every 256-route block), up to 1,024 experts: valid routes in stable
    expert order (numpy's stable argsort), invalid ones with inverse -1 and
    counted in status[0]."""
    import torch

    grouped = submodule("grouped_fp8")
    rng = np.random.default_rng(tokens + experts)
    if skew:
        p = 1.0 / np.arange(1, experts + 1) ** 2
        ids = rng.choice(experts, size=(tokens, 8), p=p / p.sum()).astype(np.int32)
    else:
        ids = rng.integers(0, experts, size=(tokens, 8)).astype(np.int32)
    bad = rng.uniform(size=ids.shape) < 0.01
    ids[bad] = np.where(rng.uniform(size=bad.sum()) < 0.5, -1, experts + 3)
    scores = rng.uniform(size=ids.shape).astype(np.float32)
    plan = grouped._route_plan(torch.from_numpy(ids).to(dev), torch.from_numpy(scores).to(dev), 8, experts)
    flat = ids.reshape(-1)
    valid = (flat >= 0) & (flat < experts)
    order = np.nonzero(valid)[0][np.argsort(flat[valid], kind="stable")]
    n = order.size
    np.testing.assert_array_equal(plan["order"].cpu().numpy()[:n], order)
    inverse = np.full(flat.size, -1, np.int64)
    inverse[order] = np.arange(n)
    np.testing.assert_array_equal(plan["inverse"].cpu().numpy(), inverse)
    np.testing.assert_array_equal(plan["sorted_experts"].cpu().numpy()[:n], flat[order])
    np.testing.assert_array_equal(plan["token_ids"].cpu().numpy()[:n], order // 8)
    np.testing.assert_array_equal(plan["sorted_scores"].cpu().numpy()[:n], scores.reshape(-1)[order])
    counts = np.bincount(flat[valid], minlength=experts)
    np.testing.assert_array_equal(plan["route_offsets"].cpu().numpy(), np.concatenate([[0], np.cumsum(counts)]))
    assert int(plan["status"][0]) == int((~valid).sum())


def test_route_plan_flags_invalid_ids(dev):
    import torch

    grouped = submodule("grouped_fp8")
    ids = torch.tensor([[0, 1], [5, 300]], dtype=torch.int32, device=dev)
    plan = grouped._route_plan(ids, torch.ones(4, device=dev), 2, 8)
    assert int(plan["status"][0]) == 1
    assert int(plan["inverse"][3]) == -1


def _small_bank(M, dev, rng, experts, hidden, inter):
    import torch

    shapes = {
        "gu": (experts, 2 * inter, hidden), "gus": (experts, 2 * (inter // 128), hidden // 128),
        "dw": (experts, hidden, inter), "dws": (experts, hidden // 128, inter // 128),
    }
    gu = torch.from_numpy(random_codes(rng, shapes["gu"])).to(dev)
    dw = torch.from_numpy(random_codes(rng, shapes["dw"])).to(dev)
    gus = torch.from_numpy((rng.uniform(size=shapes["gus"]) * 0.002).astype(np.float32)).to(dev)
    dws = torch.from_numpy((rng.uniform(size=shapes["dws"]) * 0.002).astype(np.float32)).to(dev)
    return M.PackedFP8ExpertBank(*(M.owned_tensor(t) for t in (gu, gus, dw, dws)), intermediate_size=inter)


def test_grouped_linear_matches_oracle(M, O, dev):
    import torch

    rng = np.random.default_rng(12)
    bank = _small_bank(M, dev, rng, 8, 256, 128)
    tokens = 40
    ids = np.stack([rng.choice(8, size=8, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = from_bits(O.f32_to_bf16(rng.normal(size=(tokens, 256)).astype(np.float32)), dev)
    sorted_x, sorted_e, sorted_s, inverse = M.build_route_plan(x, torch.from_numpy(ids).to(dev),
                                                               torch.ones(ids.shape, device=dev))
    tile_plan = M.build_grouped_tile_plan(sorted_e, 8)
    y = M.grouped_fp8_linear(sorted_x, tile_plan, bank.gate_up_weight, bank.gate_up_scale_inv)
    plan = O.build_route_plan(ids, np.ones(ids.shape, np.float32))
    want = O.grouped_linear(to_bits(x)[plan.token_ids], plan.sorted_experts, bank.gate_up_weight.cpu().numpy(),
                            bank.gate_up_scale_inv.cpu().numpy())
    assert_parity(to_bits(y), want, O, exact_fraction=0.95)
    h = M.activate_gate_up(y, 128, 3.0)
    assert np.array_equal(to_bits(h), O.activate_gate_up(to_bits(y), 128, 3.0))
    d = M.grouped_fp8_linear(h, tile_plan, bank.down_weight, bank.down_scale_inv)
    out = M.restore_and_reduce(d, sorted_s, inverse, (tokens, 256), 8)
    want_d = O.grouped_linear(to_bits(h), plan.sorted_experts, bank.down_weight.cpu().numpy(),
                              bank.down_scale_inv.cpu().numpy())
    assert_parity(to_bits(d), want_d, O, exact_fraction=0.95)
    want_out = O.restore_and_reduce(to_bits(d), plan.sorted_scores, plan.inverse, tokens, 8)
    assert np.array_equal(to_bits(out), want_out)


def _place(bits, offset, dev):
    """Device BF16 copy of `bits` starting `offset` elements into its buffer
    (offset 1 leaves the rows 2-byte aligned only)."""
    import torch

    buf = torch.zeros(bits.size + offset, dtype=torch.bfloat16, device=dev)
    view = buf[offset:].view(bits.shape)
    view.copy_(from_bits(bits, dev))
    return view


@pytest.mark.parametrize("hidden,offset", [(256, 0), (256, 1), (200, 0)])
def test_reductions_at_any_width_and_alignment_match_oracle(M, O, dev, hidden, offset):
    """Slot-order and ascending-expert reductions with the shared add: 16-byte
    aligned rows with H % 8 == 0 take the 8-column form, the rest the
    1-column form; both match the oracle bit for bit."""
    import torch

    N = submodule("_native")
    rng = np.random.default_rng(31 + hidden + offset)
    tokens, k = 37, 8
    route = O.f32_to_bf16(rng.normal(size=(tokens * k, hidden)).astype(np.float32))
    shared = O.f32_to_bf16(rng.normal(size=(tokens, hidden)).astype(np.float32))
    ids = np.stack([rng.choice(32, size=k, replace=False) for _ in range(tokens)]).astype(np.int32)
    scores = rng.uniform(size=(tokens, k)).astype(np.float32)
    route_d, shared_d = _place(route, offset, dev), _place(shared, offset, dev)
    inverse = torch.arange(tokens * k, dtype=torch.int32, device=dev)
    scores_d = torch.from_numpy(scores.reshape(-1)).to(dev)
    ids_d = torch.from_numpy(ids.reshape(-1)).to(dev)
    lib, st = N.lib(), N.stream_handle(dev)
    out = _place(np.zeros((tokens, hidden), np.uint16), offset, dev)
    N.check(lib.glm53_restore_and_reduce(N.ptr(route_d), N.ptr(scores_d), N.ptr(inverse), tokens, k, hidden,
                                         N.ptr(shared_d), N.ptr(out), st))
    want = O.add_bf16(O.restore_and_reduce(route, scores.reshape(-1), np.arange(tokens * k), tokens, k), shared)
    assert np.array_equal(to_bits(out), want)
    out = _place(np.zeros((tokens, hidden), np.uint16), offset, dev)
    N.check(lib.glm53_direct_order_reduce(N.ptr(route_d), N.ptr(inverse), N.ptr(ids_d), N.ptr(scores_d), tokens, k,
                                          hidden, N.ptr(shared_d), N.ptr(out), st))
    want = O.add_bf16(O.direct_order_reduce(route, ids, scores), shared)
    assert np.array_equal(to_bits(out), want)


def test_grouped_linear_unaligned_activations_split_alike(M, O, dev):
    """Activation rows that are only 2-byte aligned take the two-column split;
    the GEMM output equals the aligned run bit for bit."""
    import torch

    rng = np.random.default_rng(13)
    bank = _small_bank(M, dev, rng, 8, 384, 128)  # 3 blocks per row: a partial group of 4 in the wide split
    tokens = 24
    ids = np.stack([rng.choice(8, size=8, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = from_bits(O.f32_to_bf16(rng.normal(size=(tokens, 384)).astype(np.float32)), dev)
    sorted_x, sorted_e, _, _ = M.build_route_plan(x, torch.from_numpy(ids).to(dev), torch.ones(ids.shape, device=dev))
    tile_plan = M.build_grouped_tile_plan(sorted_e, 8)
    y = M.grouped_fp8_linear(sorted_x, tile_plan, bank.gate_up_weight, bank.gate_up_scale_inv)
    shifted = _place(to_bits(sorted_x), 1, dev)
    assert shifted.data_ptr() % 16 != 0
    y_shifted = M.grouped_fp8_linear(shifted, tile_plan, bank.gate_up_weight, bank.gate_up_scale_inv)
    assert np.array_equal(to_bits(y_shifted), to_bits(y))
    plan = O.build_route_plan(ids, np.ones(ids.shape, np.float32))
    want = O.grouped_linear(to_bits(x)[plan.token_ids], plan.sorted_experts, bank.gate_up_weight.cpu().numpy(),
                            bank.gate_up_scale_inv.cpu().numpy())
    assert_parity(to_bits(y), want, O, exact_fraction=0.95)


class DeterministicGate:
    """tests/test_fp8_metal.py:160-166 of the reference."""

    def __call__(self, x):
        import torch

        rows = x.reshape(-1, x.shape[-1]).shape[0]
        routes = torch.arange(rows * 8, dtype=torch.int32, device=x.device).reshape(rows, 8)
        indices = ((routes * 5 + 3) % 8).reshape(*x.shape[:-1], 8)
        scores = torch.full(indices.shape, 0.125, dtype=torch.float32, device=x.device)
        return indices, scores


def test_grouped_matches_direct_and_keeps_decode_fallback(M, O, dev):
    """tests/test_fp8_metal.py:154-198: H=256, I=128, E=8, limit 3."""
    import torch

    rng = np.random.default_rng(21)
    cfg = SimpleNamespace(hidden_size=256, moe_intermediate_size=128, swiglu_limit=3.0, n_routed_experts=8,
                          num_experts_per_tok=8)
    direct = M.DirectFP8MoE(cfg, DeterministicGate(), None, device=dev)
    for expert in direct.experts:
        for proj in (expert.gate_proj, expert.up_proj, expert.down_proj):
            proj.weight.copy_(torch.from_numpy(random_codes(rng, tuple(proj.weight.shape))))
            proj.weight_scale_inv.copy_(torch.from_numpy(
                (rng.uniform(size=tuple(proj.weight_scale_inv.shape)) * 0.002).astype(np.float32)))
    bank = M.PackedFP8ExpertBank.pack(direct.experts)
    grouped = M.SortedGroupedFP8MoE(bank, cfg, direct.gate, None)
    assert grouped.min_routes == 256
    x = from_bits(O.f32_to_bf16(rng.normal(size=(1, 32, 256)).astype(np.float32)), dev)
    expected = direct(x)
    actual = grouped(x)
    assert torch.allclose(actual.float(), expected.float(), rtol=0.02, atol=0.02)
    ids, sc = DeterministicGate()(x)
    want = O.direct_moe(to_bits(x).reshape(32, -1), host_bank(bank), ids.reshape(32, 8).cpu().numpy(),
                        sc.reshape(32, 8).cpu().numpy(), 3.0)
    assert_parity(to_bits(actual).reshape(32, -1), want, O)
    exact = M.SortedGroupedFP8MoE(bank, cfg, direct.gate, None, reduction="direct")
    assert_parity(to_bits(exact(x)).reshape(32, -1), want, O, exact_fraction=0.8)

    d1 = from_bits(O.f32_to_bf16(rng.normal(size=(1, 1, 256)).astype(np.float32)), dev)
    assert torch.equal(grouped(d1).view(torch.int16), direct(d1).view(torch.int16))


@pytest.fixture(scope="module")
def config2_layer(dev):
    syn = submodule("synthetic")
    cfg = syn.layer_config()
    bank, shared, gate = syn.synth_layer(cfg, seed=4242, device=dev)
    return cfg, bank, shared, gate


def _touched(bank, experts):
    import torch

    e = np.unique(experts)
    remap = {int(v): i for i, v in enumerate(e)}
    return host_bank(bank, e), np.vectorize(remap.get)(experts).astype(np.int32)


@pytest.mark.parametrize("reduction", ["grouped", "direct"])
def test_config4_prefill_256_tokens_matches_oracle(M, O, dev, config2_layer, reduction):
    """256 tokens -> 2,048 routes over 288 experts."""
    syn = submodule("synthetic")
    cfg, bank, shared, gate = config2_layer
    moe = M.SortedGroupedFP8MoE(bank, cfg, gate, shared, reduction=reduction)
    x = syn.normal_bf16((1, 256, cfg.hidden_size), syn.key(4242, "prefill"), device=dev)
    y = moe(x)
    xb = to_bits(x).reshape(256, -1)
    # the MoE arithmetic is compared on the device's own selection; the
    # selection itself is checked against the oracle with the near-tie rule
    gids, gsc = gate(x)
    ids, sc = gids.reshape(256, 8).cpu().numpy(), gsc.reshape(256, 8).cpu().numpy()
    from test_gpu_decode import _router_check

    _router_check(O, gate, xb, ids, sc)
    sub, local = _touched(bank, ids)
    want_direct = O.direct_moe(xb, sub, local, sc, cfg.swiglu_limit, host_shared(shared))
    stats = assert_parity(to_bits(y).reshape(256, -1), want_direct, O)
    if reduction == "direct":
        assert stats["bit_exact_fraction"] >= 0.75, stats
    else:
        want_grouped = O.grouped_moe(xb, sub, local, sc, cfg.swiglu_limit, host_shared(shared))
        assert_parity(to_bits(y).reshape(256, -1), want_grouped, O, exact_fraction=0.75)


class SkewedGate:
    """Experts 0, 1 and 2 take every token, the other 5 slots are drawn from
    the remaining experts: the heavy experts hold many descriptors and the
    light ones partial ones."""

    def __init__(self, experts, seed):
        self.experts, self.seed = experts, seed

    def __call__(self, x):
        import torch

        rows = x.reshape(-1, x.shape[-1]).shape[0]
        rng = np.random.default_rng(self.seed)
        ids = np.stack([np.concatenate([[0, 1, 2], 3 + rng.choice(self.experts - 3, size=5, replace=False)])
                        for _ in range(rows)]).astype(np.int32)
        sc = rng.uniform(0.05, 0.3, size=ids.shape).astype(np.float32)
        return (torch.from_numpy(ids).to(x.device).reshape(*x.shape[:-1], 8),
                torch.from_numpy(sc).to(x.device).reshape(*x.shape[:-1], 8))


@pytest.mark.parametrize("reduction", ["grouped", "direct"])
def test_skewed_routing_many_descriptors_matches_oracle(M, O, dev, reduction):
    """1,024 tokens over 16 experts (512 routes per expert on average): the
    prefill takes the wide GEMM shape (128-route descriptors, 128-token
    dense tiles for the shared expert); experts 0-2 hold 1,024 routes each
    (8 descriptors of one expert side by side)."""
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=256, intermediate=128, experts=16, top_k=8, limit=7.0)
    bank, shared, _ = syn.synth_layer(cfg, seed=77, device=dev)
    gate = SkewedGate(16, 5)
    moe = M.SortedGroupedFP8MoE(bank, cfg, gate, shared, reduction=reduction)
    T = 1024
    x = syn.normal_bf16((1, T, cfg.hidden_size), syn.key(77, "wide"), device=dev)
    y = moe(x)
    ids, sc = (t.reshape(T, 8).cpu().numpy() for t in gate(x))
    xb = to_bits(x).reshape(T, -1)
    want = O.direct_moe(xb, host_bank(bank), ids, sc, cfg.swiglu_limit, host_shared(shared))
    stats = assert_parity(to_bits(y).reshape(T, -1), want, O)
    if reduction == "grouped":
        want_g = O.grouped_moe(xb, host_bank(bank), ids, sc, cfg.swiglu_limit, host_shared(shared))
        assert_parity(to_bits(y).reshape(T, -1), want_g, O, exact_fraction=0.75)
    else:
        assert stats["bit_exact_fraction"] >= 0.75, stats


class WeightedGate:
    """Each token takes top_k distinct experts drawn with weights 1 / (e + 1):
    expert route counts fall from about a third of the tokens to a few, so
    descriptors of every fill (full, part-filled wavefront rows, one group)
    occur side by side."""

    def __init__(self, experts, top_k, seed):
        self.experts, self.top_k, self.seed = experts, top_k, seed

    def __call__(self, x):
        import torch

        rows = x.reshape(-1, x.shape[-1]).shape[0]
        rng = np.random.default_rng(self.seed)
        w = 1.0 / np.arange(1, self.experts + 1)
        ids = np.stack([rng.choice(self.experts, size=self.top_k, replace=False, p=w / w.sum())
                        for _ in range(rows)]).astype(np.int32)
        sc = rng.uniform(0.05, 0.3, size=ids.shape).astype(np.float32)
        return (torch.from_numpy(ids).to(x.device).reshape(*x.shape[:-1], self.top_k),
                torch.from_numpy(sc).to(x.device).reshape(*x.shape[:-1], self.top_k))


@pytest.mark.parametrize("inter,codes_480", [(384, False), (384, True), (256, True), (128, True)])
def test_wide_gemm_shape_ragged_tiles_matches_oracle(M, O, dev, inter, codes_480):
    """The wide GEMM shape (128-route descriptors x 512 weight rows: 256 gate
    rows with the matching 256 up rows for gate/up, 512 output columns for
    down; taken when experts average at least 48 routes): 300 tokens x top-4
    over 8 experts with skewed counts (descriptors full, part-filled and
    single groups), hidden 640 (the down GEMM's second item ends 384 rows
    past the matrix: whole wavefronts past it re-read its last 8 rows, its
    last scale block clamped), intermediate 384 (the second gate/up item
    half past the matrix: a partial last gate tile), 256 (one whole
    gate/up item) or 128 (the down GEMM one 128-deep stage, so its first
    stage is its last), the shared expert as dense
    descriptors in the same launches; with 0x7F / 0xFF codes in the routed
    gate/up and down weights, the fixup path of both modes (also on the
    partial gate tile at intermediate 256).  Against the oracle's Direct
    MoE."""
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=640, intermediate=inter, experts=8, top_k=4, limit=7.0)
    bank, shared, _ = syn.synth_layer(cfg, seed=131, device=dev)
    if codes_480:
        bank.gate_up_weight[1, ::7, ::13] = 0x7F
        bank.gate_up_weight[0, 5::11, 3::17] = 0xFF
        bank.down_weight[2, ::9, 1::7] = 0x7F
    gate = WeightedGate(8, 4, seed=13)
    T = 300
    x = syn.normal_bf16((1, T, cfg.hidden_size), syn.key(131, "wide"), device=dev)
    ids, sc = (t.reshape(T, 4).cpu().numpy() for t in gate(x))
    counts = np.bincount(ids.reshape(-1), minlength=8)
    assert counts.max() > 128 and counts.min() < 96, counts
    y = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)(x)
    want = O.direct_moe(to_bits(x).reshape(T, -1), host_bank(bank), ids, sc, cfg.swiglu_limit, host_shared(shared))
    assert_parity(to_bits(y).reshape(T, -1), want, O)


def test_wide_gemm_full_width_with_480_codes_matches_oracle(M, O, dev):
    """The wide GEMM shape at the model's widths (hidden 4,096: 32 stages of
    the gate/up K loop; intermediate 1,536: 12 of the down one), 8 experts
    with skewed counts, so that descriptors of every pair count from full
    (the next stage's weight tiles issued one per pair) to one pair run,
    with 0x7F / 0xFF codes in the routed gate/up and down weights (the
    fixup path of both modes) and the shared expert as dense descriptors.
    Against the oracle's Direct MoE."""
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=4096, intermediate=1536, experts=8, top_k=4, limit=7.0)
    bank, shared, _ = syn.synth_layer(cfg, seed=171, device=dev)
    bank.gate_up_weight[3, ::11, ::29] = 0x7F
    bank.gate_up_weight[0, 7::13, 5::31] = 0xFF
    bank.down_weight[1, ::17, 2::11] = 0xFF
    gate = WeightedGate(8, 4, seed=17)
    T = 300
    x = syn.normal_bf16((1, T, cfg.hidden_size), syn.key(171, "wide-full"), device=dev)
    ids, sc = (t.reshape(T, 4).cpu().numpy() for t in gate(x))
    counts = np.bincount(ids.reshape(-1), minlength=8)
    assert counts.max() > 128 and counts.min() < 96, counts
    y = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)(x)
    want = O.direct_moe(to_bits(x).reshape(T, -1), host_bank(bank), ids, sc, cfg.swiglu_limit, host_shared(shared))
    assert_parity(to_bits(y).reshape(T, -1), want, O)


@pytest.mark.parametrize("shared_experts", [1, 2])
def test_prefill_shared_expert_merged_or_separate_matches_oracle(M, O, dev, shared_experts):
    """A shared expert of the routed width runs as extra dense descriptors
    inside the routed GEMM launches; two shared experts (width 2 I) take the
    separate dense GEMM pair.  Both against the oracle's Direct MoE."""
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=32, top_k=8, limit=7.0, shared=shared_experts)
    bank, shared, gate = syn.synth_layer(cfg, seed=51 + shared_experts, device=dev)
    moe = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)
    T = 96
    x = syn.normal_bf16((1, T, cfg.hidden_size), syn.key(51, shared_experts), device=dev)
    y = moe(x)
    ids, sc = (t.reshape(T, 8).cpu().numpy() for t in gate(x))
    xb = to_bits(x).reshape(T, -1)
    want = O.direct_moe(xb, host_bank(bank), ids, sc, cfg.swiglu_limit, host_shared(shared))
    assert_parity(to_bits(y).reshape(T, -1), want, O)


def test_prefill_shared_rows_follow_each_calls_routes(M, O, dev):
    """The merged shared expert's hidden rows sit right after the call's
    routed rows (rows R .. R + T - 1, R = T k of that call) and share one
    split launch with them: calls of 300, 96 and 300 tokens on one plan
    (wide shape, 32-route shape, wide again), each against the oracle."""
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=32, top_k=8, limit=7.0, shared=1)
    bank, shared, gate = syn.synth_layer(cfg, seed=71, device=dev)
    moe = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)
    for call, T in enumerate((300, 96, 300)):
        x = syn.normal_bf16((1, T, cfg.hidden_size), syn.key(71, call), device=dev)
        y = moe(x)
        ids, sc = (t.reshape(T, 8).cpu().numpy() for t in gate(x))
        xb = to_bits(x).reshape(T, -1)
        want = O.direct_moe(xb, host_bank(bank), ids, sc, cfg.swiglu_limit, host_shared(shared))
        assert_parity(to_bits(y).reshape(T, -1), want, O)


@pytest.mark.parametrize("which", ["gate", "up", "down"])
@pytest.mark.parametrize("shared_experts", [1, 2])
def test_prefill_480_codes_in_one_shared_weight(M, O, dev, shared_experts, which):
    """0x7F / 0xFF codes (+-480) in one shared weight only: the routed
    problem's flag stays clear while the shared items (merged into the routed
    launches, or the separate pair) must take the fixup path; without it the
    MFMA would read those codes as NaN."""
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=32, top_k=8, limit=7.0, shared=shared_experts)
    bank, shared, gate = syn.synth_layer(cfg, seed=61 + shared_experts, device=dev)
    w = getattr(shared, f"{which}_proj").weight
    w[::7, ::13] = 0x7F
    w[3::11, 5::17] = 0xFF
    moe = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)
    T = 80
    x = syn.normal_bf16((1, T, cfg.hidden_size), syn.key(61, shared_experts), device=dev)
    y = moe(x)
    ids, sc = (t.reshape(T, 8).cpu().numpy() for t in gate(x))
    want = O.direct_moe(to_bits(x).reshape(T, -1), host_bank(bank), ids, sc, cfg.swiglu_limit, host_shared(shared))
    assert_parity(to_bits(y).reshape(T, -1), want, O)


@pytest.mark.parametrize("reduction", ["grouped", "direct"])
def test_prefill_hc_expand_epilogue_matches_plain_then_oracle(M, O, dev, reduction):
    """glm53_prefill_moe_hc: the hyper-connection expand fused into the
    reduction equals the oracle's expand (metal:2362-2388) applied to the
    plain prefill output, bit for bit."""
    import torch

    N = submodule("_native")
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=32, top_k=8, limit=7.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=91, device=dev)
    T = 70
    x = syn.normal_bf16((T, 512), syn.key(91, "x"), device=dev)
    rng = np.random.default_rng(91)
    residual = from_bits(O.f32_to_bf16(rng.normal(size=(T, 4, 512)).astype(np.float32)), dev)
    post = torch.from_numpy(rng.normal(size=(T, 4)).astype(np.float32)).to(dev)
    comb = torch.from_numpy(rng.normal(size=(T, 4, 4)).astype(np.float32)).to(dev)
    plan = M.PrefillPlan(512, 256, 256, 32, 8, T, 7.0)
    red = N.REDUCE_DIRECT if reduction == "direct" else N.REDUCE_GROUPED
    plain = torch.empty((T, 512), dtype=torch.bfloat16, device=dev)
    plan.run(bank, shared, gate, x, T, None, None, red, plain, dev)
    hc = torch.empty((T, 4, 512), dtype=torch.bfloat16, device=dev)
    plan.run_hc(bank, shared, gate, x, T, None, None, red, residual, post, comb, hc, dev)
    want = O.hc_expand(to_bits(plain), to_bits(residual), post.cpu().numpy(), comb.cpu().numpy())
    assert np.array_equal(to_bits(hc), want)


def test_prefill_4096_tokens_matches_oracle(M, O, dev):
    """A long prompt on a small layer: 32,768 routes (128 route-count blocks,
    the many-token router, the wide GEMM shape) against the oracle's
    Direct MoE."""
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=32, top_k=8, limit=7.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=101, device=dev)
    T = 4096
    x = syn.normal_bf16((1, T, 512), syn.key(101, "x"), device=dev)
    y = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)(x)
    ids, sc = (t.reshape(T, 8).cpu().numpy() for t in gate(x))
    want = O.direct_moe(to_bits(x).reshape(T, -1), host_bank(bank), ids, sc, cfg.swiglu_limit, host_shared(shared))
    assert_parity(to_bits(y).reshape(T, -1), want, O)


@pytest.mark.parametrize("tokens", [300, 2048])
def test_prefill_graph_replays_match_eager(M, dev, tokens):
    """A prefill (many-token BF16-MFMA router, route plan, grouped GEMMs --
    the 64-route shape at 300 tokens, the wide shape at 2,048 -- and the
    reduction) captured in a HIP graph: every replay, with eager work and
    synchronisations between replays, equals the eager output bit for bit."""
    import torch

    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=32, top_k=8, limit=7.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=111, device=dev)
    moe = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)
    x = syn.normal_bf16((1, tokens, 512), syn.key(111, "x", tokens), device=dev)
    eager = moe(x).clone()
    torch.cuda.synchronize(dev)
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        moe(x)  # warm the capture stream's plan (plans are per stream) and the cached code flags
    torch.cuda.current_stream(dev).wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = moe(x)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize(dev)
        assert torch.equal(out, eager), i
        noise = syn.normal_bf16((1, tokens, 512), syn.key(111, "noise", i), device=dev)
        with torch.cuda.stream(stream):
            moe(noise)  # eager work on the captured plan (same stream) between replays
        torch.cuda.synchronize(dev)
    plan = moe._prefill_plans[(dev.index, stream.cuda_stream)]
    assert plan.dynamic_allocation_count == 0 and plan.host_synchronization_count == 0
    assert plan.execution_count == 5  # warm-up, capture, three eager calls (replays are not calls)
    assert len(plan.buffer_identities) == 16


def test_prefill_plan_growth_keeps_captured_plans_alive(M, dev):
    """A call with more tokens than the stream's plan holds replaces the plan;
    a graph captured with the old one still replays correctly (its arena is
    retired with the module, not freed)."""
    import torch

    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=32, top_k=8, limit=7.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=113, device=dev)
    moe = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)
    x = syn.normal_bf16((1, 64, 512), syn.key(113, "x"), device=dev)
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        eager = moe(x).clone()
    torch.cuda.current_stream(dev).wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = moe(x)
    with torch.cuda.stream(stream):
        moe(syn.normal_bf16((1, 600, 512), syn.key(113, "long"), device=dev))  # grows the plan past 256 tokens
    torch.cuda.synchronize(dev)
    assert len(moe._retired_prefill_plans) == 1
    torch.cuda.empty_cache()
    filler = torch.full((64 << 20,), 7, dtype=torch.uint8, device=dev)  # reuse of freed memory would show
    graph.replay()
    torch.cuda.synchronize(dev)
    assert torch.equal(out, eager)
    del filler


def test_config5_zipf_2048_tokens_matches_oracle(M, O, dev, config5):
    """BASELINE config 5 as bench.py runs it: 2,048 tokens on the config-2
    layer (seed of the bench) with the Zipf(1.1) router bias -> 16,384
    routes, heavy experts with over 5% of the routes (several 128-route
    descriptors of one expert, the wide GEMM shape) and many experts under
    10 routes; the
    many-token router above 1,024 tokens.  Every token's selection is
    checked against the oracle's router (near-tie rule); the MoE output of
    every token against the oracle's Direct MoE (BASELINE gates) and, for
    each reduction, against the oracle's same-order combine with the
    elementwise gate as well (grouped_fp8.py:279-328), on the device's
    selection and the touched experts."""
    cfg, bank, shared, gate, x, tokens = config5
    ids_d, sc_d = gate(x.reshape(tokens, -1))
    ids, sc = ids_d.cpu().numpy(), sc_d.cpu().numpy()
    counts = np.bincount(ids.reshape(-1), minlength=cfg.n_routed_experts)
    assert counts.max() / ids.size > 0.05, counts.max()
    assert (counts < 10).sum() >= 100, (counts < 10).sum()
    xb = to_bits(x).reshape(tokens, -1)
    from test_gpu_decode import _router_check

    _router_check(O, gate, xb, ids, sc)
    sub, local = _touched(bank, ids)
    want = O.moe_reductions(xb, sub, local, sc, cfg.swiglu_limit, host_shared(shared))
    for reduction in ("grouped", "direct"):
        y = M.SortedGroupedFP8MoE(bank, cfg, gate, shared, reduction=reduction)(x)
        got = to_bits(y).reshape(tokens, -1)
        assert_parity(got, want["direct"], O, elementwise=reduction == "direct")
        stats = assert_parity(got, want[reduction], O, exact_fraction=0.75)
        print(f"config 5 {reduction}: {stats}")


@pytest.fixture(scope="module")
def config5(dev):
    from conftest import pkg as package

    syn = submodule("synthetic")
    pkg = package()
    cfg = syn.layer_config()
    bank, shared, gate0 = syn.synth_layer(cfg, 20260901, 0, dev)  # bench.py's seed, layer 0
    gate = pkg.Float32Gate(gate0.weight, syn.zipf_bias(cfg.n_routed_experts).to(dev), top_k=8)
    tokens = 2048
    x = syn.normal_bf16((1, tokens, cfg.hidden_size), syn.key(20260901, "config5_2048_tokens_zipf"), device=dev)
    return cfg, bank, shared, gate, x, tokens


@pytest.mark.parametrize("tokens", [9, 256, 2048])
def test_direct_order_prefill_equals_direct_bit_for_bit(M, dev, config2_layer, tokens):
    """The Direct-order parity anchor (native_indexer_plan.metal:1997-2207;
    README.md:819-823 of the reference): DirectFP8MoE's host bucket loop
    (ascending experts, every bucket -- one-row buckets included -- on the
    FP8 MFMA tree, BF16 accumulation) and the fused grouped plan with
    reduction="direct" produce the same bytes, at 9 tokens (below the
    grouped threshold: called directly), 256 and 2,048 tokens (the
    many-token router)."""
    import torch

    syn = submodule("synthetic")
    cfg, bank, shared, gate = config2_layer
    x = syn.normal_bf16((1, tokens, cfg.hidden_size), syn.key(4242, "anchor", tokens), device=dev)
    direct = M.PackedFP8MoE(bank, cfg, gate, shared)  # T > 1: the Direct semantics over the bank's experts
    exact = M.SortedGroupedFP8MoE(bank, cfg, gate, shared, min_routes=0, reduction="direct")
    want = direct(x)
    got = exact(x)
    torch.cuda.synchronize()
    ids, _ = gate(x.reshape(tokens, -1))
    singletons = int((torch.bincount(ids.reshape(-1).long(), minlength=cfg.n_routed_experts) == 1).sum())
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (tokens, singletons)


def test_custom_ops_compile_without_graph_breaks(M, dev):
    """The MoE modules call the glm53 custom ops: torch.compile with
    fullgraph=True (no graph break allowed) traces decode and prefill, and
    the compiled calls equal the eager ones bit for bit; torch.library.opcheck
    validates the FP8 linear op's registration (schema, fake tensor, AOT
    dispatch) against its real kernel."""
    import torch

    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=32, top_k=8, limit=7.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=131, device=dev)
    moe = M.SortedGroupedFP8MoE(bank, cfg, gate, shared)
    xd = syn.normal_bf16((1, 1, 512), syn.key(131, "d"), device=dev)
    xp = syn.normal_bf16((1, 96, 512), syn.key(131, "p"), device=dev)

    def step(a, b):
        return moe(a) * 2, moe(b) + 1

    compiled = torch.compile(step, fullgraph=True, backend="aot_eager")
    want = step(xd, xp)
    got = compiled(xd, xp)
    torch.cuda.synchronize()
    for g, w in zip(got, want):
        assert torch.equal(g.view(torch.int16), w.view(torch.int16))
    x = syn.normal_bf16((4, 256), syn.key(131, "lin"), device=dev)
    torch.library.opcheck(torch.ops.glm53.block_fp8_linear,
                          (x, shared.gate_proj.weight[:, :256].contiguous(),
                           shared.gate_proj.weight_scale_inv[:, :2].contiguous(), None),
                          test_utils=("test_schema", "test_faketensor", "test_aot_dispatch_dynamic"))
