"""GPU tests of the re-laid expert bank (row groups, glm53_moe.h glm53_bank).

The layout is this build's own (the reference reads row-major [E, rows,
cols] banks, packed.py:782-850), so it is pinned by an independent NumPy
formulation (a reshape / transpose, not the kernel's index formula) and
round trips; every kernel family that reads a bank -- the three-launch
decode step, the any-shape decode, the routed diagnostic, the narrow and
wide grouped GEMMs -- must give the same bits from a row-major bank and
from its re-laid copy, since only addresses change.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import submodule, to_bits

pytestmark = pytest.mark.gpu


def _numpy_groups(w: np.ndarray, g: int) -> np.ndarray:
    """[E, N, K] row-major -> row groups of 2^g rows: group-major, then
    128-column block, then row within the group, then column."""
    E, N, K = w.shape
    r = 1 << g
    return w.reshape(E, N // r, r, K // 128, 128).transpose(0, 1, 3, 2, 4).reshape(E, N, K)


@pytest.mark.parametrize("g", [1, 4, 5, 7])
def test_relayout_matches_numpy_formulation(dev, g):
    import torch

    N = submodule("_native")
    rng = np.random.default_rng(g)
    w = rng.integers(0, 256, size=(3, 256, 384), dtype=np.int64).astype(np.uint8)
    src = torch.from_numpy(w).to(dev)
    dst = torch.empty_like(src)
    N.relayout(src, dst, 0, g)
    back = torch.empty_like(src)
    N.relayout(dst, back, g, 0)
    other = torch.empty_like(src)
    N.relayout(dst, other, g, 2)  # group to group
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), _numpy_groups(w, g))
    assert np.array_equal(back.cpu().numpy(), w)
    assert np.array_equal(other.cpu().numpy(), _numpy_groups(w, 2))


def test_relayout_refuses_overlap_and_bad_shapes(dev):
    import torch

    N = submodule("_native")
    w = torch.zeros((2, 64, 256), dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="overlap"):
        N.relayout(w, w, 0, 4)
    with pytest.raises(ValueError, match="multiple of the row group"):
        N.relayout(w, torch.empty_like(w), 0, 7)  # 64 rows, groups of 128
    odd = torch.zeros((2, 64, 200), dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="cols % 128"):
        N.relayout(odd, torch.empty_like(odd), 0, 4)


def test_synthetic_bank_is_the_same_matrices_in_either_layout(dev):
    import torch

    syn = submodule("synthetic")
    rows = syn.synth_bank(6, 512, 256, seed=5, device=dev, layout="rows")
    tiled = syn.synth_bank(6, 512, 256, seed=5, device=dev, layout="tiled")
    assert (rows.layout, tiled.layout) == ("rows", "tiled")
    gu, dw = tiled.reference_weights()
    assert torch.equal(gu, rows.gate_up_weight) and torch.equal(dw, rows.down_weight)
    assert torch.equal(tiled.gate_up_scale_inv, rows.gate_up_scale_inv)
    assert not torch.equal(tiled.gate_up_weight, rows.gate_up_weight)
    gu3, dw3 = tiled.reference_weights([4, 1])
    assert torch.equal(gu3, rows.gate_up_weight[[4, 1]]) and torch.equal(dw3, rows.down_weight[[4, 1]])


def test_relayout_in_place_needs_owned_weights(dev):
    import torch

    syn = submodule("synthetic")
    own = submodule("ownership")
    packed = submodule("packed")
    bank = syn.synth_bank(4, 256, 128, seed=9, device=dev, layout="rows")
    before = bank.gate_up_weight.clone(), bank.down_weight.clone()
    ptr = bank.gate_up_weight.data_ptr()
    bank.relayout_("tiled")
    assert bank.layout == "tiled" and bank.gate_up_weight.data_ptr() == ptr  # in place
    assert not torch.equal(bank.gate_up_weight, before[0])
    bank.relayout_(5).relayout_("rows")
    assert torch.equal(bank.gate_up_weight, before[0]) and torch.equal(bank.down_weight, before[1])
    borrowed = packed.PackedFP8ExpertBank(*(own.borrowed_stable_tensor(t, owner=bank) for t in
                                            (bank.gate_up_weight, bank.gate_up_scale_inv, bank.down_weight,
                                             bank.down_scale_inv)), intermediate_size=128)
    with pytest.raises(ValueError, match="borrows"):
        borrowed.relayout_("tiled")
    with pytest.raises(ValueError, match="multiples of 128"):
        syn.synth_bank(2, 257, 129, seed=1, device=dev, layout="rows").relayout_("tiled")


def _layer_pair(syn, cfg, seed, dev):
    a = syn.synth_layer(cfg, seed, device=dev, layout="rows")
    b = syn.synth_layer(cfg, seed, device=dev, layout="tiled")
    assert a[0].layout == "rows" and b[0].layout == "tiled"
    return a, b


@pytest.mark.parametrize("hidden,inter", [(1024, 512), (4096, 1536), (768, 384)])
def test_decode_bits_do_not_depend_on_the_layout(dev, hidden, inter):
    """(1024, 512) and (4096, 1536) run the three-launch step, (768, 384)
    the any-shape decode kernels; router, routed and residual forms."""
    import torch

    syn = submodule("synthetic")
    packed = submodule("packed")
    N = submodule("_native")
    E = 288 if hidden == 4096 else 32
    cfg = syn.layer_config(hidden=hidden, intermediate=inter, experts=E, top_k=8, limit=10.0)
    (ba, sa, ga), (bb, sb, gb) = _layer_pair(syn, cfg, 77, dev)
    plans = [packed.DecodePlan(hidden, inter, inter, E, 8, cfg.swiglu_limit) for _ in range(2)]
    ids = torch.tensor([3, 17, 0, 29, 5, 11, 30, 8], dtype=torch.int32, device=dev)
    sc = torch.linspace(0.2, 0.05, 8, device=dev)
    for step in range(2):
        x = syn.normal_bf16((hidden,), syn.key(77, step), device=dev)
        res = syn.normal_bf16((hidden,), syn.key(78, step), device=dev)
        outs = []
        for plan, (bank, shared, gate) in zip(plans, ((ba, sa, ga), (bb, sb, gb))):
            y_full, y_routed, y_res = (torch.empty_like(x) for _ in range(3))
            plan.full(bank, shared, gate, x, y_full, None, None, dev)
            plan.routed(bank, shared, x, ids, sc, y_routed, dev)
            plan.step(bank, shared, gate, x, res, y_res, N.STAGE_ALL, dev)
            outs.append((y_full, y_routed, y_res))
        torch.cuda.synchronize()
        for ya, yb in zip(*outs):
            assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))
        assert torch.isfinite(outs[0][0].float()).all()


@pytest.mark.parametrize("hidden,inter,experts,tokens", [(1024, 512, 32, 40), (1024, 512, 16, 80),
                                                         (4096, 1536, 288, 256), (640, 384, 8, 300),
                                                         (1024, 512, 8, 700)])
def test_prefill_bits_do_not_depend_on_the_layout(dev, M, hidden, inter, experts, tokens):
    """32-route and 64-route descriptors (few routes per expert), the wide
    128-route shape (many), both reductions, the shared expert merged into
    the routed launches."""
    import torch

    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=hidden, intermediate=inter, experts=experts, top_k=8, limit=7.0)
    (ba, sa, ga), (bb, sb, gb) = _layer_pair(syn, cfg, 91, dev)
    x = syn.normal_bf16((1, tokens, hidden), syn.key(91, "x"), device=dev)
    for reduction in ("grouped", "direct"):
        ya = M.SortedGroupedFP8MoE(ba, cfg, ga, sa, min_routes=1, reduction=reduction)(x)
        yb = M.SortedGroupedFP8MoE(bb, cfg, gb, sb, min_routes=1, reduction=reduction)(x)
        torch.cuda.synchronize()
        assert torch.equal(ya.view(torch.int16), yb.view(torch.int16)), reduction
        assert torch.isfinite(ya.float()).all()


def test_routed_diagnostic_reads_either_layout(dev, M):
    import torch

    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=1024, intermediate=512, experts=32, top_k=8, limit=10.0)
    (ba, _, _), (bb, _, _) = _layer_pair(syn, cfg, 13, dev)
    x = syn.normal_bf16((1024,), syn.key(13, "d"), device=dev)
    ids = torch.tensor([31, 2, 9, 0, 4, 18, 7, 22], dtype=torch.int32, device=dev)
    got = []
    for bank in (ba, bb):
        diag = M.RoutedDiagnostic(32, hidden_size=1024, intermediate_size=512)
        diag.execute(x, ids, bank.gate_up_weight, bank.gate_up_scale_inv, layout=bank.layout)
        torch.cuda.synchronize()
        got.append([to_bits(getattr(diag, s)) for s in ("gate", "up", "hidden")])
    for a, b in zip(*got):
        assert np.array_equal(a, b)


def test_bank_import_owns_a_relaid_copy(dev):
    """glm53_bank_import through the C ABI: the handle's weights are the
    tiled bytes of the source bank, its scales a copy, and a decode through
    the handle equals the Python tiled bank's bit for bit after the source
    buffers are freed."""
    import torch

    syn = submodule("synthetic")
    packed = submodule("packed")
    N = submodule("_native")
    cfg = syn.layer_config(hidden=1024, intermediate=512, experts=32, top_k=8, limit=10.0)
    (ba, sa, ga), (bb, sb, gb) = _layer_pair(syn, cfg, 55, dev)
    desc = ba.as_c_struct()
    handle = ctypes.POINTER(N.Bank)()
    N.check(N.lib().glm53_bank_import(ctypes.byref(desc), N.TILED_LAYOUT, N.stream_handle(dev),
                                      ctypes.byref(handle)))
    try:
        b = handle.contents
        assert b.row_group_log2 == N.TILED_LAYOUT and b.gate_up_weight != desc.gate_up_weight
        torch.cuda.synchronize()

        def owned(address, like):  # a view of handle-owned device bytes shaped like `like`
            return packed._device_view(address, like.numel(), torch.int32).view(torch.uint8).reshape(like.shape)

        assert torch.equal(owned(b.gate_up_weight, bb.gate_up_weight), bb.gate_up_weight)
        assert torch.equal(owned(b.down_weight, bb.down_weight), bb.down_weight)
        del desc, ba  # the source may go once the import returned
        torch.cuda.empty_cache()
        plan = packed.DecodePlan(1024, 512, 512, 32, 8, cfg.swiglu_limit)
        x = syn.normal_bf16((1024,), syn.key(55, "x"), device=dev)
        y_handle, y_bank = torch.empty_like(x), torch.empty_like(x)
        s, r = sb.as_c_struct(), gb.as_c_struct()
        N.check(N.lib().glm53_decode_moe(plan.handle, handle, ctypes.byref(s), ctypes.byref(r), N.ptr(x),
                                         N.ptr(y_handle), None, None, N.stream_handle(dev)))
        plan.full(bb, sb, gb, x, y_bank, None, None, dev)
        torch.cuda.synchronize()
        assert torch.equal(y_handle.view(torch.int16), y_bank.view(torch.int16))
    finally:
        torch.cuda.synchronize()
        N.lib().glm53_bank_destroy(handle)
