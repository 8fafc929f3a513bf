"""CPU tests of the layer-by-layer installer and the bank's storage contracts.

The installer cases follow the reference's tests/test_fp8_metal.py:240-329
(every Direct layer replaced one at a time, the report keys, a second call
converting nothing, the decode policy never installing grouped modules);
the reference runs them on Metal, here packing runs on host tensors (no
device work is needed to pack or to construct the modules).
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest

from conftest import submodule

torch = pytest.importorskip("torch")


def _model(layers: int, experts: int = 2):
    fp8 = submodule("fp8")
    config = SimpleNamespace(hidden_size=128, moe_intermediate_size=128, swiglu_limit=3.0, n_routed_experts=experts,
                             num_experts_per_tok=2)

    def gate(x):
        shape = (*x.shape[:-1], 2)
        return torch.zeros(shape, dtype=torch.int32), torch.ones(shape, dtype=torch.float32)

    rows = [SimpleNamespace(mlp=fp8.DirectFP8MoE(config, gate, None), compile_ffn=True) for _ in range(layers)]
    for i, row in enumerate(rows):
        for e, expert in enumerate(row.mlp.experts):
            for j, proj in enumerate((expert.gate_proj, expert.up_proj, expert.down_proj)):
                proj.weight.fill_((i * 31 + e * 7 + j) % 120)  # distinct bytes per (layer, expert, projection)
    return SimpleNamespace(language_model=SimpleNamespace(model=SimpleNamespace(layers=rows))), rows


def test_grouped_installer_replaces_every_direct_layer_once():
    loader = submodule("loader")
    grouped = submodule("grouped_fp8")
    model, rows = _model(3)
    before = [[(e.gate_proj.weight.clone(), e.up_proj.weight.clone(), e.down_proj.weight.clone())
               for e in row.mlp.experts] for row in rows]
    report = loader.install_packed_grouped_moe(model)
    assert report["converted_layers"] == [0, 1, 2]
    assert report["converted_count"] == 3
    assert report["remaining_direct_layers"] == []
    assert report["all_old_expert_modules_detached"]
    assert report["backend"] == "packed-grouped" and report["grouped_enabled"] is True
    assert all(isinstance(r.mlp, grouped.SortedGroupedFP8MoE) for r in rows)
    assert all(not hasattr(r.mlp, "experts") and not r.compile_ffn for r in rows)
    for row_report, row, experts in zip(report["layers"], rows, before):
        assert row_report["old_expert_count"] == 2
        assert row_report["bank_bytes"] == row.mlp.bank.nbytes
        bank = row.mlp.bank
        for e, (g, u, d) in enumerate(experts):  # the bank holds each expert's bytes where the layout says
            assert torch.equal(bank.gate_up_weight[e, :128], g) and torch.equal(bank.gate_up_weight[e, 128:], u)
            assert torch.equal(bank.down_weight[e], d)
        assert all(c["ownership"] == "owned" for c in bank.storage_contracts.values())
    assert model._glm53_moe_backend == "packed-grouped"
    assert model._glm53_packed_grouped_report is report
    second = loader.install_packed_grouped_moe(model)
    assert second["converted_count"] == 0 and second["remaining_direct_layers"] == []


def test_decode_installer_never_installs_grouped_modules():
    loader = submodule("loader")
    packed = submodule("packed")
    grouped = submodule("grouped_fp8")
    model, rows = _model(2)
    report = loader.install_packed_decode_moe(model)
    assert report["converted_count"] == 2
    assert report["backend"] == "packed-decode" and report["grouped_enabled"] is False
    assert all(type(r.mlp) is packed.PackedFP8MoE for r in rows)
    assert not any(isinstance(r.mlp, grouped.SortedGroupedFP8MoE) for r in rows)
    assert model._glm53_packed_decode_report is report
    assert loader.install_packed_decode_moe(model)["converted_count"] == 0
    # a packed-decode layer cannot be re-packed as grouped in place
    with pytest.raises(ValueError, match="in place"):
        loader.install_packed_grouped_moe(model)


def test_bank_refuses_bare_and_ephemeral_storage():
    """PackedFP8ExpertBank takes storage leases (reference ownership.py:
    13-198): a bare tensor has no lifetime contract, an ephemeral lease must
    be materialised first, a borrowed-stable lease keeps its owner."""
    own = submodule("ownership")
    packed = submodule("packed")
    gu = torch.zeros((2, 256, 128), dtype=torch.uint8)
    gus = torch.ones((2, 2, 1), dtype=torch.float32)
    dw = torch.zeros((2, 128, 128), dtype=torch.uint8)
    dws = torch.ones((2, 1, 1), dtype=torch.float32)
    with pytest.raises(TypeError, match="TensorLease"):
        packed.PackedFP8ExpertBank(gu, gus, dw, dws, intermediate_size=128)
    eph = own.borrowed_ephemeral_tensor(gu)
    with pytest.raises(own.TensorOwnershipError, match="materialize_owned"):
        packed.PackedFP8ExpertBank(eph, own.owned_tensor(gus), own.owned_tensor(dw), own.owned_tensor(dws),
                                   intermediate_size=128)
    owner = object()
    bank = packed.PackedFP8ExpertBank(own.materialize_owned(eph), own.borrowed_stable_tensor(gus, owner=owner),
                                      own.owned_tensor(dw), own.owned_tensor(dws), intermediate_size=128)
    assert bank.storage_contracts["gate_up_weight"] == {"ownership": "owned", "layout": "row-major-contiguous"}
    assert bank.storage_contracts["gate_up_scale_inv"]["ownership"] == "borrowed-stable"
    assert owner in bank._storage_owners
    assert bank.gate_up_weight.data_ptr() != gu.data_ptr()  # materialised: shares nothing with the staging copy
    with pytest.raises(own.TensorOwnershipError, match="owner"):
        own.borrowed_stable_tensor(gu, owner=None)
    with pytest.raises(own.TensorOwnershipError):
        own.ResidentTensor(gu, own.TensorOwnership.OWNED, own.TensorLayout.UNKNOWN)
    with pytest.raises(ValueError, match="layout mismatch"):
        packed.PackedFP8ExpertBank(own.owned_tensor(gu), own.owned_tensor(gus), own.owned_tensor(dw[:, :64]),
                                   own.owned_tensor(dws), intermediate_size=128)


def test_pack_rejects_mixed_shapes_and_dtypes():
    fp8 = submodule("fp8")
    packed = submodule("packed")
    experts = [fp8.DirectFP8Expert(128, 128, 10.0) for _ in range(3)]
    bank = packed.PackedFP8ExpertBank.pack(experts)
    assert tuple(bank.gate_up_weight.shape) == (3, 256, 128) and bank.expert_count == 3
    odd = fp8.DirectFP8Expert(128, 256, 10.0)
    with pytest.raises(ValueError, match="expert 1 gate_proj"):
        packed.PackedFP8ExpertBank.pack([experts[0], odd])
    experts[2].down_proj.weight_scale_inv = experts[2].down_proj.weight_scale_inv.double()
    with pytest.raises(ValueError, match="expert 2 down_proj"):
        packed.PackedFP8ExpertBank.pack(experts)
    with pytest.raises(ValueError):
        packed.PackedFP8ExpertBank.pack([])
