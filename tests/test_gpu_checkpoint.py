"""GPU: a synthetic layer written as a block-FP8 safetensors checkpoint and
imported with checkpoint.load_moe_layer is byte-identical to the source
layer, and the packed decode and grouped prefill over it match the source
layer's outputs bit for bit and the oracle to the parity gates."""

from __future__ import annotations

import numpy as np
import pytest

from checkpoint_files import layer_tensors, write_checkpoint
from conftest import assert_parity, host_bank, host_shared, submodule, to_bits

pytestmark = pytest.mark.gpu


def _host(t):
    return t.detach().cpu().numpy()


def _as_tensors(bank, shared, gate, layer):
    sh = {p: (_host(getattr(shared, f"{p}_proj").weight), _host(getattr(shared, f"{p}_proj").weight_scale_inv))
          for p in ("gate", "up", "down")}
    gate_up, down = bank.reference_weights()  # a checkpoint holds the row-major layout
    return layer_tensors("model.language_model.", layer, _host(gate_up), _host(bank.gate_up_scale_inv),
                         _host(down), _host(bank.down_scale_inv), sh, _host(gate.weight),
                         _host(gate.e_score_correction_bias))


def test_imported_layer_matches_source(M, O, dev, tmp_path):
    import torch

    syn = submodule("synthetic")
    C = submodule("checkpoint")
    cfg = syn.layer_config(hidden=1024, intermediate=512, experts=32, top_k=8, limit=10.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=71, layer=5, device=dev)
    decoy = syn.synth_layer(cfg, seed=72, layer=4, device=dev)
    tensors = {**_as_tensors(bank, shared, gate, 5), **_as_tensors(*decoy, 4)}
    config = {"hidden_size": 1024, "moe_intermediate_size": 512, "swiglu_limit": 10.0, "n_routed_experts": 32,
              "num_experts_per_tok": 8, "n_shared_experts": 1, "routed_scaling_factor": gate.routed_scaling_factor,
              "norm_topk_prob": gate.norm_topk_prob}
    root = write_checkpoint(tmp_path / "ck", tensors, config, shards=3)
    b2, s2, g2 = C.load_moe_layer(root, 5, dev)
    assert b2.layout == bank.layout  # both the package's default layout
    for name in ("gate_up_weight", "gate_up_scale_inv", "down_weight", "down_scale_inv"):
        assert torch.equal(getattr(b2, name), getattr(bank, name)), name
    tiled, _, _ = C.load_moe_layer(root, 5, dev, layout="tiled")
    assert tiled.layout == "tiled" and not torch.equal(tiled.gate_up_weight, tiled.reference_weights()[0])
    for got, want in zip(tiled.reference_weights(), bank.reference_weights()):
        assert torch.equal(got, want)
    for p in ("gate", "up", "down"):
        assert torch.equal(getattr(s2, f"{p}_proj").weight, getattr(shared, f"{p}_proj").weight)
        assert torch.equal(getattr(s2, f"{p}_proj").weight_scale_inv, getattr(shared, f"{p}_proj").weight_scale_inv)
    assert torch.equal(g2.weight, gate.weight) and torch.equal(g2.e_score_correction_bias, gate.e_score_correction_bias)
    assert (g2.top_k, g2.routed_scaling_factor, g2.norm_topk_prob) == (8, gate.routed_scaling_factor,
                                                                         gate.norm_topk_prob)
    lcfg = C.layer_config(root)
    x1 = syn.normal_bf16((1, 1, 1024), syn.key(71, 1), device=dev)
    want = M.PackedFP8MoE(bank, cfg, gate, shared)(x1)
    got = M.PackedFP8MoE(b2, lcfg, g2, s2)(x1)
    assert torch.equal(got, want)
    xt = syn.normal_bf16((1, 300, 1024), syn.key(71, 300), device=dev)
    got_p = M.SortedGroupedFP8MoE(b2, lcfg, g2, s2)(xt)
    assert torch.equal(got_p, M.SortedGroupedFP8MoE(bank, cfg, gate, shared)(xt))
    ids, sc = (t.reshape(300, 8).cpu().numpy() for t in g2(xt))
    oracle = O.direct_moe(to_bits(xt).reshape(300, -1), host_bank(b2), ids, sc, 10.0, host_shared(s2))
    assert_parity(to_bits(got_p).reshape(300, -1), oracle, O)


def test_invalid_pairs_are_refused_before_any_copy(dev, tmp_path):
    import torch

    syn = submodule("synthetic")
    C = submodule("checkpoint")
    cfg = syn.layer_config(hidden=512, intermediate=256, experts=8, top_k=4, limit=10.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=73, device=dev)
    tensors = _as_tensors(bank, shared, gate, 0)
    tensors["model.language_model.layers.0.mlp.experts.3.down_proj.weight_scale_inv"] = torch.ones((4, 4))
    config = {"hidden_size": 512, "moe_intermediate_size": 256, "n_routed_experts": 8, "num_experts_per_tok": 4}
    root = write_checkpoint(tmp_path / "ck", tensors, config)
    with pytest.raises(C.CheckpointError, match="experts.3.down_proj.weight_scale_inv"):
        C.load_moe_layer(root, 0, dev)
