"""GPU parity of BASELINE config 3 -- the benchmark's workload -- against the
CPU oracle.

bench.py times one decoder step over 42 distinct config-2 layers (H=4096,
I=1536, 288 experts top-8 + one shared expert, FP32 router): for each layer
the three-launch step of glm53_decode_moe_ex with the whole stage mask and
x, residual and out all the same buffer, i.e. x <- T(x + T(moe(x))) in
place, captured as one HIP graph.  Here the same 42 layers (229 GB of
weights, the bench's seeds) run that exact call eagerly for three steps;
after every layer the device state is read back and checked against the
oracle on the device's own input:

* the selected ids against the oracle's FP32 router (set-equal except a
  near-tie within 1 FP32 ulp) and the scores to 2e-6 relative;
* x_out against O.add_bf16(x_in, O.decode_moe(x_in, touched experts,
  device ids / scores, shared)) -- the reference's decode composition
  (packed.py:896-923) plus the decoder's BF16 residual add -- under the
  BASELINE gates, a floor on bit-identical outputs, and the reference's
  elementwise gate on the summed parts (conftest.assert_residual_parity);
* the plan's error flag stays clear.

Then the 42-layer step is captured in a HIP graph and replayed: every
replay (with eager steps of the same plans between replays) reproduces the
eager run's final state bit for bit.
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from conftest import assert_residual_parity, host_bank, host_shared, submodule, to_bits

pytestmark = pytest.mark.gpu

LAYERS = 42
SEED = 20260901  # bench.py's weight seed


@pytest.fixture(scope="module")
def stack(dev):
    import torch

    torch.cuda.empty_cache()
    syn = submodule("synthetic")
    packed = submodule("packed")
    cfg = syn.layer_config()
    H, I, E = cfg.hidden_size, cfg.moe_intermediate_size, cfg.n_routed_experts
    layers = []
    for layer in range(LAYERS):
        bank, shared, gate = syn.synth_layer(cfg, SEED, layer, dev)
        bank.code_flags()
        layers.append(SimpleNamespace(bank=bank, shared=shared, gate=gate,
                                      plan=packed.DecodePlan(H, I, I, E, 8, cfg.swiglu_limit)))
    torch.cuda.synchronize()
    yield cfg, layers
    layers.clear()
    torch.cuda.empty_cache()


def _touched(bank, ids):
    return host_bank(bank, ids)


def _run_step(layers, x, dev, N):
    for l in layers:
        l.plan.step(l.bank, l.shared, l.gate, x, x, x, N.STAGE_ALL, dev)


def test_config3_in_place_residual_stack_matches_oracle(stack, dev, O):
    import torch

    from test_gpu_decode import _router_check

    syn = submodule("synthetic")
    N = submodule("_native")
    cfg, layers = stack
    hosts = {}
    worst = 1.0
    finals = []
    for step in range(3):
        x = syn.normal_bf16((cfg.hidden_size,), syn.key(SEED, "config3", step), device=dev)
        x0 = x.clone()
        for li, l in enumerate(layers):
            x_in = to_bits(x).reshape(-1)
            l.plan.step(l.bank, l.shared, l.gate, x, x, x, N.STAGE_ALL, dev)
            torch.cuda.synchronize()
            ids = l.plan.debug_scratch(1).cpu().numpy()
            scores = l.plan.debug_scratch(2).cpu().numpy()
            _router_check(O, l.gate, x_in[None], ids[None], scores[None])
            if li not in hosts:
                hosts[li] = host_shared(l.shared)
            moe, parts = O.decode_moe(x_in, _touched(l.bank, ids), np.arange(8), scores, cfg.swiglu_limit, hosts[li],
                                      return_stages=True)
            want = O.add_bf16(x_in, moe)
            st = assert_residual_parity(to_bits(x).reshape(-1), want, x_in, (parts.routed, parts.shared, moe), O,
                                        exact_fraction=0.9)
            worst = min(worst, st["bit_exact_fraction"])
        finals.append((x0, x.clone()))
    assert all(l.plan.error_flag() == 0 for l in layers)
    print(f"config 3: 3 steps x {LAYERS} layers checked, worst bit-exact fraction {worst:.4f}")

    # the captured 42-layer step replays to the eager bits, with eager steps between replays
    xg = torch.empty_like(finals[0][0])
    graph = torch.cuda.CUDAGraph()
    xg.copy_(finals[0][0])
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        _run_step(layers, xg, dev, N)
    for rep in range(3):
        x0, want = finals[rep % len(finals)]
        xg.copy_(x0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(xg.view(torch.int16), want.view(torch.int16)), rep
        other = finals[(rep + 1) % len(finals)][0].clone()
        _run_step(layers, other, dev, N)  # eager work on the same plans between replays
        torch.cuda.synchronize()
        assert torch.equal(other.view(torch.int16), finals[(rep + 1) % len(finals)][1].view(torch.int16)), rep
    assert all(l.plan.error_flag() == 0 for l in layers)


def test_stage_masks_compose_to_the_whole_step(stack, dev):
    """Router + gate/up, then down alone with no router (the routed launches
    read the plan's selection): equals the whole mask bit for bit."""
    import torch

    syn = submodule("synthetic")
    N = submodule("_native")
    cfg, layers = stack
    l = layers[0]
    x = syn.normal_bf16((cfg.hidden_size,), syn.key(SEED, "masks"), device=dev)
    whole = torch.empty_like(x)
    l.plan.step(l.bank, l.shared, l.gate, x, x, whole, N.STAGE_ALL, dev)
    split = torch.empty_like(x)
    l.plan.step(l.bank, l.shared, l.gate, x, x, split, N.STAGE_ROUTER | N.STAGE_GATE_UP, dev)
    l.plan.step(l.bank, l.shared, None, x, x, split, N.STAGE_DOWN, dev)
    torch.cuda.synchronize()
    assert torch.equal(whole.view(torch.int16), split.view(torch.int16))
    assert l.plan.error_flag() == 0


def test_out_of_range_expert_id_flags_and_nans(dev):
    """A caller id >= E never reads out of bounds: its slot is NaN, the
    layer output is NaN and error-flag bit 0 is raised; the next clean call
    is finite again."""
    import torch

    syn = submodule("synthetic")
    packed = submodule("packed")
    cfg = syn.layer_config(hidden=1024, intermediate=512, experts=32, top_k=8, limit=10.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=43, device=dev)
    plan = packed.DecodePlan(1024, 512, 512, 32, 8, 10.0)
    x = syn.normal_bf16((1024,), syn.key(43), device=dev)
    ids = torch.tensor([0, 1, 2, 3, 4, 5, 6, 1000], dtype=torch.int32, device=dev)
    sc = torch.full((8,), 0.125, device=dev)
    y = torch.empty_like(x)
    plan.routed(bank, shared, x, ids, sc, y, dev)
    torch.cuda.synchronize()
    assert plan.error_flag() == 1
    assert torch.isnan(y.float()).all()
    ids[7] = 7
    plan.routed(bank, shared, x, ids, sc, y, dev)
    torch.cuda.synchronize()
    assert plan.error_flag() == 0
    assert torch.isfinite(y.float()).all()
