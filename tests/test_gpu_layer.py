"""GPU parity of the one-launch decode layer (layer.hip) against the
three-launch kernels and the CPU oracle.

Both forms compute the same roundings (T(gate), T(up), SwiGLU, T(down),
ordered FP32 slot sum); they differ in the FP32 summation order inside a
down-projection row (one wavefront vs one half-wavefront per row) and of
the router logits, so outputs agree to within the BF16 rounding of those
sums: checked against each other with the tolerance gates and a floor on
bit-identical outputs, and against the CPU oracle.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity, host_shared, submodule, to_bits

pytestmark = pytest.mark.gpu


def _layer(dev, hidden, intermediate, experts, seed):
    syn = submodule("synthetic")
    cfg = syn.layer_config(hidden=hidden, intermediate=intermediate, experts=experts, top_k=8, limit=10.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=seed, device=dev)
    return cfg, bank, shared, gate


@pytest.fixture(scope="module")
def small(dev):
    return _layer(dev, 1024, 512, 32, 31)


@pytest.fixture(scope="module")
def config2(dev):
    return _layer(dev, 4096, 1536, 288, 32)


def _plans(cfg):
    packed = submodule("packed")
    N = submodule("_native")
    H, I, E = cfg.hidden_size, cfg.moe_intermediate_size, cfg.n_routed_experts
    single = packed.DecodePlan(H, I, I, E, 8, cfg.swiglu_limit)
    single.set_mode(N.DECODE_SINGLE_LAUNCH)
    three = packed.DecodePlan(H, I, I, E, 8, cfg.swiglu_limit)
    three.set_mode(N.DECODE_THREE_LAUNCH)
    return single, three


def _bits_equal(a, b):
    import torch

    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("which", ["small", "config2"])
def test_routed_single_launch_matches_three_launch(which, small, config2, dev, O):
    """Given ids, over several calls (the launch epoch advances every call),
    with and without the shared expert."""
    import torch

    syn = submodule("synthetic")
    cfg, bank, shared, gate = small if which == "small" else config2
    single, three = _plans(cfg)
    rng = np.random.default_rng(4)
    for step in range(5):
        x = syn.normal_bf16((cfg.hidden_size,), syn.key(40, which, step), device=dev)
        ids = torch.as_tensor(rng.choice(cfg.n_routed_experts, 8, replace=False).astype(np.int32), device=dev)
        sc = torch.as_tensor(rng.uniform(0.05, 0.3, 8).astype(np.float32), device=dev)
        sh = shared if step % 2 == 0 else None
        y1 = torch.empty_like(x)
        y3 = torch.empty_like(x)
        single.routed(bank, sh, x, ids, sc, y1, dev)
        three.routed(bank, sh, x, ids, sc, y3, dev)
        torch.cuda.synchronize()
        assert_parity(to_bits(y1).reshape(-1), to_bits(y3).reshape(-1), O, exact_fraction=0.95)
    assert single.error_flag() == 0 and three.error_flag() == 0


@pytest.mark.parametrize("which", ["small", "config2"])
def test_router_single_launch_matches_oracle(which, small, config2, dev, O):
    """Router in the launch: ids vs the oracle (near-tie rule), the published
    ids / scores, and the output against the oracle on the touched experts."""
    import torch

    from test_gpu_decode import _router_check, _touched_bank

    syn = submodule("synthetic")
    cfg, bank, shared, gate = small if which == "small" else config2
    single, three = _plans(cfg)
    hs = host_shared(shared)
    N = submodule("_native")
    for step in range(3):
        x = syn.normal_bf16((cfg.hidden_size,), syn.key(41, which, step), device=dev)
        y1 = torch.empty_like(x)
        ids_d = torch.empty(8, dtype=torch.int32, device=dev)
        sc_d = torch.empty(8, dtype=torch.float32, device=dev)
        single.full(bank, shared, gate, x, y1, ids_d, sc_d, dev)
        y3 = torch.empty_like(x)
        three.full(bank, shared, gate, x, y3, None, None, dev)
        torch.cuda.synchronize()
        xb = to_bits(x).reshape(-1)
        ids, sc = ids_d.cpu().numpy()[None], sc_d.cpu().numpy()[None]
        _router_check(O, gate, xb[None], ids, sc)
        want = O.decode_moe(xb, _touched_bank(bank, ids[0]), np.arange(8), sc[0], cfg.swiglu_limit, hs)
        assert_parity(to_bits(y1).reshape(-1), want, O, exact_fraction=0.9)
        st = O.compare(to_bits(y1).reshape(-1), to_bits(y3).reshape(-1))
        assert st["cosine"] >= 0.9999 and st["max_abs_rel"] <= 2e-2, st
    assert single.error_flag() == 0
    assert N.DECODE_SINGLE_LAUNCH == 1


def test_in_place_residual_step_and_graph_replay(config2, dev, O):
    """Decoder-step form out = T(x + T(moe(x))) written in place over x, as
    the benchmark runs it: a captured graph of 3 single-launch layers
    replays to exactly the bits of the same layers run eagerly, replay after
    replay with eager work in between (the epoch and ticket counters live on
    the device), and agrees with the three-launch form within the gates."""
    import torch

    syn = submodule("synthetic")
    N = submodule("_native")
    cfg, bank, shared, gate = config2
    single, three = _plans(cfg)
    x0 = syn.normal_bf16((cfg.hidden_size,), syn.key(42), device=dev)

    def run(plan, x):
        for _ in range(3):
            plan.step(bank, shared, gate, x, x, x, N.STAGE_ALL, dev)

    eager = x0.clone()
    run(single, eager)
    ref3 = x0.clone()
    run(three, ref3)
    torch.cuda.synchronize()
    st = O.compare(to_bits(eager).reshape(-1), to_bits(ref3).reshape(-1))
    assert st["cosine"] >= 0.9999 and st["max_abs_rel"] <= 2e-2, st

    xg = x0.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(single, xg)
    for rep in range(4):
        xg.copy_(x0)
        g.replay()
        other = x0.clone()
        run(single, other)  # eager launches of the same plan between replays
        torch.cuda.synchronize()
        assert _bits_equal(xg, eager), rep
        assert _bits_equal(other, eager), rep
    assert single.error_flag() == 0


def test_single_launch_bad_expert_id_flags_and_nans(small, dev):
    import torch

    syn = submodule("synthetic")
    cfg, bank, shared, gate = small
    single, _ = _plans(cfg)
    x = syn.normal_bf16((cfg.hidden_size,), syn.key(43), device=dev)
    ids = torch.tensor([0, 1, 2, 3, 4, 5, 6, 1000], dtype=torch.int32, device=dev)
    sc = torch.full((8,), 0.125, device=dev)
    y = torch.empty_like(x)
    single.routed(bank, shared, x, ids, sc, y, dev)
    torch.cuda.synchronize()
    assert single.error_flag() & 1
    assert torch.isnan(y.float()).all()
    # the next call is clean again
    ids[7] = 7
    single.routed(bank, shared, x, ids, sc, y, dev)
    torch.cuda.synchronize()
    assert single.error_flag() == 0
    assert torch.isfinite(y.float()).all()
