"""GPU test of the allocation-free decode entry point, glm53_decode_moe_static,
called through the C ABI, against the plan form it mirrors
(glm53_decode_moe_ex with the whole stage mask).

Two calls in a row on one GPU's static scratch: the BASELINE config-2 layer
(H=4096, I=1536, 288 experts), then a smaller layer (H=1024, I=512, 32
experts), each with a separate residual and in place (out = x = residual);
both must equal the plan form bit for bit (same kernels, same inputs).
Shapes outside the limits are refused before any device work.
"""

from __future__ import annotations

import ctypes

import pytest

from conftest import submodule

pytestmark = pytest.mark.gpu


def _static(lib, N, cfg, bank, shared, gate, x, residual, out, dev):
    b, s, r = bank.as_c_struct(), shared.as_c_struct(), gate.as_c_struct()
    return lib.glm53_decode_moe_static(cfg.hidden_size, cfg.moe_intermediate_size, cfg.n_routed_experts,
                                       cfg.num_experts_per_tok, float(cfg.swiglu_limit), ctypes.byref(b),
                                       ctypes.byref(s), ctypes.byref(r), N.ptr(x), N.ptr(residual), N.ptr(out),
                                       N.stream_handle(dev))


@pytest.mark.parametrize("seed", [7])
def test_static_decode_equals_plan_decode_on_two_calls(dev, seed):
    import torch

    syn = submodule("synthetic")
    packed = submodule("packed")
    N = submodule("_native")
    lib = N.lib()
    shapes = [syn.layer_config(), syn.layer_config(hidden=1024, intermediate=512, experts=32, top_k=8, limit=10.0)]
    for i, cfg in enumerate(shapes):  # the second call is the smaller input
        bank, shared, gate = syn.synth_layer(cfg, seed=seed + i, device=dev)
        plan = packed.DecodePlan(cfg.hidden_size, cfg.moe_intermediate_size, cfg.moe_intermediate_size,
                                 cfg.n_routed_experts, 8, cfg.swiglu_limit)
        x = syn.normal_bf16((cfg.hidden_size,), syn.key(seed, i, "x"), device=dev)
        res = syn.normal_bf16((cfg.hidden_size,), syn.key(seed, i, "res"), device=dev)
        want = torch.empty_like(x)
        plan.step(bank, shared, gate, x, res, want, N.STAGE_ALL, dev)
        got = torch.full_like(x, float("nan"))
        N.check(_static(lib, N, cfg, bank, shared, gate, x, res, got, dev))
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (i, "separate residual")
        # in place, as the decoder step runs it
        xp, xs = x.clone(), x.clone()
        plan.step(bank, shared, gate, xp, xp, xp, N.STAGE_ALL, dev)
        N.check(_static(lib, N, cfg, bank, shared, gate, xs, xs, xs, dev))
        torch.cuda.synchronize()
        assert torch.equal(xs.view(torch.int16), xp.view(torch.int16)), (i, "in place")
        assert plan.error_flag() == 0
        del bank, shared, gate, plan
        torch.cuda.empty_cache()


def test_static_decode_refuses_inputs_beyond_its_limits(dev):
    import torch

    syn = submodule("synthetic")
    N = submodule("_native")
    lib = N.lib()
    cfg = syn.layer_config(hidden=1024, intermediate=512, experts=32, top_k=8, limit=10.0)
    bank, shared, gate = syn.synth_layer(cfg, seed=3, device=dev)
    x = syn.normal_bf16((1024,), syn.key(3), device=dev)
    out = torch.empty_like(x)
    b, s, r = bank.as_c_struct(), shared.as_c_struct(), gate.as_c_struct()
    P = ctypes.c_void_p
    cases = [
        ((1024, 384, 32, 8), "fused step shapes"),   # a width without step kernels
        ((1024, 512, 400, 8), "at most 320 experts"),
        ((1024, 512, 32, 9), "invalid dimensions"),
        ((1024, 512, 16, 8), "bank shape"),          # dimensions that disagree with the bank
    ]
    for (H, I, E, k), fragment in cases:
        rc = lib.glm53_decode_moe_static(H, I, E, k, 10.0, ctypes.byref(b), ctypes.byref(s), ctypes.byref(r),
                                         N.ptr(x), None, N.ptr(out), N.stream_handle(dev))
        assert rc == N.INVALID_ARGUMENT, fragment
        assert fragment in lib.glm53_last_error().decode(), (fragment, lib.glm53_last_error())
    rc = lib.glm53_decode_moe_static(1024, 512, 32, 8, 10.0, ctypes.byref(b), ctypes.byref(s), ctypes.byref(r),
                                     P(N.ptr(x).value + 2), None, N.ptr(out), N.stream_handle(dev))
    assert rc == N.INVALID_ARGUMENT and "aligned" in lib.glm53_last_error().decode()
