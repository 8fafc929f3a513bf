"""Shared fixtures: package import, oracle, BF16 <-> NumPy bit helpers."""

from __future__ import annotations

import importlib
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PACKAGE = "glm53-flash-mlx_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pkg():
    return importlib.import_module(PACKAGE)


def submodule(name: str):
    return importlib.import_module(f"{PACKAGE}.{name}")


@pytest.fixture(scope="session")
def O():
    from oracle import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def M():
    return pkg()


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a ROCm device")
    return torch.device("cuda:0")


def to_bits(t) -> np.ndarray:
    """BF16 torch tensor -> np.uint16 bit patterns (host)."""
    import torch

    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def from_bits(bits: np.ndarray, device):
    """np.uint16 BF16 bit patterns -> BF16 torch tensor on `device`."""
    import torch

    arr = np.ascontiguousarray(bits, dtype=np.uint16)
    return torch.from_numpy(arr.view(np.int16)).to(device).view(torch.bfloat16)


def host_bank(bank, expert_ids=None):
    """The bank (or the experts `expert_ids`, in that order) on the host in
    the reference row-major layout, whatever the device bank's layout, as
    the oracle reads it."""
    import torch

    gu, dw = bank.reference_weights(expert_ids)
    gus, dws = bank.gate_up_scale_inv, bank.down_scale_inv
    if expert_ids is not None:
        idx = torch.as_tensor(np.asarray(expert_ids, dtype=np.int64), device=gus.device).reshape(-1)
        gus, dws = gus.index_select(0, idx), dws.index_select(0, idx)
    return SimpleNamespace(
        gate_up_weight=gu.cpu().numpy(),
        gate_up_scale_inv=gus.cpu().numpy(),
        down_weight=dw.cpu().numpy(),
        down_scale_inv=dws.cpu().numpy(),
        intermediate_size=bank.intermediate_size,
    )


def host_shared(shared):
    if shared is None:
        return None
    return SimpleNamespace(
        gate=(shared.gate_proj.weight.cpu().numpy(), shared.gate_proj.weight_scale_inv.cpu().numpy()),
        up=(shared.up_proj.weight.cpu().numpy(), shared.up_proj.weight_scale_inv.cpu().numpy()),
        down=(shared.down_proj.weight.cpu().numpy(), shared.down_proj.weight_scale_inv.cpu().numpy()),
    )


def random_codes(rng, shape, high=247):
    """Random E4M3 codes as the reference tests draw them: randint(0, 247)
    (tests/test_fp8_metal.py:29), which includes 0x7F (= 480)."""
    return rng.integers(0, high, size=shape, dtype=np.int64).astype(np.uint8)


def assert_parity(actual_bits, expected_bits, O, *, cos=0.9999, rel=2e-2, exact_fraction=None, elementwise=True):
    """BASELINE gates: max-abs-rel <= 2e-2 (max |a-e| / max |e|) and cosine >= 0.9999,
    and (elementwise) the reference's own gate against Direct, every output
    within allclose(rtol=0.02, atol=0.02) (tests/test_fp8_metal.py:192).

    exact_fraction bounds the share of BF16 outputs equal to the oracle's bit
    for bit.  The oracle rounds the exact sum; an FP32 device sum lands one
    BF16 ulp away when it sits near a rounding midpoint (about 0.5% of
    outputs for the streaming GEMV, about 1.2% for the FP8 MFMA, whose
    128-deep internal accumulation is coarser than FP32), and a flipped
    gate/up value propagates through SwiGLU and the down projection, so
    whole-layer outputs share fewer exact bits than single projections."""
    stats = O.compare(actual_bits, expected_bits)
    assert stats["max_abs_rel"] <= rel, stats
    assert stats["cosine"] >= cos, stats
    if elementwise:
        assert stats["allclose_0_02"], stats
    if exact_fraction is not None:
        assert stats["bit_exact_fraction"] >= exact_fraction, stats
    return stats


def assert_residual_parity(actual_bits, expected_bits, x_bits, parts, O, *, exact_fraction=None):
    """Parity of a decoder-step output out = T(x + T(moe(x))) against the
    oracle's, where moe = T(T(routed) + T(shared)): the BASELINE gates on the
    output, and the reference's elementwise gate (0.02 + 0.02 |value|,
    tests/test_fp8_metal.py:192) applied to the terms that are summed --
    |out - want| <= 0.02 + 0.02 max |part| + one BF16 ulp of the largest of
    x and want.  `parts` are the oracle's BF16 routed, shared and moe
    vectors.  Where routed and shared, or x and moe, cancel, a within-gate
    difference (one ulp) of a large part survives in a small result, so the
    allowance follows the parts, not the result."""
    stats = assert_parity(actual_bits, expected_bits, O, exact_fraction=exact_fraction, elementwise=False)
    f = lambda b: O.bf16_to_f32(b).astype(np.float64).reshape(-1)  # noqa: E731
    a, e, x = f(actual_bits), f(expected_bits), f(x_bits)
    part = np.max(np.stack([np.abs(f(p)) for p in parts]), axis=0)
    big = np.maximum(np.abs(e), np.abs(x))
    ulp = np.exp2(np.floor(np.log2(np.maximum(big, 2.0 ** -126))) - 7)
    excess = np.abs(a - e) - (0.02 + 0.02 * part + ulp)
    assert np.all(excess <= 0), {"worst_excess": float(excess.max()), "index": int(excess.argmax())}
    return stats
