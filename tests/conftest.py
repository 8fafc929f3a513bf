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


def host_bank(bank):
    return SimpleNamespace(
        gate_up_weight=bank.gate_up_weight.cpu().numpy(),
        gate_up_scale_inv=bank.gate_up_scale_inv.cpu().numpy(),
        down_weight=bank.down_weight.cpu().numpy(),
        down_scale_inv=bank.down_scale_inv.cpu().numpy(),
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


def assert_parity(actual_bits, expected_bits, O, *, cos=0.9999, rel=2e-2, exact_fraction=None):
    """BASELINE gates: max-abs-rel <= 2e-2 (max |a-e| / max |e|) and cosine >= 0.9999.

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
    if exact_fraction is not None:
        assert stats["bit_exact_fraction"] >= exact_fraction, stats
    return stats
