"""GPU: the activation split (glm53_split_activations) bit for bit against
the model in e4m3_split.py, over every BF16 value the E4M3 range can hold,
random block magnitudes, non-finite blocks, and both load layouts."""

from __future__ import annotations

import numpy as np
import pytest

import e4m3_split as S
from conftest import submodule

pytestmark = pytest.mark.gpu


def _run_split(bits: np.ndarray, dev, offset: int = 0, stride_pad: int = 0):
    import torch

    N = submodule("_native")
    rows, cols = bits.shape
    stride = cols + stride_pad
    padded = np.zeros((rows, stride), np.uint16)
    padded[:, :cols] = bits
    buf = torch.zeros(padded.size + offset, dtype=torch.int16, device=dev)
    buf[offset:].copy_(torch.from_numpy(padded.reshape(-1).view(np.int16)).to(dev))
    x = buf[offset:]
    hi = torch.empty((rows, cols), dtype=torch.uint8, device=dev)
    lo = torch.empty((rows, cols), dtype=torch.uint8, device=dev)
    scale = torch.empty((rows, cols // 128), dtype=torch.float32, device=dev)
    N.check(N.lib().glm53_split_activations(N.ptr(x), rows, cols, stride, N.ptr(hi), N.ptr(lo), N.ptr(scale),
                                            N.stream_handle(dev)))
    torch.cuda.synchronize(dev)
    return hi.cpu().numpy(), lo.cpu().numpy(), scale.cpu().numpy()


def _check(bits, dev, **layout):
    hi, lo, scale = _run_split(bits, dev, **layout)
    want_hi, want_lo, want_scale = S.split(bits)
    # IEEE 754 leaves the sign of a NaN product open: compare magnitudes there.
    nan = np.isnan(S.bf16_to_f32(bits))
    for got, want in ((hi, want_hi), (lo, want_lo)):
        got[nan] &= 0x7F
        want[nan] &= 0x7F
    assert np.array_equal(scale.view(np.uint32), want_scale.view(np.uint32))
    bad = np.argwhere(hi != want_hi)
    assert bad.size == 0, f"hi differs at {bad[:4].tolist()}: {hi[tuple(bad[0])]:#x} vs {want_hi[tuple(bad[0])]:#x}"
    bad = np.argwhere(lo != want_lo)
    assert bad.size == 0, f"lo differs at {bad[:4].tolist()}: {lo[tuple(bad[0])]:#x} vs {want_lo[tuple(bad[0])]:#x}"


def _exhaustive_rows(shift: int) -> np.ndarray:
    """Every BF16 value with |v| <= 448 (both signs), 127 per block with 448
    in column 0 so s = 1 (times 2^shift), four blocks per row."""
    pos = np.arange(0, 0x43E1, dtype=np.uint16)
    values = np.concatenate([pos, pos | np.uint16(0x8000)])
    per_block = 127
    nblocks = -(-values.size // per_block)
    nblocks += (-nblocks) % 4
    blocks = np.zeros((nblocks, 128), np.uint16)
    blocks[:, 0] = 0x43E0
    flat = blocks[:, 1:].reshape(-1)
    flat[:values.size] = values
    blocks[:, 1:] = flat.reshape(nblocks, per_block)
    x = S.bf16_to_f32(blocks) * np.float32(2.0) ** shift
    return (x.view(np.uint32) >> 16).astype(np.uint16).reshape(nblocks // 4, 512)


@pytest.mark.parametrize("shift", [0, -40, 17])
@pytest.mark.parametrize("offset", [0, 1])
def test_split_every_bf16_value_in_range(dev, shift, offset):
    _check(_exhaustive_rows(shift), dev, offset=offset)


@pytest.mark.parametrize("cols,offset,stride_pad", [(512, 0, 0), (384, 0, 8), (384, 1, 3), (128, 0, 0)])
def test_split_random_block_magnitudes(dev, cols, offset, stride_pad):
    rng = np.random.default_rng(cols + offset)
    rows = 67
    x = rng.normal(size=(rows, cols)).astype(np.float32)
    x *= np.float32(2.0) ** rng.integers(-126, 100, size=(rows, cols // 128)).repeat(128, axis=1).astype(np.float32)
    bits = (x.view(np.uint32) >> 16).astype(np.uint16)
    bits[3, :128] = 0                              # zero block: s = 1
    bits[4, 5] = 0x7F80                            # +inf: s = 1, values saturate
    bits[5, 7] = 0x7FC1                            # NaN: ignored by amax, encodes as saturated
    bits[6, 9] = 0xFFC0                            # negative NaN
    bits[7, :128] = 0x0001                         # BF16 subnormals only: s clamps at 2^-126
    bits[8, :128] = 0x7F7F                         # largest finite BF16
    _check(bits, dev, offset=offset, stride_pad=stride_pad)
