"""CPU pins of the activation-split model (tests/e4m3_split.py)."""

from __future__ import annotations

import numpy as np

import e4m3_split as S


def _all_bf16_up_to_448() -> np.ndarray:
    pos = np.arange(0, 0x43E1, dtype=np.uint16)  # 0x43E0 = 448
    return np.concatenate([pos, pos | np.uint16(0x8000)])


def test_table_matches_oracle_lut(O):
    lut = O.e4m3_lut()
    assert np.array_equal(S.e4m3_table().astype(np.float32), lut[:127])
    assert S.e4m3_table()[126] == 448.0 and S.e4m3_table()[1] == 2.0 ** -9


def test_nearest_matches_torch_cast_on_every_bf16_value_in_range():
    import torch

    bits = _all_bf16_up_to_448()
    v = S.bf16_to_f32(bits)
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(S.nearest_e4m3(v), want)


def test_nearest_known_answers():
    cases = {1.0: 0x38, 1.0625: 0x38, 1.1875: 0x3A, -448.0: 0xFE, 500.0: 0x7E, 2.0 ** -10: 0x00,
             3 * 2.0 ** -10: 0x02, -(2.0 ** -12): 0x80, float("inf"): 0x7E, float("-inf"): 0xFE}
    got = S.nearest_e4m3(np.array(list(cases), np.float32))
    assert [int(c) for c in got] == list(cases.values())


def test_block_scale_puts_amax_in_the_top_binade():
    rng = np.random.default_rng(5)
    amax = np.float32(2.0) ** rng.uniform(-110, 120, size=4000).astype(np.float32)
    s = S.block_scale(amax)
    assert np.all(np.frexp(s)[0] == 0.5)  # powers of two
    ratio = amax.astype(np.float64) / s
    assert np.all((ratio > 224) & (ratio <= 448))
    assert np.array_equal(S.block_scale(np.array([0.0, np.inf, np.nan], np.float32)), np.ones(3, np.float32))


def test_split_reconstructs_within_the_residual_step():
    rng = np.random.default_rng(6)
    x = rng.normal(size=(8, 512)).astype(np.float32) * np.float32(2.0) ** rng.integers(-30, 30, size=(8, 1))
    bits = (x.view(np.uint32) >> 16).astype(np.uint16)
    hi, lo, scale = S.split(bits)
    v = S.bf16_to_f32(bits).astype(np.float64)
    s = np.repeat(scale, 128, axis=1).astype(np.float64)
    recon = s * (S.e4m3_signed_value(hi) + S.e4m3_signed_value(lo) / 16.0)
    # hi leaves |q - hi| <= 16; lo rounds 16 (q - hi) with a 3-bit mantissa
    # (or to the 2^-9 subnormal step), so |q - hi - lo / 16| <= |q - hi| / 16 + 2^-14.
    err = np.abs(v - recon) / s
    assert np.all(err <= np.abs(v / s - S.e4m3_signed_value(hi)) / 16 + 2.0 ** -14)
    assert np.all(err <= 1.0 + 2.0 ** -14)
