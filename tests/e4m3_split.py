"""Test model of the activation split that feeds the grouped FP8 GEMM.

Per row and 128-column block: s = 2^ceil(log2(amax / 448)) so amax / s lies
in (224, 448] (s = 1 for a zero or non-finite amax); q = x / s; hi =
E4M3(q); lo = E4M3(16 (q - hi)), round to nearest even, saturating at +-448,
the sign taken from q's sign bit.  The split has no counterpart in the
reference, which multiplies BF16 activations by dequantised weights
(grouped_fp8.py:206-262); this model is pinned in test_split_model.py against
the oracle's decode table (fp8.py:22-39) and torch's float8_e4m3fn cast.
"""

from __future__ import annotations

import numpy as np

BLOCK = 128


def e4m3_table() -> np.ndarray:
    """Magnitudes of codes 0x00..0x7E from the format: 3-bit mantissa m,
    4-bit exponent e, bias 7; e = 0 is subnormal (m * 2^-9)."""
    c = np.arange(127)
    e, m = c >> 3, c & 7
    return np.where(e == 0, m * 2.0 ** -9, (1 + m / 8.0) * 2.0 ** (e.astype(np.float64) - 7))


_TABLE = e4m3_table()


def nearest_e4m3(q) -> np.ndarray:
    """Round float32 values to E4M3 codes: nearest, ties to the even code,
    |q| >= 448 and NaN saturate to 0x7E; sign bit kept (so -0 -> 0x80)."""
    q = np.asarray(q, dtype=np.float32)
    mag = np.abs(q).astype(np.float64)
    idx = np.clip(np.searchsorted(_TABLE, np.nan_to_num(mag, nan=0.0)), 1, 126)
    below, above = _TABLE[idx - 1], _TABLE[idx]
    pick_above = (above - mag < mag - below) | ((above - mag == mag - below) & (idx % 2 == 0))
    code = np.where(pick_above, idx, idx - 1)
    code = np.where(~(mag < 448.0), 126, code)
    return (code | np.where(np.signbit(q), 0x80, 0)).astype(np.uint8)


def e4m3_signed_value(code) -> np.ndarray:
    code = np.asarray(code, dtype=np.int64)
    mag = _TABLE[np.minimum(code & 0x7F, 126)]
    return np.where(code & 0x80, -mag, mag).astype(np.float32)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def block_scale(amax: np.ndarray) -> np.ndarray:
    amax = np.asarray(amax, dtype=np.float32)
    out = np.ones(amax.shape, dtype=np.float32)
    for idx, a in np.ndenumerate(amax):
        if not (a > 0 and np.isfinite(a)):
            continue
        t = np.float32(a / np.float32(448.0))
        e = max(int(np.frexp(t)[1]) - 1, -126)  # ilogb
        s = np.float32(np.ldexp(np.float32(1.0), e))
        if np.float32(a / s) > np.float32(448.0):
            s = np.float32(np.ldexp(np.float32(1.0), e + 1))
        out[idx] = s
    return out


def split(x_bits: np.ndarray):
    """x_bits uint16 BF16 [rows, cols] -> hi u8 [rows, cols], lo u8, scale f32
    [rows, cols / 128]."""
    x = bf16_to_f32(x_bits)
    rows, cols = x.shape
    blocks = x.reshape(rows, cols // BLOCK, BLOCK)
    amax = np.fmax.reduce(np.abs(blocks), axis=-1, initial=np.float32(0.0))
    scale = block_scale(amax)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        q = (blocks * inv[..., None]).astype(np.float32)
        hi = nearest_e4m3(q)
        r = ((q - e4m3_signed_value(hi)) * np.float32(16.0)).astype(np.float32)
    lo = nearest_e4m3(r)
    return hi.reshape(rows, cols), lo.reshape(rows, cols), scale
