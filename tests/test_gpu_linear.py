"""GPU parity: block_fp8_linear (fp8.py:254-299) and the SwiGLU epilogue."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from conftest import assert_parity, from_bits, random_codes, submodule, to_bits

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _linear(M, dev, x_bits, codes, scale):
    import torch

    x = from_bits(x_bits, dev)
    w = torch.from_numpy(codes).to(dev)
    s = torch.from_numpy(scale).to(dev)
    return to_bits(M.block_fp8_linear(x, w, s))


def test_config1_gemv_matches_oracle(M, O, dev):
    """x bf16 [1,4096] ~N(0,1), W E4M3 [4096,4096] from N(0,0.02)."""
    rng = np.random.default_rng(1)
    w = rng.normal(0.0, 0.02, size=(4096, 4096)).astype(np.float32)
    codes, scale = O.quantize_e4m3_blocks(w)
    x = O.f32_to_bf16(rng.normal(size=(1, 4096)).astype(np.float32))
    got = _linear(M, dev, x, codes, scale)
    want = O.fp8_linear(x, codes, scale)
    assert_parity(got, want, O, exact_fraction=0.97)


@pytest.mark.parametrize("k,n", [(1024, 256), (1536, 512), (2048, 130), (4096, 64)])
def test_gemv_random_codes_decode_like_reference_lut(M, O, dev, k, n):
    """Random codes 0..246 include 0x7F, which the reference LUT decodes to
    480 (fp8.py:22-27); the exact E4M3->FP16 register decode must agree."""
    rng = np.random.default_rng(k + n)
    codes = random_codes(rng, (n, k))
    scale = (rng.uniform(size=(-(-n // 128), k // 128)) * 0.002).astype(np.float32)
    x = O.f32_to_bf16((rng.normal(size=(1, k)) * 2).astype(np.float32))
    got = _linear(M, dev, x, codes, scale)
    want = O.fp8_linear(x, codes, scale)
    assert_parity(got, want, O, exact_fraction=0.98)


@pytest.mark.parametrize("k,n", [(12288, 200), (16384, 130), (65536, 8)])
@pytest.mark.parametrize("with_480", [False, True])
def test_wide_gemv_split_k_matches_oracle(M, O, dev, k, n, with_480):
    """One-row linear with K a multiple of 4096 above 8192 (an attention
    output projection is 16384 wide): one wavefront per 4096-wide K part,
    parts added in order.  Codes with 0x7F/0xFF take the exact software
    decode, codes without them the hardware one."""
    rng = np.random.default_rng(k + n + with_480)
    if with_480:
        codes = random_codes(rng, (n, k))
    else:
        codes = (rng.integers(0, 0x7F, size=(n, k)) | (rng.integers(0, 2, size=(n, k)) << 7)).astype(np.uint8)
    scale = (rng.uniform(size=(-(-n // 128), k // 128)) * 0.002).astype(np.float32)
    x = O.f32_to_bf16((rng.normal(size=(1, k)) * 2).astype(np.float32))
    got = _linear(M, dev, x, codes, scale)
    want = O.fp8_linear(x, codes, scale)
    assert_parity(got, want, O, exact_fraction=0.98)


def test_reference_kat_non_aligned_129x257(M, O, dev):
    """tests/test_fp8_metal.py:23-39: 129 x 257 crosses both block edges;
    error vs the dequantised matmul <= 0.03125."""
    rng = np.random.default_rng(7)
    m, k = 129, 257
    codes = random_codes(rng, (m, k))
    scale = (rng.uniform(size=(2, 3)) * 0.02).astype(np.float32)
    x = O.f32_to_bf16(rng.normal(size=(2, k)).astype(np.float32))
    got = _linear(M, dev, x, codes, scale)
    dense = O.dequantize(codes, scale)
    expected = O.f32_to_bf16((O.bf16_to_f32(x).astype(np.float64) @ dense.T).astype(np.float32))
    err = np.max(np.abs(O.bf16_to_f32(got) - O.bf16_to_f32(expected)))
    assert err <= 0.03125
    assert_parity(got, O.fp8_linear(x, codes, scale), O, exact_fraction=0.97)


@pytest.mark.parametrize("rows", [2, 7, 8, 9, 33, 100])
def test_multi_row_mfma_path_matches_oracle(M, O, dev, rows):
    """M > 1 with K % 128 == 0 runs the FP8 MFMA GEMM on the exact hi/lo
    activation split; the result must match the FP32-exact oracle."""
    rng = np.random.default_rng(rows)
    k, n = 512, 144
    w = rng.normal(0.0, 0.02, size=(n, k)).astype(np.float32)
    codes, scale = O.quantize_e4m3_blocks(w)
    x = O.f32_to_bf16(rng.normal(size=(rows, k)).astype(np.float32))
    got = _linear(M, dev, x, codes, scale)
    assert_parity(got, O.fp8_linear(x, codes, scale), O, exact_fraction=0.97)


@pytest.mark.parametrize("rows", [1, 5, 64])
def test_both_480_codes_gemv_and_mfma(M, O, dev, rows):
    """Codes over the whole byte range, so 0x7F (+480) and 0xFF (-480) both
    occur: the reference LUT decodes them as finite +-480 (fp8.py:22-27),
    OCP E4M3 (and the MFMA) as NaN.  M = 1 takes the register-decode GEMV,
    M > 1 the MFMA GEMM with its chained +-32 correction."""
    rng = np.random.default_rng(480 + rows)
    k, n = 1024, 272
    codes = random_codes(rng, (n, k), high=256)
    codes[:, :8] = 0xFF  # every row carries both signs
    codes[:, 8:16] = 0x7F
    scale = (rng.uniform(size=(-(-n // 128), k // 128)) * 0.002).astype(np.float32)
    x = O.f32_to_bf16(rng.normal(size=(rows, k)).astype(np.float32))
    got = _linear(M, dev, x, codes, scale)
    want = O.fp8_linear(x, codes, scale)
    assert np.isfinite(O.bf16_to_f32(got)).all()
    # full-range codes spread the products over ~2^16: more FP32 sums land
    # one BF16 ulp from the exact one than for checkpoint-like weights
    assert_parity(got, want, O, exact_fraction=0.95)


def test_input_layout_invariance(M, O, dev):
    """tests/test_metal_input_layout.py:27-95: strided / offset inputs give
    byte-identical results to row-contiguous ones."""
    import torch

    rng = np.random.default_rng(3)
    k, n = 1024, 256
    codes = random_codes(rng, (n, k))
    scale = (rng.uniform(size=(2, 8)) * 0.002).astype(np.float32)
    w = torch.from_numpy(codes).to(dev)
    s = torch.from_numpy(scale).to(dev)
    for tokens in (1, 7, 8, 9, 127, 128, 129, 255, 256, 1023, 1024):
        base = from_bits(O.f32_to_bf16(rng.normal(size=(tokens, 2 * k)).astype(np.float32)), dev)
        strided = base[:, ::2]
        contiguous = strided.contiguous()
        a = M.block_fp8_linear(strided, w, s)
        b = M.block_fp8_linear(contiguous, w, s)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), tokens


def test_sigmoid_matches_reference_exhaustive_sweep_hash(M, dev):
    """The device sigmoid over all 33,346 finite BF16 values in [-10, 10]
    hashes to the MLX reference hash recorded by the reference's sweep."""
    import torch

    golden = json.loads((GOLDEN / "sigmoid_sweep.json").read_text())
    bits = np.arange(1 << 16, dtype=np.uint16)
    vals = (bits.astype(np.uint32) << 16).view(np.float32)
    domain = bits[np.isfinite(vals) & (np.abs(vals) <= np.float32(10.0))]
    assert hashlib.sha256(domain.tobytes()).hexdigest() == golden["domain_bits_sha256"]
    N = submodule("_native")
    g = from_bits(domain, dev)
    out = torch.empty_like(g)
    N.check(N.lib().glm53_sigmoid_bf16(N.ptr(g), g.numel(), N.ptr(out), N.stream_handle(dev)))
    got = to_bits(out)
    assert hashlib.sha256(got.tobytes()).hexdigest() == golden["reference_sigmoid_sha256"]


def test_sigmoid_every_bf16_pattern_matches_oracle(O, dev):
    """The device sigmoid (the hardware-exponential form every SwiGLU uses,
    with its correctly rounding fallback for |g| > 87 and the fast::exp
    point) on all 65,536 BF16 patterns equals the oracle's MLX sigmoid bit
    for bit on every non-NaN input (NaN in, NaN out)."""
    import torch

    N = submodule("_native")
    bits = np.arange(1 << 16, dtype=np.uint16)
    vals = (bits.astype(np.uint32) << 16).view(np.float32)
    g = from_bits(bits, dev)
    out = torch.empty_like(g)
    N.check(N.lib().glm53_sigmoid_bf16(N.ptr(g), g.numel(), N.ptr(out), N.stream_handle(dev)))
    got = to_bits(out)
    ok = ~np.isnan(vals)
    want = O.sigmoid_bf16(bits[ok])
    bad = np.flatnonzero(got[ok] != want)
    assert bad.size == 0, [(hex(int(bits[ok][i])), hex(int(got[ok][i])), hex(int(want[i]))) for i in bad[:8]]
    nan_out = (got[~ok] & 0x7F80) == 0x7F80
    assert nan_out.all() and (got[~ok] & 0x007F).all()


def test_swiglu_bit_exact_against_oracle(M, O, dev):
    rng = np.random.default_rng(11)
    bits = np.arange(1 << 16, dtype=np.uint16)
    vals = (bits.astype(np.uint32) << 16).view(np.float32)
    gate = bits[np.isfinite(vals) & (np.abs(vals) <= 40.0)]
    up = O.f32_to_bf16(rng.normal(scale=6.0, size=gate.size).astype(np.float32))
    for limit in (10.0, 3.0, 20.0):
        got = to_bits(M.swiglu(from_bits(gate, dev), from_bits(up, dev), limit))
        assert np.array_equal(got, O.swiglu(gate, up, limit)), limit


def test_swiglu_every_gate_pattern_matches_oracle(M, O, dev):
    """The straight-line SwiGLU (two values per conversion, the form of the
    grouped GEMM epilogues) with its fall-back to the exact sequence, over
    all 65,536 BF16 gate patterns (NaN, +-inf, |g| > 87 and 0xC0DB included)
    against up values with +-0, +-inf, NaN and values past the clamp: equal
    to the oracle bit for bit wherever the oracle's result is not NaN, NaN
    where it is."""
    rng = np.random.default_rng(12)
    gate = np.arange(1 << 16, dtype=np.uint16)
    up = O.f32_to_bf16(rng.normal(scale=12.0, size=gate.size).astype(np.float32))
    special = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0xFFC1, 0x3F80, 0xBF80, 0x4120, 0xC120],
                       dtype=np.uint16)
    pick = rng.choice(gate.size, size=4096, replace=False)
    up[pick] = special[rng.integers(0, special.size, size=pick.size)]
    # an odd count: the last value is paired with itself
    gate, up = gate[:-1], up[:-1]
    for limit in (7.0, 10.0, float("inf")):
        got = to_bits(M.swiglu(from_bits(gate, dev), from_bits(up, dev), limit))
        want = O.swiglu(gate, up, limit)
        nan_want = (want & 0x7F80) == 0x7F80
        nan_want &= (want & 0x007F) != 0
        bad = np.flatnonzero(~nan_want & (got != want))
        assert bad.size == 0, (limit, [(hex(int(gate[i])), hex(int(up[i])), hex(int(got[i])), hex(int(want[i])))
                                       for i in bad[:8]])
        assert ((got[nan_want] & 0x7F80) == 0x7F80).all() and (got[nan_want] & 0x007F).all(), limit
