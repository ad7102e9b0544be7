"""Pin the oracle's number formats (CPU only).

The oracle encodes/decodes e4m3fn, fp16 and bf16 from the format definitions
(oracle/gdn_oracle.py numpy, oracle/fp8_quant.c integer arithmetic). The
reference gets the same conversions from torch's casts
(prototype/gdn_replay_fp8_reference.py:87,91,99,134): `.to(torch.float16)`,
`.to(torch.float8_e4m3fn)`, `.float()`. Here both restatements are checked
against those library casts on exhaustive or adversarial inputs: every code,
every rounding midpoint and its neighbours, saturation, subnormals, signed
zero, inf and NaN.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import fp8_quant, gdn_oracle


def torch_e4m3fn(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def torch_f16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float16).view(torch.int16).numpy().view(np.uint16)


def torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _neighbours(values: np.ndarray, ulps: int = 2) -> np.ndarray:
    """values and their fp32 neighbours within +-ulps (both signs)."""
    v = np.abs(np.asarray(values, dtype=np.float32))
    bits = v.view(np.int32)[:, None] + np.arange(-ulps, ulps + 1, dtype=np.int32)[None, :]
    bits = np.clip(bits, 0, 0x7F800000)
    out = bits.astype(np.int32).view(np.float32).ravel()
    return np.concatenate([out, -out])


def e4m3fn_probe_values() -> np.ndarray:
    table = gdn_oracle.E4M3FN_TABLE
    finite = np.unique(np.abs(table[~np.isnan(table)]))
    mids = (finite[:-1].astype(np.float64) + finite[1:]) / 2
    specials = np.array([0.0, 448.0, 464.0, 480.0, 500.0, 1e4, 2.0 ** -10, 2.0 ** -11, 1e-30, 1e-45,
                         np.inf, 2.0 ** -126, 2.0 ** -127], dtype=np.float64)
    base = np.concatenate([finite, mids, specials]).astype(np.float32)
    rng = np.random.default_rng(0)
    rand = np.concatenate([rng.uniform(-500, 500, 20000), rng.normal(0, 1e-2, 20000),
                           rng.normal(0, 1e-3, 5000)]).astype(np.float32)
    return np.concatenate([_neighbours(base), rand, [np.nan, -np.nan]]).astype(np.float32)


def test_e4m3fn_decode_every_code():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = gdn_oracle.e4m3fn_decode(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert nan.sum() == 2  # 0x7F and 0xFF only (no infinities in e4m3fn)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # the C decoder too (scale 1 through the block dequantiser)
    c_vals = fp8_quant.dequantize_vblock32(codes.reshape(1, 1, 2, 128).repeat(16, axis=2)[..., :32, :],
                                           np.ones((1, 1, 1), np.float16))
    c_codes = codes.reshape(1, 1, 2, 128).repeat(16, axis=2)[..., :32, :]
    assert np.array_equal(np.isnan(c_vals), np.isnan(gdn_oracle.e4m3fn_decode(c_codes)))


def test_e4m3fn_known_values():
    """Hand-derived anchors of the OCP e4m3fn format (bias 7, 3 mantissa bits)."""
    enc = gdn_oracle.e4m3fn_encode
    assert enc(np.float32(448.0)) == 0x7E          # max finite S.1111.110
    assert enc(np.float32(-448.0)) == 0xFE
    assert enc(np.float32(1.0)) == 0x38            # exponent 7 (bias), mantissa 0
    assert enc(np.float32(2.0 ** -6)) == 0x08      # smallest normal
    assert enc(np.float32(2.0 ** -9)) == 0x01      # smallest subnormal
    assert enc(np.float32(2.0 ** -10)) == 0x00     # tie to even (0)
    assert enc(np.float32(3 * 2.0 ** -10)) == 0x02 # tie 1.5 units -> 2 (even)
    assert enc(np.float32(1.0625)) == 0x38         # 1 + 1/16: tie between 1.0 and 1.125 -> even (1.0)
    assert enc(np.float32(1.1875)) == 0x3A         # 1 + 3/16: tie between 1.125 and 1.25 -> even (1.25)
    assert enc(np.float32(-0.0)) == 0x80
    assert enc(np.float32(np.nan)) & 0x7F == 0x7F


def test_e4m3fn_encode_matches_torch_cast():
    x = e4m3fn_probe_values()
    want = torch_e4m3fn(x)
    got_np = gdn_oracle.e4m3fn_encode(x)
    got_c = fp8_quant.e4m3fn_encode(x)
    nan = np.isnan(x)
    # NaN inputs: any NaN code (0x7F/0xFF) is acceptable -- sign of NaN is not a value
    for got in (got_np, got_c):
        assert np.all((got[nan] & 0x7F) == 0x7F)
        bad = np.nonzero(got[~nan] != want[~nan])[0]
        assert bad.size == 0, (x[~nan][bad[:5]], got[~nan][bad[:5]], want[~nan][bad[:5]])


def test_e4m3fn_encode_exhaustive_clamped_range():
    """Every fp32 in [-448, 448] whose top 20 bits vary (all rounding classes
    of e4m3fn's 3-bit mantissa: the 20 low bits are covered by a fixed
    pattern set: 0, 1, half-1, half, half+1, max)."""
    hi = np.arange(0, 0x43E0 + 1, dtype=np.uint32) << 16       # up to 448.0 = 0x43E00000
    lows = np.array([0, 1, 0x7FFFF, 0x80000, 0x80001, 0xFFFFF], dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    x = bits.view(np.float32)
    x = x[np.abs(x) <= 448.0]
    x = np.concatenate([x, -x])
    want = torch_e4m3fn(x)
    assert np.array_equal(gdn_oracle.e4m3fn_encode(x), want)
    assert np.array_equal(fp8_quant.e4m3fn_encode(x), want)


def test_f16_bits_matches_torch_cast():
    rng = np.random.default_rng(1)
    base = np.concatenate([
        rng.normal(0, 1, 20000), rng.uniform(-70000, 70000, 5000),
        np.exp2(rng.uniform(-30, -14, 20000)),           # fp16 subnormal range and below
        [0.0, 65504.0, 65519.99, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -25, 2.0 ** -14, 1e-8, np.inf],
    ]).astype(np.float32)
    x = np.concatenate([_neighbours(base, 1), [np.nan]]).astype(np.float32)
    want = torch_f16_bits(x)
    got_c = fp8_quant.f16_bits(x)
    got_np = np.asarray(x, np.float32).astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    for got in (got_c, got_np):
        assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)
        assert np.array_equal(got[~nan], want[~nan])


def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(2)
    base = np.concatenate([rng.normal(0, 1, 50000), np.exp2(rng.uniform(-140, 120, 20000)),
                           [0.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 3.3895e38]]).astype(np.float32)
    x = np.concatenate([_neighbours(base, 1), [np.nan, np.inf]]).astype(np.float32)
    want = torch_bf16_bits(x)
    got = gdn_oracle.bf16_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(np.isnan((got[nan].astype(np.uint32) << 16).view(np.float32)))
