"""The flush requantiser's quotient (csrc/gdnr_device.h quotient_f64):
RN32(x * RN64(1 / s)) must equal the IEEE float32 quotient x / s that the
reference quantiser computes (prototype/gdn_replay_fp8_reference.py:36-37,
83-99: x / scale in fp32) for every x the flush feeds it: |x| <= amax, s =
amax / 448 rounded to float32, amax finite and s >= 2^-64.

numpy's float32 division is the IEEE quotient; numpy's float64 multiply and
float64 -> float32 cast are the two roundings of the device path. The cases
cover random blocks over the whole exponent range, quotients placed on f32
rounding midpoints' neighbourhoods and on e4m3 rounding midpoints, and the
block maximum itself (quotient 448 up to one ulp)."""

from __future__ import annotations

import numpy as np


def _device_quotient(x: np.ndarray, s: np.float32) -> np.ndarray:
    r64 = np.float64(1.0) / np.float64(s)
    return (x.astype(np.float64) * r64).astype(np.float32)


def _check(x: np.ndarray, s: np.float32) -> None:
    want = x / s                                   # float32 / float32: IEEE
    got = _device_quotient(x, s)
    assert want.dtype == np.float32 and got.dtype == np.float32
    bad = want.view(np.uint32) != got.view(np.uint32)
    assert not bad.any(), (x[bad][:4], s, want[bad][:4], got[bad][:4])


def test_random_blocks_all_exponents():
    rng = np.random.default_rng(0)
    for _ in range(200):
        e = rng.integers(-60, 60)
        x = (rng.standard_normal(20000) * np.exp2(e)).astype(np.float32)
        amax = np.float32(np.abs(x).max())
        s = np.float32(amax / np.float32(448.0))
        _check(x, s)
        _check(np.array([amax, -amax], dtype=np.float32), s)


def test_random_significands_fixed_scale():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 23, size=200000, dtype=np.uint32)
    for s_bits in rng.integers(0x1F800000, 0x60000000, size=50, dtype=np.uint32):  # s in [2^-64, 2^65)
        s = np.uint32(s_bits).view(np.float32)
        # x spanning [s, 448 s] over every significand
        for e in range(0, 9):
            x = ((bits | np.uint32(0x3F800000)).view(np.float32) * np.float32(2.0 ** e) * s).astype(np.float32)
            _check(x, s)


def test_near_f32_midpoints():
    """x chosen so that x / s lies within a few ulps of an f32 rounding
    midpoint (the cases a one-correction quotient gets wrong)."""
    rng = np.random.default_rng(2)
    for _ in range(100):
        s = np.float32(rng.uniform(1.0, 2.0) * 2.0 ** rng.integers(-30, 30))
        q = (rng.integers(1 << 23, 1 << 24, size=5000) * 2.0 ** rng.integers(-30, -14)).astype(np.float64)
        mid = q + 0.5 * np.spacing(q.astype(np.float32)).astype(np.float64)
        x0 = (mid * np.float64(s)).astype(np.float32)
        for d in range(-3, 4):
            x = (x0.view(np.uint32) + np.uint32(d & 0xFFFFFFFF)).view(np.float32)
            _check(x[np.isfinite(x)], s)


def test_near_e4m3_midpoints():
    """x / s close to the rounding midpoints of e4m3 (where the fp8 code turns)."""
    rng = np.random.default_rng(3)
    grid = []
    for e in range(-9, 9):                             # e4m3 normal and subnormal steps
        step = 2.0 ** (max(e, -6) - 3)
        grid.extend(np.arange(2.0 ** e, 2.0 ** (e + 1), step) + step / 2)
    grid = np.array([g for g in grid if g <= 464.0])
    for _ in range(50):
        s = np.float32(rng.uniform(1.0, 2.0) * 2.0 ** rng.integers(-40, 40))
        x0 = (grid * np.float64(s)).astype(np.float32)
        for d in range(-4, 5):
            x = (x0.view(np.uint32) + np.uint32(d & 0xFFFFFFFF)).view(np.float32)
            _check(np.concatenate([x, -x]), s)


def test_zero_signs_and_tiny():
    s = np.float32(3.0e-3)
    x = np.array([0.0, -0.0, 1e-45, -1e-45, 1e-38, -1e-38], dtype=np.float32)
    _check(x, s)
    got = _device_quotient(x, s)
    assert np.array_equal(np.signbit(got), np.signbit(x))
