"""Pin the oracle's vblock32 quantiser (CPU only).

Two restatements of prototype/gdn_replay_fp8_reference.py:36-37,40-106,109-134
are checked against each other bit for bit (numpy float ops with library
casts in oracle/gdn_oracle.py; integer arithmetic in oracle/fp8_quant.c) and
against hand-derived special cases chosen so that plausible mistakes fail:

* dividing by the fp16-ROUNDED scale instead of amax/448 (the reference's
  vblock branch divides by the unrounded fp32 scale, ref:83-86,94) fails
  ``test_fp16_scale_underflow_keeps_finite_codes``;
* a scale of 0 or NaN for an all-zero block (ref:36-37 uses 1) fails
  ``test_zero_block``;
* a per-row or per-tile amax instead of per-32-row block fails
  ``test_block_boundaries``;
* truncating instead of rounding the fp16 scale fails
  ``test_scale_rounds_to_nearest_even``.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import fp8_quant, gdn_oracle


def both(state):
    """(codes, scale f16, saturated-count) from each restatement."""
    state = np.asarray(state, dtype=np.float32)
    nq = gdn_oracle.quantize_checkpoint(state, "vblock", 32)
    c_codes, c_scale, c_sat = fp8_quant.quantize_vblock32(state)
    return nq, (c_codes, c_scale, c_sat)


def assert_same(nq, c):
    c_codes, c_scale, c_sat = c
    assert np.array_equal(nq.payload, c_codes)
    assert np.array_equal(nq.scale.view(np.uint16), c_scale.view(np.uint16))
    assert nq.saturation_fraction == pytest.approx(c_sat.sum() / nq.payload.size)


def test_random_states_agree():
    rng = np.random.default_rng(0)
    for scale in (1e-4, 0.02, 1.0, 300.0):
        state = (rng.standard_normal((2, 3, 64, 128)) * scale).astype(np.float32)
        # heavy tails: a few large entries per block
        state[..., ::17, ::29] *= 50
        nq, c = both(state)
        assert_same(nq, c)


def test_zero_block():
    state = np.zeros((1, 1, 32, 128), np.float32)
    state[0, 0, 3, 7] = -0.0
    nq, c = both(state)
    assert_same(nq, c)
    assert nq.scale.astype(np.float32)[0, 0, 0] == 1.0          # _safe_scale: amax == 0 -> 1
    assert np.all((nq.payload & 0x7F) == 0)
    assert nq.payload[0, 0, 3, 7] == 0x80                      # -0 keeps its sign


def test_fp16_scale_underflow_keeps_finite_codes():
    """amax = 1e-5: amax/448 = 2.2e-8 rounds to fp16 0 (below 2^-25), but the
    codes are computed with the unrounded scale, so they stay finite and the
    largest element encodes to 448; the dequantised block is all zero."""
    rng = np.random.default_rng(1)
    block = rng.uniform(-1, 1, (1, 1, 32, 128)).astype(np.float32)
    block *= np.float32(1e-5) / np.abs(block).max()
    nq, c = both(block)
    assert_same(nq, c)
    assert nq.scale[0, 0, 0] == 0.0
    assert not np.any((nq.payload & 0x7F) == 0x7F)              # no NaN codes
    amax_code = nq.payload.ravel()[np.argmax(np.abs(block))]
    assert amax_code & 0x7F == 0x7E                             # |x|/s = 448
    assert np.all(gdn_oracle.dequantize_vblock32(nq.payload, nq.scale) == 0)


def test_subnormal_fp16_scale():
    """amax = 448 * 2^-20 -> scale 2^-20, an fp16 subnormal (16 * 2^-24)."""
    block = np.zeros((1, 1, 32, 128), np.float32)
    block[0, 0, 0, 0] = np.float32(448.0 * 2.0 ** -20)
    block[0, 0, 5, 9] = np.float32(-3.0 * 2.0 ** -20)
    nq, c = both(block)
    assert_same(nq, c)
    assert nq.scale.view(np.uint16)[0, 0, 0] == 16
    assert nq.payload[0, 0, 0, 0] == 0x7E
    assert nq.payload[0, 0, 5, 9] == gdn_oracle.e4m3fn_encode(np.float32(-3.0))
    deq = gdn_oracle.dequantize_vblock32(nq.payload, nq.scale)
    assert deq[0, 0, 5, 9] == np.float32(-3.0 * 2.0 ** -20)


def test_scale_rounds_to_nearest_even():
    """amax/448 exactly halfway between two fp16 values -> the even one."""
    lo = np.float16(1.0)
    step = np.float32(2.0 ** -10)                               # fp16 ulp at 1.0
    for k, want_bits in ((1, 0x3C00), (3, 0x3C02)):             # 1 + 0.5 ulp -> 1.0; 1 + 1.5 ulp -> 1 + 2 ulp
        s32 = np.float32(1.0) + np.float32(k) * step / 2
        amax = np.float32(s32 * np.float32(448.0))
        assert np.float32(amax / np.float32(448.0)) == s32       # the tie survives the divide
        block = np.zeros((1, 1, 32, 128), np.float32)
        block[0, 0, 31, 127] = amax
        nq, c = both(block)
        assert_same(nq, c)
        assert nq.scale.view(np.uint16)[0, 0, 0] == want_bits, (k, hex(nq.scale.view(np.uint16)[0, 0, 0]))
    del lo


def test_block_boundaries():
    """One large value per 32-row block sets that block's scale only."""
    state = np.full((1, 2, 128, 128), 0.5, np.float32)
    peaks = {(0, 0): 1.0, (0, 1): 7.0, (0, 2): 0.5, (0, 3): 100.0, (1, 0): 2.0, (1, 1): 0.5, (1, 2): 3.0, (1, 3): 9.0}
    for (h, blk), peak in peaks.items():
        state[0, h, 32 * blk + 31, 0] = peak
    nq, c = both(state)
    assert_same(nq, c)
    for (h, blk), peak in peaks.items():
        assert nq.scale[0, h, blk] == np.float16(np.float32(peak) / np.float32(448.0))


def test_nan_block():
    """NaN amax: amax > 0 is false -> scale 1 (ref:36-37); NaN stays NaN
    through clamp and encodes to a NaN code, other values are x / 1."""
    block = np.full((1, 1, 32, 128), 0.25, np.float32)
    block[0, 0, 4, 4] = np.nan
    block[0, 0, 0, 1] = 1000.0
    nq, c = both(block)
    assert np.array_equal(nq.payload, c[0])
    assert nq.scale[0, 0, 0] == 1.0
    assert nq.payload[0, 0, 4, 4] & 0x7F == 0x7F
    assert nq.payload[0, 0, 0, 1] == 0x7E                        # 1000 clamped to 448
    assert nq.payload[0, 0, 0, 0] == gdn_oracle.e4m3fn_encode(np.float32(0.25))


def test_saturation_fraction():
    """|x / s| > 448 counts as saturated; x = amax may land a hair above 448."""
    rng = np.random.default_rng(3)
    state = rng.standard_normal((3, 2, 64, 128)).astype(np.float32)
    nq, c = both(state)
    assert_same(nq, c)
    s32 = gdn_oracle.safe_scale(np.abs(state.reshape(3, 2, 2, 32, 128)).max(axis=(-2, -1)), 448.0)
    ratio = np.abs(state.reshape(3, 2, 2, 32, 128)) / s32[..., None, None]
    assert nq.saturation_fraction == pytest.approx(float(np.mean(ratio > 448.0)))


def test_dequantize_roundtrip_error_bound():
    """Dequantised values are within half an e4m3fn ulp (2^-4 relative for
    normals) plus fp16 scale rounding (2^-11) of the source."""
    rng = np.random.default_rng(4)
    state = rng.standard_normal((2, 2, 64, 128)).astype(np.float32)
    nq, _ = both(state)
    deq = gdn_oracle.dequantize_checkpoint(nq)
    blocks = np.abs(state.reshape(2, 2, 2, 32, 128)).max(axis=(-2, -1), keepdims=True)
    s = np.broadcast_to(blocks / 448.0, (2, 2, 2, 32, 128)).reshape(state.shape)
    normal = np.abs(state) >= s * 2.0 ** -6
    err = np.abs(deq - state)
    bound = np.abs(state) * (2.0 ** -4 + 2.0 ** -10) + 1e-30
    assert np.all(err[normal] <= bound[normal])
    assert np.all(err[~normal] <= s[~normal] * 2.0 ** -10 + np.abs(state[~normal]) * 2.0 ** -10)


def test_other_granularities_shapes():
    """head / row / tile / vblock_int8 formats (ref:48-106) exist with the
    reference's scale shapes; only vblock/32 is on the HIP path."""
    rng = np.random.default_rng(5)
    state = rng.standard_normal((1, 2, 64, 128)).astype(np.float32)
    assert gdn_oracle.quantize_checkpoint(state, "head", 32).scale.shape == (1, 2, 1, 1)
    assert gdn_oracle.quantize_checkpoint(state, "row", 32).scale.shape == (1, 2, 64, 1)
    assert gdn_oracle.quantize_checkpoint(state, "tile", 32).scale.shape == (1, 2, 2, 4)
    q8 = gdn_oracle.quantize_checkpoint(state, "vblock_int8", 32)
    assert q8.payload.dtype == np.int8 and q8.scale.shape == (1, 2, 2)
    for gran in ("head", "row", "tile", "vblock", "vblock_int8"):
        q = gdn_oracle.quantize_checkpoint(state, gran, 32)
        deq = gdn_oracle.dequantize_checkpoint(q)
        assert gdn_oracle.relative_l2(deq, state) < (1e-2 if gran.endswith("int8") else 6e-2)
