"""Pins of the oracle's other checkpoint formats (gdn_oracle.quantize_checkpoint
for granularity head / row / tile / vblock and the *_int8 codes,
prototype/gdn_replay_fp8_reference.py:40-106), tied to the vblock path the
other oracle tests pin and to hand-derived values:

* tile with tile_size = K groups exactly like vblock with the same tile_size;
* row and head equal vblock(1) and vblock(V) when every group's amax/448 is
  exact in fp16 (then the rounded and unrounded scales coincide);
* where they differ, row divides by the fp16-ROUNDED scale (ref:92-93) and
  vblock(1) by the unrounded one: a value between two codes' midpoints
  under the two scales lands on different codes;
* int8 codes are round-half-to-even of x / s, clamped to +-127, checked
  element by element with Python's round() on exact ties;
* dequantisation multiplies each code by its group's stored scale.
int8 NaN codes are 0 here; torch's NaN -> int8 cast is platform-defined, so
that case is parity unpinned.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import gdn_oracle

Q = gdn_oracle.quantize_checkpoint


def _rand(shape, seed=0):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def test_tile_of_full_width_is_vblock():
    x = _rand((2, 3, 64, 16), 1)
    a, b = Q(x, "tile", 16), Q(x, "vblock", 16)
    assert np.array_equal(a.payload, b.payload)
    assert np.array_equal(a.scale[..., 0], b.scale)


def _exact_scale_state(groups_rows, rows_per_group, K, seed):
    """Rows whose group amax is 448 * 2^k (an fp16-exact scale)."""
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (1, 1, groups_rows * rows_per_group, K)).astype(np.float32)
    for gidx in range(groups_rows):
        blk = x[0, 0, gidx * rows_per_group:(gidx + 1) * rows_per_group]
        blk *= np.float32(448.0 * 2.0 ** int(rng.integers(-6, 4))) / np.abs(blk).max()
    return x


def test_row_and_head_equal_vblock_when_scales_are_exact():
    x = _exact_scale_state(8, 1, 32, 2)
    r, v1 = Q(x, "row", 1), Q(x, "vblock", 1)
    assert np.array_equal(r.payload, v1.payload)
    assert np.array_equal(r.scale[..., 0], v1.scale)
    xh = _exact_scale_state(1, 8, 32, 3)
    h, v8 = Q(xh, "head", 1), Q(xh, "vblock", 8)
    assert np.array_equal(h.payload, v8.payload)
    assert np.array_equal(h.scale.reshape(-1), v8.scale.reshape(-1))


def test_row_divides_by_the_rounded_scale():
    delta = 2.0 ** -12
    amax = np.float32(448.0 * (1 + delta))  # s32 = 1 + 2^-12, fp16(s32) = 1
    x = np.zeros((1, 1, 1, 4), dtype=np.float32)
    x[0, 0, 0, 0] = amax
    x[0, 0, 0, 1] = np.float32(1.0625 * (1 + delta / 2))  # between the 1.0 / 1.125 midpoints of the two scales
    r, v = Q(x, "row", 1), Q(x, "vblock", 1)
    assert gdn_oracle.e4m3fn_decode(r.payload[0, 0, 0, 1]) == 1.125
    assert gdn_oracle.e4m3fn_decode(v.payload[0, 0, 0, 1]) == 1.0


def test_int8_round_half_even_and_clamp():
    s = 2.0 ** -3  # amax = 127 s: exact scale
    vals = np.array([127 * s, 2.5 * s, 3.5 * s, -2.5 * s, -3.5 * s, 0.49 * s, -0.5 * s, 126.5 * s, 1.5 * s],
                    dtype=np.float32)
    x = np.zeros((1, 1, 1, vals.size), dtype=np.float32)
    x[0, 0, 0] = vals
    q = Q(x, "row_int8", 1)
    expect = [max(-127, min(127, round(float(v) / s))) for v in vals]  # Python's round: half to even
    assert q.payload.dtype == np.int8
    assert q.payload[0, 0, 0].tolist() == expect
    assert np.float32(q.scale.reshape(-1)[0]) == np.float32(s)


def test_int8_nan_is_zero():
    x = _rand((1, 1, 4, 8), 4)
    x[0, 0, 1, 3] = np.nan
    q = Q(x, "vblock_int8", 4)
    assert q.payload[0, 0, 1, 3] == 0


@pytest.mark.parametrize("gran,tile", [("head", 32), ("row", 32), ("tile", 8), ("vblock", 16), ("tile_int8", 8),
                                       ("row_int8", 1)])
def test_dequantize_multiplies_by_the_group_scale(gran, tile):
    x = _rand((2, 2, 32, 16), 5)
    q = Q(x, gran, tile)
    deq = gdn_oracle.dequantize_checkpoint(q)
    codes = q.payload.astype(np.float32) if gran.endswith("int8") else gdn_oracle.e4m3fn_decode(q.payload)
    # the group scale of element (b, h, r, c), looked up independently
    base = gran.removesuffix("_int8")
    for (b, h, r, c) in [(0, 0, 0, 0), (1, 1, 31, 15), (0, 1, 17, 9), (1, 0, 8, 7)]:
        if base == "head":
            sc = q.scale[b, h, 0, 0]
        elif base == "row":
            sc = q.scale[b, h, r, 0]
        elif base == "tile":
            sc = q.scale[b, h, r // tile, c // tile]
        else:
            sc = q.scale[b, h, r // tile]
        assert deq[b, h, r, c] == np.float32(codes[b, h, r, c]) * np.float32(sc)
