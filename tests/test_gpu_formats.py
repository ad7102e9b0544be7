"""GPU parity of every checkpoint format (gdnr_quantize_checkpoint /
gdnr_dequantize_checkpoint, the reference's quantize_checkpoint /
dequantize_checkpoint, prototype/gdn_replay_fp8_reference.py:40-134) against
the oracle, marked `gpu`: payload codes, fp16 scales and saturation counts
bit-exact given the same fp32 state, and the dequantised state bit-exact.
The states mix a warmed GDN state with edge groups: all zero, one NaN, one
huge and one tiny magnitude."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth
from gpu_helpers import np32
from oracle import gdn_oracle

pytestmark = pytest.mark.gpu

FORMATS = [("head", 32), ("row", 32), ("tile", 16), ("tile", 32), ("vblock", 16), ("vblock", 64),
           ("head_int8", 32), ("row_int8", 32), ("tile_int8", 32), ("vblock_int8", 32)]


def _state(device, seed):
    shape = synth.Shape(2)
    gen = synth.generator(seed, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    x = synth.warm_state(shape, 16, gen, device, a_log, dt_bias)
    x[0, 1] = 0.0                                  # an all-zero head (every group zero)
    x[1, 2, 5, 7] = float("nan")                   # a NaN element
    x[1, 3, 64:96] *= 3.0e4                        # huge magnitudes (fp16 scale overflow for head/row)
    x[0, 4, 32:64] *= 1.0e-30                      # tiny magnitudes (fp16 scale underflow)
    return x


@pytest.mark.parametrize("gran,tile", FORMATS)
def test_format_matches_oracle(device, gran, tile):
    x = _state(device, 70)
    q = gk.quantize_checkpoint(x, gran, tile)
    ref = gdn_oracle.quantize_checkpoint(np32(x), gran, tile)
    got_payload = q.payload.view(torch.int8 if gran.endswith("int8") else torch.uint8).cpu().numpy()
    assert np.array_equal(got_payload, ref.payload)
    assert np.array_equal(q.scale.cpu().numpy().view(np.uint16), ref.scale.astype(np.float16).view(np.uint16))
    assert q.saturation_fraction == pytest.approx(ref.saturation_fraction, abs=1e-12)
    deq = gk.dequantize_checkpoint(q)
    ref_deq = gdn_oracle.dequantize_checkpoint(ref)
    assert np.array_equal(np32(deq), ref_deq, equal_nan=True)


def test_vblock32_paths_agree(device):
    """The decode path's fast vblock32 quantiser and the generic one write the same bytes."""
    x = _state(device, 71)
    fast = gk.quantize_checkpoint(x, "vblock", 32)
    payload = torch.empty_like(fast.payload)
    scale = torch.empty_like(fast.scale)
    import gdnr_lib
    gdnr_lib.call("gdnr_quantize_checkpoint", [x, payload, scale, None], [3, 32],
                  gdnr_lib.current_stream(device))
    assert torch.equal(payload.view(torch.uint8), fast.payload.view(torch.uint8))
    assert torch.equal(scale, fast.scale)
