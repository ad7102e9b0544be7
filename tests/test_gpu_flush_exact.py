"""Bit-exact check of the flush's in-kernel requantiser (marked `gpu`).

With the g ring at 0 (gamma = exp(0) = 1: no decay) and the beta ring at 0
(no delta update), the state the flush rebuilds is the dequantised checkpoint
itself, exactly, so the codes and fp16 scales it writes must equal the
reference quantiser (ref:36-37,83-99) applied to dequantize(codes0, scale0)
bit for bit. The codes are hand-built: every vblock's largest code sits below
0x7E, so the new scale differs from the old one and every quotient is a real
division, and some vblocks hold NaN codes. A NaN code turns its whole row to
NaN in the rebuild, as in the reference recurrence (kernel:218-224: the
retrieved value is NaN and NaN * beta = NaN); those vblocks are checked
against the oracle's recurrence (gdn_oracle.replay_step) instead.

Signs of zeros and NaNs are the freedoms: the reference recurrence adds
beta (v - S k) k^T = +-0 to the state, which turns -0 into +0 or not by the
signs of v - S k and k, so codes 0x00 and 0x80 (both the value 0) compare as
equal, and so do 0x7F and 0xFF (IEEE arithmetic leaves a NaN's sign open).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gdn_replayssm_fp8_kernel as gk
from gpu_helpers import codes_np, np32
from oracle import gdn_oracle

pytestmark = pytest.mark.gpu

H, HV, K, V, VB = 16, 32, 128, 128, 32


def _hand_built_checkpoint(batch: int, seed: int):
    """Codes with per-vblock maximum code below 0x7E, zero blocks, NaN blocks;
    fp16 scales over a wide range (normal and subnormal)."""
    rng = np.random.default_rng(seed)
    nvb = V // VB
    codes = np.zeros((batch, HV, V, K), dtype=np.uint8)
    top = rng.integers(0x08, 0x7E, size=(batch, HV, nvb))           # per-vblock largest magnitude code
    for b in range(batch):
        for hv in range(HV):
            for p in range(nvb):
                mag = rng.integers(0, top[b, hv, p] + 1, size=(VB, K), dtype=np.int64)
                mag[rng.integers(0, VB), rng.integers(0, K)] = top[b, hv, p]  # the maximum is attained
                sign = rng.integers(0, 2, size=(VB, K), dtype=np.int64) << 7
                codes[b, hv, VB * p:VB * (p + 1)] = (mag | sign).astype(np.uint8)
    codes[0, 0, 0:VB] = 0                                              # amax == 0: scale 1, codes 0
    codes[0, 1, VB:2 * VB] = 0x80                                      # negative zeros
    nan_blocks = [(0, 2, 0), (1, 5, 3), (batch - 1, HV - 1, 2)]
    for b, hv, p in nan_blocks:
        codes[b, hv, VB * p + 3, 7] = 0x7F                             # +NaN
        codes[b, hv, VB * p + 9, 100] = 0xFF                           # -NaN
    exps = rng.integers(-20, -2, size=(batch, HV, nvb))
    scale = (rng.uniform(1.0, 2.0, size=(batch, HV, nvb)) * np.exp2(exps)).astype(np.float16)
    scale[0, 3, 1] = np.float16(2.0 ** -24)                            # subnormal fp16 scale
    return codes, scale, nan_blocks


@pytest.mark.parametrize("ring_len,block_v,act", [
    (4, 32, torch.bfloat16), (16, 128, torch.bfloat16), (16, 64, torch.float16), (8, 128, torch.float32),
    (64, 64, torch.bfloat16)])
def test_flush_requantiser_bit_exact(device, ring_len, block_v, act):
    batch = 3
    codes0, scale0, nan_blocks = _hand_built_checkpoint(batch, seed=ring_len + block_v)
    gen = torch.Generator().manual_seed(ring_len)
    q = torch.randn(batch, H, K, generator=gen).to(act).to(device)
    k = torch.randn(batch, ring_len, H, K, generator=gen).to(act).to(device)
    v = torch.randn(batch, ring_len, HV, V, generator=gen).to(act).to(device)
    g = torch.zeros(batch, ring_len, HV, dtype=act, device=device)
    beta = torch.zeros(batch, ring_len, HV, dtype=act, device=device)
    valid = torch.tensor([ring_len, ring_len // 2, 1][:batch], dtype=torch.int32, device=device)
    flush = torch.ones(batch, dtype=torch.bool, device=device)
    payload = torch.from_numpy(codes0.copy()).to(device).view(torch.float8_e4m3fn)
    scale = torch.from_numpy(scale0.copy()).to(device)
    gk.gdn_replay_fp8(payload, scale, q, k, v, g, beta, valid, flush, block_v=block_v)
    got_codes = codes_np(payload)
    got_scale = scale.cpu().numpy()

    deq = gdn_oracle.dequantize_vblock32(codes0, scale0)
    direct = gdn_oracle.quantize_checkpoint(deq, "vblock", VB)
    _, rec_codes, rec_scale = gdn_oracle.replay_step(codes0, scale0, np32(q), np32(k), np32(v), np32(g), np32(beta),
                                                     valid.cpu().numpy(), flush.cpu().numpy(), np.float64)
    nan_mask = np.zeros((batch, HV, V // VB), dtype=bool)
    for b, hv, p in nan_blocks:
        nan_mask[b, hv, p] = True
    rows = np.repeat(nan_mask, VB, axis=2)                               # [B, HV, V] rows of NaN vblocks

    def zero_sign_free(c):
        c = np.where(c == 0x80, 0, c)
        return np.where(c == 0xFF, 0x7F, c)

    got_codes, rec_codes = zero_sign_free(got_codes), zero_sign_free(rec_codes)
    direct_codes = zero_sign_free(direct.payload)
    # finite vblocks: the reference quantiser on the dequantised checkpoint, bit for bit
    assert np.array_equal(got_codes[~rows], direct_codes[~rows]), np.mean(got_codes[~rows] != direct_codes[~rows])
    assert np.array_equal(got_scale[~nan_mask].view(np.uint16),
                          direct.scale.astype(np.float16)[~nan_mask].view(np.uint16))
    # ... which is also what the oracle's recurrence gives there
    assert np.array_equal(rec_codes[~rows], direct_codes[~rows])
    # NaN vblocks: as the reference recurrence leaves them (NaN rows, scale 1)
    assert np.array_equal(got_codes[rows], rec_codes[rows])
    assert np.array_equal(got_scale[nan_mask].view(np.uint16), rec_scale[nan_mask].astype(np.float16).view(np.uint16))
    # the quotients were real divisions: most scales changed
    assert np.mean(got_scale[~nan_mask] != scale0[~nan_mask]) > 0.9
