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
    (64, 64, torch.bfloat16), (48, 64, torch.float16), (64, 64, torch.float32)])
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


# ---------------------------------------------------------------------------
# The same construction on the launch shapes of the decode kernel that carry
# the headline and the other instantiations: multi-unit workgroups, the DMA
# refill of a row wave's later vblocks, helper waves (the unit's own chain
# wave, and the partner unit's when that unit replays) with their LDS o
# partials and separate scale stores, single-unit workgroups, V = 64 / 256
# and odd GQA groups. Each case names the plan the library picks for it
# (gdnr_decode_plan), so a change of plan cannot silently move a case off the
# instantiation it is meant to cover.
# ---------------------------------------------------------------------------

def _device_checkpoint(batch, value_heads, value_dim, seed, device):
    """Hand-built codes on the device (as _hand_built_checkpoint: every
    vblock's largest magnitude code below 0x7E and attained, random signs, an
    all-zero and a negative-zero vblock, three vblocks holding a NaN code) and
    fp16 scales over 2^-20 .. 2^-2 with one subnormal. Returns (codes u8
    [B,HV,V,K], scale f16 [B,HV,V/32], NaN vblocks)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    nvb = value_dim // VB
    top = torch.randint(0x08, 0x7E, (batch, value_heads, nvb, 1), generator=gen, device=device)
    mag = (torch.rand(batch, value_heads, nvb, VB * K, generator=gen, device=device) * (top + 1).float()).floor()
    mag = torch.minimum(mag, top.float()).to(torch.uint8)
    at = torch.randint(0, VB * K, (batch, value_heads, nvb, 1), generator=gen, device=device)
    mag.scatter_(3, at, top.to(torch.uint8))
    sign = torch.randint(0, 2, mag.shape, generator=gen, device=device, dtype=torch.uint8) << 7
    codes = (mag | sign).view(batch, value_heads, value_dim, K)
    codes[0, 0, 0:VB] = 0
    codes[0, 1 % value_heads, VB:2 * VB] = 0x80
    # (in flushing sequences whichever the pattern: even indices flush in both)
    nan_blocks = [(0, 2 % value_heads, 0), (2, 5 % value_heads, nvb - 1), (batch - 2, value_heads - 1, nvb // 2)]
    for b, hv, p in nan_blocks:
        codes[b, hv, VB * p + 3, 7] = 0x7F
        codes[b, hv, VB * p + 9, 100] = 0xFF
    exps = torch.randint(-20, -2, (batch, value_heads, nvb), generator=gen, device=device).float()
    scale = ((torch.rand(batch, value_heads, nvb, generator=gen, device=device) + 1.0) * torch.exp2(exps)).half()
    scale[0, 3 % value_heads, nvb - 1] = 2.0 ** -24
    return codes.contiguous(), scale.contiguous(), nan_blocks


def _expected_requant(codes, scale, seqs):
    """The reference quantiser (C restatement of ref:36-37,83-99) on the
    dequantised checkpoint of the sequences `seqs`; in a vblock holding a NaN
    code every row with a NaN becomes NaN (the rebuild's delta term is
    0 * NaN there, as in the reference recurrence, kernel:218-224)."""
    from oracle import fp8_quant

    idx = torch.as_tensor(seqs, device=codes.device)
    c = codes[idx].cpu().numpy()
    s = scale[idx].cpu().numpy()
    deq = gdn_oracle.dequantize_vblock32(c, s)
    nan_rows = np.isnan(deq).any(axis=-1, keepdims=True)
    deq = np.where(nan_rows, np.float32(np.nan), deq)
    want_codes, want_scale, _ = fp8_quant.quantize_vblock32(deq)
    return want_codes, want_scale


def _zero_sign_free(c):
    c = np.where(c == 0x80, 0, c)
    return np.where(c == 0xFF, 0x7F, c)


def flush_pattern_flushes(pattern, b):
    return pattern == "all" or b % 2 == 0


HEADLINE_CASES = {
    # id: (batch, heads, value_heads, value_dim, flush pattern, expected plan (rows/wave, waves/head, gw, units)
    #      [, ring length: 16 when absent])
    "B64_all_flush": (64, 16, 32, 128, "all", (128, 1, 2, 4)),
    "B64_alternate": (64, 16, 32, 128, "alternate", (128, 1, 2, 4)),
    "B512_all_flush": (512, 16, 32, 128, "all", (128, 1, 2, 1)),
    "B512_alternate": (512, 16, 32, 128, "alternate", (128, 1, 2, 1)),
    "V256_G1_B32_alternate": (32, 16, 16, 256, "alternate", (128, 2, 1, 2)),
    "V256_G1_B64_alternate": (64, 16, 16, 256, "alternate", (128, 2, 1, 4)),
    "V256_G2_B64_alternate": (64, 16, 32, 256, "alternate", (128, 2, 2, 2)),
    "V64_G2_B64_alternate": (64, 16, 32, 64, "alternate", (64, 1, 2, 4)),
    "V128_G1_B16_alternate": (16, 16, 16, 128, "alternate", (32, 4, 1, 1)),
    "B8_all_flush": (8, 16, 32, 128, "all", (32, 4, 1, 1)),
    "V128_G1_B64_alternate": (64, 16, 16, 128, "alternate", (128, 1, 1, 4)),
    # rings of several 16-token chunks (one value head per unit; waves of 32
    # rows while the workgroups do not outnumber the compute units, else 64)
    "L64_B8_all_flush": (8, 16, 32, 128, "all", (32, 4, 1, 1), 64),
    "L64_B8_alternate": (8, 16, 32, 128, "alternate", (32, 4, 1, 1), 64),
    "L48_V64_B8_alternate": (8, 16, 32, 64, "alternate", (32, 2, 1, 1), 48),
    "L32_V64_B8_all_flush": (8, 16, 32, 64, "all", (32, 2, 1, 1), 32),
    "L64_B16_alternate": (16, 16, 32, 128, "alternate", (64, 2, 1, 1), 64),
    "L32_V64_B16_all_flush": (16, 16, 32, 64, "all", (64, 1, 1, 1), 32),
}


@pytest.mark.parametrize("fused", [False, True], ids=["replay", "prep_replay"])
@pytest.mark.parametrize("case", list(HEADLINE_CASES))
def test_decode_flush_requantiser_bit_exact(device, case, fused):
    """g = 0 and beta = 0 on every ring token (in the full contract the new
    token's gates come from A_log = -inf and b = -inf: g = -0, beta = 0), so
    every flushing sequence's rebuilt state is its dequantised checkpoint, and
    its codes and scales must equal the reference quantiser's on that state
    bit for bit, whichever wave (row wave, own chain wave or partner chain
    wave) rebuilt each vblock. Replaying sequences keep their codes and
    scales untouched. bf16."""
    import gdnr_lib

    batch, heads, value_heads, value_dim, pattern, plan, *ring = HEADLINE_CASES[case]
    ring = ring[0] if ring else 16
    got_plan = gdnr_lib.decode_plan(batch, heads, value_heads, value_dim, ring)
    assert got_plan is not None
    assert (got_plan["rows_per_wave"], got_plan["waves_per_head"], got_plan["heads_per_unit"],
            got_plan["units"]) == plan, got_plan
    print(f"{case} fused={fused}: plan {got_plan}", flush=True)
    codes0, scale0, nan_blocks = _device_checkpoint(batch, value_heads, value_dim, seed=batch + value_dim, device=device)
    assert all(flush_pattern_flushes(pattern, b) for b, _, _ in nan_blocks)
    gen = torch.Generator(device=device).manual_seed(11)
    act = torch.bfloat16
    k_ring = torch.randn(batch, ring, heads, K, generator=gen, device=device).to(act)
    v_ring = torch.randn(batch, ring, value_heads, value_dim, generator=gen, device=device).to(act)
    g_ring = torch.zeros(batch, ring, value_heads, dtype=act, device=device)
    beta_ring = torch.zeros(batch, ring, value_heads, dtype=act, device=device)
    flush = torch.ones(batch, dtype=torch.bool, device=device)
    if pattern == "alternate":
        flush[1::2] = False
    valid = torch.where(flush, ring, torch.randint(1, ring, (batch,), generator=gen, device=device)).to(torch.int32)
    payload = codes0.clone().view(torch.float8_e4m3fn)
    scale = scale0.clone()
    if fused:
        mixed = torch.randn(batch, 2 * heads * K + value_heads * value_dim, generator=gen, device=device).to(act)
        a = torch.randn(batch, value_heads, generator=gen, device=device).to(act)
        b = torch.full((batch, value_heads), -float("inf"), dtype=act, device=device)
        a_log = torch.full((value_heads,), -float("inf"), device=device)
        dt_bias = torch.zeros(value_heads, device=device)
        q_out = torch.empty(batch, heads, K, dtype=act, device=device)
        gk.gdn_prep_replay_fp8(mixed, a, b, a_log, dt_bias, valid - 1, payload, scale, q_out, k_ring, v_ring, g_ring,
                               beta_ring, valid, flush, block_v=min(128, value_dim))
        # the new token's gates were appended as g = -0, beta = 0
        pos = (valid - 1).long()
        rows = torch.arange(batch, device=device)
        assert torch.all(g_ring[rows, pos] == 0) and torch.all(beta_ring[rows, pos] == 0)
    else:
        q = torch.randn(batch, heads, K, generator=gen, device=device).to(act)
        gk.gdn_replay_fp8(payload, scale, q, k_ring, v_ring, g_ring, beta_ring, valid, flush, block_v=32)
    torch.cuda.synchronize()
    got_codes = payload.view(torch.uint8)
    fl = flush.cpu().numpy()
    replaying = np.nonzero(~fl)[0]
    if len(replaying):
        idx = torch.as_tensor(replaying, device=device)
        assert torch.equal(got_codes[idx], codes0[idx])
        assert torch.equal(scale[idx].view(torch.int16), scale0[idx].view(torch.int16))
    flushing = np.nonzero(fl)[0]
    changed = total = 0
    for lo in range(0, len(flushing), 64):
        seqs = flushing[lo:lo + 64]
        want_codes, want_scale = _expected_requant(codes0, scale0, seqs)
        idx = torch.as_tensor(seqs, device=device)
        gc = got_codes[idx].cpu().numpy()
        gs = scale[idx].cpu().numpy()
        bad = _zero_sign_free(gc) != _zero_sign_free(want_codes)
        assert not bad.any(), (case, int(bad.sum()), np.argwhere(bad)[:4])
        assert np.array_equal(gs.view(np.uint16), want_scale.view(np.uint16)), (case, np.argwhere(gs.view(np.uint16) != want_scale.view(np.uint16))[:4])
        changed += int(np.sum(gs != scale0[idx].cpu().numpy()))
        total += gs.size
    # the quotients were real divisions: most scales changed
    assert changed > 0.9 * total, (changed, total)
