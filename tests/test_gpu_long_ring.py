"""GPU parity of the long-ring full-contract path (marked `gpu`): rings of 17
to 64 tokens, which gdn_prep_replay_fp8 runs on the decode kernel's chunked
path at small batches (csrc/gdnr_decode.hip, up to 16 sequences of 32 value
heads) and on the fused replay kernel beyond (prep + replay or flush in one
launch, csrc/gdnr_kernels.hip).

The reference's full-contract cycle (prototype/bench_gdn_full_contract.py
:225-308) over a little more than one ring with mixed ring phases, so that
every sequence flushes once and the launches mix replays and flushes. The
outputs are checked against the fp64 oracle (gdn_oracle.full_contract_decode,
which restates prototype/gdn_replay_fp8_reference.py:189-244 and the prep of
prototype/gdn_replayssm_fp8_kernel.py:453-576) to the 2e-3 rel-L2 gate; the
requantised codes to rounding-boundary flips (< 1e-3 of the codes); the
prepared query and the ring slots the prep appended to within one bf16 ulp
of the oracle's prep (the device forms them in fp32, the oracle in fp64).
The fused launch also equals the unfused pair (prep, then replay) bit for
bit at L = 64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth
from conftest import rel_l2
from gpu_helpers import codes_np, np32
from oracle import gdn_oracle

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-3
CODE_FLIP_TOL = 1e-3


def _zero_rings(batch, window, shape, device):
    return [torch.zeros(batch, window, shape.heads, shape.key_dim, dtype=torch.bfloat16, device=device),
            torch.zeros(batch, window, shape.value_heads, shape.value_dim, dtype=torch.bfloat16, device=device),
            torch.zeros(batch, window, shape.value_heads, dtype=torch.bfloat16, device=device),
            torch.zeros(batch, window, shape.value_heads, dtype=torch.bfloat16, device=device)]


def _within_bf16_ulp(got, want):
    ulp = np.abs(want) * 2.0 ** -7 + 1e-30
    return bool(np.all(np.abs(got - want) <= ulp)) and float(np.mean(got != want)) < 0.01


@pytest.mark.parametrize("batch", [3, 20], ids=["decode_kernel", "replay_kernel"])
@pytest.mark.parametrize("window", [32, 64])
def test_long_ring_cycle_matches_oracle(device, window, batch):
    import gdnr_lib

    shape = synth.Shape(batch)
    # (the kernel each batch is meant to run on)
    assert (gdnr_lib.decode_plan(batch, shape.heads, shape.value_heads, shape.value_dim, window) is not None) == (batch == 3)
    gen = synth.generator(4100 + window, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 16, gen, device, a_log, dt_bias)
    steps = window + 1
    mixed, a, b = synth.raw_step_inputs(shape, steps, gen, device)
    phase = np.array([0, window // 2, window - 1] + [(5 * i) % window for i in range(batch - 3)])
    ck = gk.quantize_checkpoint(state)
    codes0, scale0 = codes_np(ck.payload).copy(), ck.scale.cpu().numpy().copy()
    q_out = torch.zeros(batch, shape.heads, shape.key_dim, dtype=torch.bfloat16, device=device)
    rings = _zero_rings(batch, window, shape, device)
    # the oracle's prep into rings of its own, step by step (the rings depend on the prep alone)
    oq = np.zeros((batch, shape.heads, shape.key_dim), np.float32)
    orings = [np.zeros(r.shape, np.float32) for r in rings]
    phase_t = torch.as_tensor(phase, dtype=torch.int32, device=device)
    outs = []
    for step in range(steps):
        fill = (phase_t + step) % window + 1
        outs.append(np32(gk.gdn_prep_replay_fp8(mixed[:, step].contiguous(), a[:, step].contiguous(),
                                                b[:, step].contiguous(), a_log, dt_bias, fill - 1, ck.payload,
                                                ck.scale, q_out, *rings, fill, fill == window)))
        gdn_oracle.prep_ring(np32(mixed[:, step]), np32(a[:, step]), np32(b[:, step]), np32(a_log), np32(dt_bias),
                             (phase + step) % window, oq, *orings)
    ref, ref_codes, _ = gdn_oracle.full_contract_decode(
        codes0, scale0, np32(mixed), np32(a), np32(b), np32(a_log), np32(dt_bias), window, shape.heads,
        shape.key_dim, shape.value_heads, shape.value_dim, phase=phase, dtype=np.float64)
    got = np.stack(outs, axis=1)
    err = rel_l2(got, ref)
    flips = float(np.mean(codes_np(ck.payload) != ref_codes))
    print(f"L={window}: output rel-L2 {err:.3e}, code flips {flips:.2e}")
    assert err <= OUT_TOL, err
    assert flips < CODE_FLIP_TOL, flips
    assert _within_bf16_ulp(np32(q_out), oq)
    for got_r, want_r in zip(rings, orings):
        assert _within_bf16_ulp(np32(got_r), want_r)


def test_long_ring_fused_equals_prep_then_replay(device):
    """gdn_prep_replay_fp8 == gdn_prep_ring + gdn_replay_fp8 bit for bit at
    L = 64: outputs, query, ring slots, codes and scales, with replays and
    flushes in the same launch and a new token outside the replayed prefix."""
    batch, window = 5, 64
    shape = synth.Shape(batch)
    gen = synth.generator(4199, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 16, gen, device, a_log, dt_bias)
    mixed, a, b = synth.raw_step_inputs(shape, 1, gen, device)
    mixed, a, b = mixed[:, 0].contiguous(), a[:, 0].contiguous(), b[:, 0].contiguous()
    _, k, v, g, beta = synth.ring_inputs(shape, window, gen, device, a_log, dt_bias)
    pos = torch.tensor([0, 17, 63, 40, 63], dtype=torch.int32, device=device)
    valid = pos + 1
    valid[3] = 20  # the new token outside the replayed prefix
    flush = torch.tensor([0, 0, 1, 0, 1], dtype=torch.bool, device=device)
    results = []
    for fused in (False, True):
        ck = gk.quantize_checkpoint(state)
        q_out = torch.zeros(batch, shape.heads, shape.key_dim, dtype=torch.bfloat16, device=device)
        rk, rv, rg, rb = k.clone(), v.clone(), g.clone(), beta.clone()
        if fused:
            out = gk.gdn_prep_replay_fp8(mixed, a, b, a_log, dt_bias, pos, ck.payload, ck.scale, q_out, rk, rv, rg,
                                         rb, valid, flush)
        else:
            gk.gdn_prep_ring(mixed, a, b, a_log, dt_bias, pos, q_out, rk, rv, rg, rb)
            out = gk.gdn_replay_fp8(ck.payload, ck.scale, q_out, rk, rv, rg, rb, valid, flush)
        results.append([out, q_out, rk, rv, rg, rb, ck.payload.view(torch.uint8), ck.scale])
    for x, y in zip(*results):
        assert torch.equal(x, y)


def test_long_ring_tiles_identical(device):
    """The V-tile height of the long-ring kernel (block_v 32, 64 or 128; the
    library also lowers it on its own for small launches) changes nothing:
    outputs, requantised codes and scales are bit-identical at L = 64, with
    replaying and flushing sequences in the same launch. (Batch 16: no tile
    is lowered below the requested one.)"""
    from gpu_helpers import make_replay_case, run_replay

    valid = [64, 17, 33, 64, 1, 64, 50, 63, 64, 2, 40, 64, 9, 64, 31, 64]
    flush = [v == 64 for v in valid]
    results = []
    for bv in (128, 64, 32):
        case = make_replay_case(16, 64, device, seed=4300, warmup=16, valid=valid, flush=flush)
        out = run_replay(case, block_v=bv)
        results.append((out, case["ckpt"].payload.view(torch.uint8).clone(), case["ckpt"].scale.clone()))
    for other in results[1:]:
        for x, y in zip(results[0], other):
            assert torch.equal(x, y)
