"""Bounded waits that give up (marked `gpu`).

The waves of a decode or step workgroup hand the coefficient chain, the
flush factors and the flush helpers' results to each other through LDS
flags; every wait for one is bounded. The host forces every wait to give up
at once (a poll budget of 0, gdnr_set_wait_polls): every kernel still runs
to its end, the device status word counts the waits that gave up, and the
waves whose waits gave up store no checkpoint codes or scales, so a flush
step leaves the checkpoint exactly as it was. With the default budget
restored, the same step flushes as it should.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth
import gdnr_lib
from conftest import rel_l2
from gpu_helpers import codes_np, make_replay_case, np32, oracle_replay, run_replay

pytestmark = pytest.mark.gpu


def _prep_args(case, device, seed=3):
    """Raw full-contract inputs of one step for a replay case (bf16)."""
    batch = case["q"].shape[0]
    shape = synth.Shape(batch)
    gen = synth.generator(seed, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    mixed, a, b = synth.raw_step_inputs(shape, 1, gen, device)
    q_out = torch.empty_like(case["q"])
    return mixed[:, 0], a[:, 0], b[:, 0], a_log, dt_bias, q_out


@pytest.mark.parametrize("act,batch,ring,entry", [
    (torch.bfloat16, 64, 16, "replay"),        # decode kernel, 4-unit workgroups, partner helpers
    (torch.bfloat16, 64, 16, "prep_replay"),   # the headline launch (fused preparation)
    (torch.bfloat16, 512, 8, "replay"),        # decode kernel, single-unit workgroups, own-chain helpers
    (torch.float32, 8, 8, "replay"),           # step kernel
])
def test_waits_that_give_up_leave_the_checkpoint(device, act, batch, ring, entry):
    valid = np.where(np.arange(batch) % 2 == 0, ring, 1 + np.arange(batch) % (ring - 1)).astype(np.int32)
    case = make_replay_case(batch, ring, device, seed=21, dtype=act, valid=valid, flush=valid == ring)
    codes0 = codes_np(case["ckpt"].payload).copy()
    scale0 = case["ckpt"].scale.clone()
    prep = _prep_args(case, device) if entry == "prep_replay" else None
    k_before = case["k"].clone()

    def step():
        if prep is None:
            return run_replay(case, block_v=128)
        mixed, a, b, a_log, dt_bias, q_out = prep
        return gk.gdn_prep_replay_fp8(mixed, a, b, a_log, dt_bias, case["valid"] - 1, case["ckpt"].payload,
                                      case["ckpt"].scale, q_out, case["k"], case["v"], case["g"], case["beta"],
                                      case["valid"], case["flush"])

    print(f"give-up: act={act} B={batch} L={ring} entry={entry}", flush=True)
    gdnr_lib.wait_timeouts(reset=True)
    previous = gdnr_lib.set_wait_polls(0)
    try:
        step()
        torch.cuda.synchronize()
    finally:
        gdnr_lib.set_wait_polls(previous)
    assert previous == gdnr_lib.DEFAULT_WAIT_POLLS
    gave_up = gdnr_lib.wait_timeouts(reset=True)
    assert gave_up > 0
    assert np.array_equal(codes_np(case["ckpt"].payload), codes0)
    assert torch.equal(case["ckpt"].scale.view(torch.int16), scale0.view(torch.int16))
    if prep is not None:
        # ring appends depend on no wait: the new key is in slot pos
        rows = torch.arange(batch, device=device)
        pos = (case["valid"] - 1).long()
        assert not torch.equal(case["k"][rows, pos], k_before[rows, pos])
        return
    # the default budget restored: the same step flushes and matches the oracle
    out = step()
    ref, ref_codes, _ = oracle_replay(case)
    assert rel_l2(np32(out), ref) <= 2e-3
    fl = valid == ring
    assert np.mean(codes_np(case["ckpt"].payload)[fl] != ref_codes[fl]) < 1e-3
    assert gdnr_lib.wait_timeouts(reset=False) == 0
