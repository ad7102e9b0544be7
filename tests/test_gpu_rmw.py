"""GPU parity of the full-state read-modify-write comparator (gdnr_bf16_step,
the reference's gdn_bf16_step, prototype/gdn_replayssm_fp8_kernel.py:245-341,408-450)
against the oracle's restatement (gdn_oracle.bf16_rmw_step), marked `gpu`.

The arithmetic is fp32 on both sides; they may round differently in the last
fp32 bit (the device exp, the order of the row sums), which can move a stored
value to the neighbouring representable one. Tolerances: every written state
element is within one storage ulp plus 1e-6 of its row's largest magnitude,
and for 2-byte storage all but < 1e-3 of them are equal; the output
rel-L2 <= 2e-3 (the stated output bound; the observed error is the storage
rounding).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth
from conftest import rel_l2
from gpu_helpers import STORAGE, np32
from oracle import gdn_oracle

pytestmark = pytest.mark.gpu

# one unit in the last place, relative, of each storage dtype (an upper bound)
ULP_REL = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -23}
# the spacing of subnormals (f16's matters at the state's magnitudes)
ULP_SUB = {torch.bfloat16: 2.0 ** -133, torch.float16: 2.0 ** -24, torch.float32: 2.0 ** -149}


def _check_state(got: torch.Tensor, ref: np.ndarray, dtype) -> None:
    """Each difference at most one storage ulp of the value (subnormal
    spacing included) plus 1e-6 of the row's largest magnitude: a value that
    is the difference of two larger terms carries their fp32 rounding, which
    is many of its own ulps."""
    g = np32(got)
    diff = np.abs(g - ref)
    row_max = np.abs(ref).max(axis=-1, keepdims=True)
    bound = ULP_REL[dtype] * np.abs(ref) + 1e-6 * row_max + ULP_SUB[dtype]
    worst = int(np.argmax(diff - bound))
    assert (diff <= bound).all(), (float(g.flat[worst]), float(ref.flat[worst]), float(bound.flat[worst]))
    if dtype != torch.float32:  # an f32 store keeps every last-bit difference of the arithmetic
        assert np.mean(diff != 0) < 1e-3


@pytest.mark.parametrize("state_dtype,act", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                             (torch.float16, torch.float16), (torch.bfloat16, torch.float32)])
def test_rmw_step_matches_oracle(device, state_dtype, act):
    """C1 shape (B=64, H=16, HV=32, K=V=128), warm state, inputs passed as
    ring slices the way the reference's benches pass them
    (bench_gdn_replayssm.py:278-287)."""
    shape = synth.Shape(64)
    gen = synth.generator(31, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state0 = synth.warm_state(shape, 32, gen, device, a_log, dt_bias).to(state_dtype)
    q, k, v, g, beta = synth.token_inputs(shape, 3, gen, device, a_log, dt_bias)
    q, k, v, g, beta = (x.to(act) for x in (q, k, v, g, beta))
    state = state0.clone()
    out = gk.gdn_bf16_step(state, q[:, -1], k[:, -1], v[:, -1], g[:, -1], beta[:, -1])
    ref_out, ref_state = gdn_oracle.bf16_rmw_step(np32(state0), np32(q[:, -1]), np32(k[:, -1]), np32(v[:, -1]),
                                                  np32(g[:, -1]), np32(beta[:, -1]), STORAGE[state_dtype],
                                                  STORAGE[act])
    _check_state(state, ref_state, state_dtype)
    assert out.dtype == act
    assert rel_l2(np32(out), ref_out) <= 2e-3


def test_rmw_step_two_tokens_in_place(device):
    """Two calls in a row update the same state in place: the result is the
    oracle applied twice (from the stored, rounded state of the first)."""
    shape = synth.Shape(8)
    gen = synth.generator(32, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 16, gen, device, a_log, dt_bias).to(torch.bfloat16)
    q, k, v, g, beta = (x.to(torch.bfloat16) for x in synth.token_inputs(shape, 2, gen, device, a_log, dt_bias))
    ref_state = np32(state)
    for t in range(2):
        out = gk.gdn_bf16_step(state, q[:, t], k[:, t], v[:, t], g[:, t], beta[:, t])
        ref_out, ref_state = gdn_oracle.bf16_rmw_step(ref_state, np32(q[:, t]), np32(k[:, t]), np32(v[:, t]),
                                                      np32(g[:, t]), np32(beta[:, t]), "bf16", "bf16")
        # continue from the device's own state so that one flipped element does not propagate
        ref_state = np32(state)
        assert rel_l2(np32(out), ref_out) <= 2e-3
