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


@pytest.mark.parametrize("state_dtype,act,gate,scale", [(torch.bfloat16, torch.bfloat16, torch.bfloat16, None),
                                                        (torch.bfloat16, torch.bfloat16, torch.float32, 0.05),
                                                        (torch.float32, torch.float16, torch.float16, None),
                                                        (torch.float16, torch.float32, torch.float32, None)])
def test_packed_step_matches_oracle(device, state_dtype, act, gate, scale):
    """The production contract (gdnr_bf16_step_packed): 12 live sequences in
    out-of-order slots of a 20-slot state plus two padding entries (slot 0),
    raw mixed_qkv rows, q/k norm and gates in the kernel. Live slots follow
    the oracle; slots not in the batch keep their bytes; the padding outputs
    are not checked (they read the null slot)."""
    B_live, S = 12, 20
    shape = synth.Shape(B_live)
    gen = synth.generator(33, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    warm = synth.warm_state(synth.Shape(S), 24, gen, device, a_log, dt_bias).to(state_dtype)
    live_slots = [7, 2, 19, 11, 4, 15, 1, 9, 13, 6, 17, 3]
    slots = live_slots[:5] + [0] + live_slots[5:] + [0]
    mixed, a, b = synth.raw_step_inputs(synth.Shape(len(slots)), 1, gen, device, dtype=act, gate_dtype=gate)
    mixed, a, b = mixed[:, 0].contiguous(), a[:, 0].contiguous(), b[:, 0].contiguous()
    state = warm.clone()
    idx = torch.tensor(slots, dtype=torch.int32, device=device)
    out = gk.gdn_bf16_step_packed(mixed, a, b, a_log, dt_bias, state, idx, scale=scale)
    ref_out, ref_state = gdn_oracle.packed_rmw_step(np32(warm), slots, np32(mixed), np32(a), np32(b), np32(a_log),
                                                    np32(dt_bias), shape.heads, STORAGE[state_dtype], STORAGE[act],
                                                    scale=scale)
    assert out.shape == (len(slots), 1, shape.value_heads, shape.value_dim) and out.dtype == act
    live = [i for i, s in enumerate(slots) if s != 0]
    _check_state(state[live_slots], ref_state[live_slots], state_dtype)
    untouched = [s for s in range(1, S) if s not in live_slots]
    assert torch.equal(state[untouched], warm[untouched])
    assert rel_l2(np32(out)[live], ref_out[live]) <= 2e-3


def test_packed_step_equals_the_plain_step_on_prepared_inputs(device):
    """f32 activations: the packed kernel's in-kernel q/k norm and gates give
    the plain comparator's result on the same values prepared in f32 on the
    device (torch), states and outputs within the storage-ulp bound."""
    shape = synth.Shape(16)
    gen = synth.generator(34, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    warm = synth.warm_state(shape, 16, gen, device, a_log, dt_bias).to(torch.bfloat16)
    mixed, a, b = synth.raw_step_inputs(shape, 1, gen, device, dtype=torch.float32, gate_dtype=torch.float32)
    mixed, a, b = mixed[:, 0].contiguous(), a[:, 0].contiguous(), b[:, 0].contiguous()
    HK = shape.heads * shape.key_dim
    q = mixed[:, :HK].reshape(16, shape.heads, -1)
    k = mixed[:, HK:2 * HK].reshape(16, shape.heads, -1)
    q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
    k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    v = mixed[:, 2 * HK:].reshape(16, shape.value_heads, -1).contiguous()
    g = -torch.exp(a_log) * torch.nn.functional.softplus(a + dt_bias, beta=1.0, threshold=20.0)
    beta = torch.sigmoid(b)
    s_plain = torch.cat([warm[:1], warm]).clone()
    s_packed = s_plain.clone()
    out_plain = gk.gdn_bf16_step(s_plain[1:], q.contiguous(), k.contiguous(), v, g.contiguous(), beta.contiguous())
    idx = torch.arange(1, 17, dtype=torch.int32, device=device)
    out_packed = gk.gdn_bf16_step_packed(mixed, a, b, a_log, dt_bias, s_packed, idx)
    _check_state(s_packed[1:], np32(s_plain[1:]), torch.bfloat16)
    assert rel_l2(np32(out_packed[:, 0]), np32(out_plain)) <= 2e-3
