"""Pins of the oracle's full-state read-modify-write step (gdn_oracle.bf16_rmw_step,
the reference's _gdn_bf16_step_kernel, prototype/gdn_replayssm_fp8_kernel.py:245-341).

- With f32 storage it is the one-token step of run_kernel (ref:137-163), which
  the recurrence tests pin by closed forms.
- From a zero state: S = beta v k^T and o = beta v (k . q) K^-1/2 (closed form).
- beta = 0 is pure decay: S = exp(g) S, o = exp(g) (S q) K^-1/2.
- The storage rounding of S and o agrees with torch's bf16 / f16 casts.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn_oracle

B, H, HV, K, V = 2, 2, 4, 128, 128


def _inputs(seed=0):
    rng = np.random.default_rng(seed)
    state = (0.3 * rng.standard_normal((B, HV, V, K))).astype(np.float32)
    q = rng.standard_normal((B, H, K)).astype(np.float32)
    k = rng.standard_normal((B, H, K)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, HV, V)).astype(np.float32)
    g = (-rng.random((B, HV)) * 2).astype(np.float32)
    beta = rng.random((B, HV)).astype(np.float32)
    return state, q, k, v, g, beta


def test_f32_storage_is_one_recurrence_token():
    state, q, k, v, g, beta = _inputs()
    out, new = gdn_oracle.bf16_rmw_step(state, q, k, v, g, beta, "f32", "f32")
    ref_out, ref_state = gdn_oracle.run_kernel(state, q[:, None], k[:, None], v[:, None], g[:, None], beta[:, None])
    np.testing.assert_allclose(out, ref_out[:, 0], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(new, ref_state, rtol=1e-6, atol=1e-7)


def test_zero_state_closed_form():
    state, q, k, v, g, beta = _inputs(1)
    out, new = gdn_oracle.bf16_rmw_step(np.zeros_like(state), q, k, v, g, beta, "f32", "f32")
    kk = np.repeat(k.astype(np.float64), HV // H, axis=1)
    qq = np.repeat(q.astype(np.float64), HV // H, axis=1)
    expect_state = beta[..., None, None] * v[..., None].astype(np.float64) * kk[:, :, None, :]
    expect_out = beta[..., None] * v * (kk * qq).sum(-1)[..., None] / np.sqrt(K)
    np.testing.assert_allclose(new, expect_state, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(out, expect_out, rtol=1e-5, atol=1e-6)


def test_zero_beta_is_pure_decay():
    state, q, k, v, g, _ = _inputs(2)
    out, new = gdn_oracle.bf16_rmw_step(state, q, k, v, g, np.zeros_like(g), "f32", "f32")
    decayed = state.astype(np.float64) * np.exp(g.astype(np.float64))[..., None, None]
    qq = np.repeat(q.astype(np.float64), HV // H, axis=1)
    np.testing.assert_allclose(new, decayed, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(out, (decayed * qq[:, :, None, :]).sum(-1) / np.sqrt(K), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("storage,torch_dtype", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_storage_rounding_matches_torch(storage, torch_dtype):
    state, q, k, v, g, beta = _inputs(3)
    out32, new32 = gdn_oracle.bf16_rmw_step(state, q, k, v, g, beta, "f32", "f32")
    out, new = gdn_oracle.bf16_rmw_step(state, q, k, v, g, beta, storage, storage)
    np.testing.assert_array_equal(new, torch.from_numpy(new32).to(torch_dtype).float().numpy())
    np.testing.assert_array_equal(out, torch.from_numpy(out32).to(torch_dtype).float().numpy())


# --- the production-contract form (gdn_oracle.packed_rmw_step) -------------

S_SLOTS = 5


def _packed_inputs(seed=1):
    rng = np.random.default_rng(seed)
    mixed = rng.standard_normal((B, 2 * H * K + HV * V)).astype(np.float32)
    a = rng.standard_normal((B, HV)).astype(np.float32)
    b = rng.standard_normal((B, HV)).astype(np.float32)
    a_log = rng.random(HV).astype(np.float32)
    dt_bias = (rng.random(HV) - 1).astype(np.float32)
    return mixed, a, b, a_log, dt_bias


def test_packed_zero_state_closed_form():
    """Zero state in slots 3 and 1: S = sigmoid(b) v khat^T and
    o = sigmoid(b) v (khat . qhat) K^-1/2, with qhat, khat = x / sqrt(|x|^2 +
    1e-6) and sigmoid from torch; the other slots keep their values."""
    mixed, a, b, a_log, dt_bias = _packed_inputs()
    rng = np.random.default_rng(9)
    state = (0.1 * rng.standard_normal((S_SLOTS, HV, V, K))).astype(np.float32)
    slots = [3, 1]
    state[slots] = 0
    out, new = gdn_oracle.packed_rmw_step(state, slots, mixed, a, b, a_log, dt_bias, H, "f32", "f32")
    t = torch.from_numpy(mixed).double()
    q = t[:, :H * K].reshape(B, H, K)
    k = t[:, H * K:2 * H * K].reshape(B, H, K)
    q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
    k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    v = t[:, 2 * H * K:].reshape(B, HV, V)
    beta = torch.sigmoid(torch.from_numpy(b).double())
    kt = k.repeat_interleave(HV // H, dim=1)
    qt = q.repeat_interleave(HV // H, dim=1)
    want_s = beta[..., None, None] * v[..., None] * kt[:, :, None, :]
    want_o = beta[..., None] * v * (kt * qt).sum(-1)[..., None] * K ** -0.5
    for i, sl in enumerate(slots):
        np.testing.assert_allclose(new[sl], want_s[i].numpy(), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(out[:, 0], want_o.numpy(), rtol=1e-4, atol=1e-6)
    for sl in (0, 2, 4):
        assert np.array_equal(new[sl], state[sl])


def test_packed_closed_gate_is_softplus_decay():
    """b = -200 closes the write (beta ~ 0): the slot's state is only decayed by
    exp(-exp(A_log) softplus(a + dt_bias)), softplus from torch with threshold
    20 (a + dt_bias above 20 included)."""
    mixed, a, b, a_log, dt_bias = _packed_inputs(2)
    a[0, :2] = 25.0  # past the softplus threshold
    b[:] = -200.0
    rng = np.random.default_rng(4)
    state = (0.1 * rng.standard_normal((S_SLOTS, HV, V, K))).astype(np.float32)
    _, new = gdn_oracle.packed_rmw_step(state, [2, 4], mixed, a, b, a_log, dt_bias, H, "f32", "f32")
    x = torch.from_numpy(a).double() + torch.from_numpy(dt_bias).double()
    gamma = torch.exp(-torch.exp(torch.from_numpy(a_log).double()) *
                      torch.nn.functional.softplus(x, beta=1.0, threshold=20.0)).numpy()
    for i, sl in enumerate((2, 4)):
        np.testing.assert_allclose(new[sl], state[sl] * gamma[i][:, None, None], rtol=1e-5, atol=1e-8)


def test_packed_permutation_and_null_slot():
    """Permuting the batch (with its slots) permutes the outputs and stores the
    same states; a padding entry (slot 0) and an out-of-range slot write
    nothing."""
    rng = np.random.default_rng(5)
    mixed = rng.standard_normal((4, 2 * H * K + HV * V)).astype(np.float32)
    a, b = rng.standard_normal((4, HV)).astype(np.float32), rng.standard_normal((4, HV)).astype(np.float32)
    a_log, dt_bias = rng.random(HV).astype(np.float32), (rng.random(HV) - 1).astype(np.float32)
    state = (0.1 * rng.standard_normal((S_SLOTS, HV, V, K))).astype(np.float32)
    slots = np.array([4, 0, 1, 7])
    out, new = gdn_oracle.packed_rmw_step(state, slots, mixed, a, b, a_log, dt_bias, H)
    perm = np.array([2, 0, 3, 1])
    out_p, new_p = gdn_oracle.packed_rmw_step(state, slots[perm], mixed[perm], a[perm], b[perm], a_log, dt_bias, H)
    assert np.array_equal(out_p, out[perm])
    assert np.array_equal(new_p, new)
    for sl in (0, 2, 3):
        assert np.array_equal(new[sl], state[sl])
    assert not np.array_equal(new[4], state[4]) and not np.array_equal(new[1], state[1])


def test_packed_scale_only_scales_the_output():
    """The production op's scale multiplies o and nothing else: a scale of
    2 K^-1/2 gives exactly twice the output (a power of two) and the same
    stored states."""
    mixed, a, b, a_log, dt_bias = _packed_inputs(3)
    rng = np.random.default_rng(6)
    state = (0.1 * rng.standard_normal((S_SLOTS, HV, V, K))).astype(np.float32)
    out1, new1 = gdn_oracle.packed_rmw_step(state, [1, 3], mixed, a, b, a_log, dt_bias, H, "f32", "f32")
    out2, new2 = gdn_oracle.packed_rmw_step(state, [1, 3], mixed, a, b, a_log, dt_bias, H, "f32", "f32",
                                            scale=2 * K ** -0.5)
    assert np.array_equal(out2, 2 * out1)
    assert np.array_equal(new2, new1)
