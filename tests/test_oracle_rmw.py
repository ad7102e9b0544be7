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
