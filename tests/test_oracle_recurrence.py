"""Pin the oracle's recurrence, replay, prep and cycle semantics (CPU only).

Checks come from the mathematics of the gated delta rule, not from the
oracle's own formulas:

* closed matrix form S' = e^g S (I - beta k k^T) + beta v k^T, o = S' q / sqrt(K)
  (prototype/gdn_replay_fp8_reference.py:155-161 / REPORT.md recurrence),
  evaluated with explicit float64 matrix products per head;
* delta-rule invariants: with beta = 1, g = 0 and |k| = 1 the updated state
  maps k to v exactly; with beta = 0 the state only decays;
* GQA mapping: value head j reads key head j // (HV/H) (repeat_interleave,
  ref:151-152), not j % H;
* the adjoint replay (kernel:121-176) equals the forward rebuild
  (kernel:177-228) -- the identity the HIP replay kernel relies on;
* config 0: fp32 replay from a full-precision checkpoint equals the
  per-token recurrence to <= 1e-6 (ref:353-415);
* the full-contract cycle equals the reference's replay_decode driven by the
  same prepared tokens.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import gdn_oracle


def _normalize(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def random_tokens(rng, B, T, H, HV, K, V, strong_decay=True):
    q = _normalize(rng.standard_normal((B, T, H, K)))
    k = _normalize(rng.standard_normal((B, T, H, K)))
    v = rng.standard_normal((B, T, HV, V))
    if strong_decay:
        a_log = rng.uniform(0, math.log(16), HV)
        g = -np.exp(a_log) * np.log1p(np.exp(rng.standard_normal((B, T, HV))))
    else:
        g = -rng.uniform(0.0, 0.1, (B, T, HV))
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, HV))))
    return q, k, v, g, beta


def matrix_form(state, q, k, v, g, beta):
    """Per-head explicit matrix recurrence in float64."""
    S = np.array(state, dtype=np.float64, copy=True)
    B, T, H, K = q.shape
    HV = v.shape[2]
    G = HV // H
    out = np.zeros((B, T, HV, v.shape[3]))
    for b in range(B):
        for t in range(T):
            for j in range(HV):
                h = j // G
                kk = k[b, t, h][:, None]
                S[b, j] = math.exp(g[b, t, j]) * S[b, j] @ (np.eye(K) - beta[b, t, j] * kk @ kk.T) \
                    + beta[b, t, j] * v[b, t, j][:, None] @ kk.T
                out[b, t, j] = S[b, j] @ q[b, t, h] / math.sqrt(K)
    return out, S


def test_run_kernel_matches_matrix_form():
    rng = np.random.default_rng(0)
    B, T, H, HV, K, V = 2, 5, 2, 4, 8, 6
    q, k, v, g, beta = random_tokens(rng, B, T, H, HV, K, V)
    state = rng.standard_normal((B, HV, V, K))
    out, S = gdn_oracle.run_kernel(state, q, k, v, g, beta, np.float64)
    ref_out, ref_S = matrix_form(state, q, k, v, g, beta)
    assert np.allclose(out, ref_out, rtol=1e-12, atol=1e-12)
    assert np.allclose(S, ref_S, rtol=1e-12, atol=1e-12)


def test_gqa_value_head_uses_key_head_j_div_group():
    """Changing key head 1 must change value heads 2,3 (G=2) and nothing else."""
    rng = np.random.default_rng(1)
    B, T, H, HV, K, V = 1, 3, 2, 4, 8, 8
    q, k, v, g, beta = random_tokens(rng, B, T, H, HV, K, V)
    state = rng.standard_normal((B, HV, V, K))
    out0, _ = gdn_oracle.run_kernel(state, q, k, v, g, beta, np.float64)
    k2 = k.copy()
    k2[:, :, 1] = _normalize(rng.standard_normal((B, T, K)))
    out1, _ = gdn_oracle.run_kernel(state, q, k2, v, g, beta, np.float64)
    diff = np.abs(out1 - out0).max(axis=(0, 1, 3))
    assert np.all(diff[:2] == 0) and np.all(diff[2:] > 1e-6)


def test_delta_rule_writes_v_at_k():
    """beta = 1, g = 0, |k| = 1: S' k = S k + (v - S k)(k.k) = v."""
    rng = np.random.default_rng(2)
    B, H, HV, K, V = 1, 1, 2, 16, 8
    q, k, v, _, _ = random_tokens(rng, B, 1, H, HV, K, V)
    state = rng.standard_normal((B, HV, V, K))
    _, S = gdn_oracle.run_kernel(state, q, k, v, np.zeros((B, 1, HV)), np.ones((B, 1, HV)), np.float64)
    for j in range(HV):
        assert np.allclose(S[0, j] @ k[0, 0, 0], v[0, 0, j], atol=1e-12)


def test_beta_zero_only_decays():
    rng = np.random.default_rng(3)
    B, H, HV, K, V = 2, 2, 2, 8, 8
    q, k, v, g, _ = random_tokens(rng, B, 1, H, HV, K, V)
    state = rng.standard_normal((B, HV, V, K))
    out, S = gdn_oracle.run_kernel(state, q, k, v, g, np.zeros((B, 1, HV)), np.float64)
    assert np.allclose(S, state * np.exp(g[:, 0])[:, :, None, None], rtol=1e-14)
    assert np.allclose(out[:, 0], np.einsum("bjvk,bjk->bjv", S, np.repeat(q[:, 0], 1, axis=1)) / math.sqrt(K))


def test_adjoint_replay_equals_forward_rebuild():
    rng = np.random.default_rng(4)
    B, L, H, HV, K, V = 3, 6, 2, 4, 16, 8
    _, k, v, g, beta = random_tokens(rng, B, L, H, HV, K, V, strong_decay=False)
    q = _normalize(rng.standard_normal((B, H, K)))
    state = rng.standard_normal((B, HV, V, K))
    for valid in ([0, 3, 6], [6, 6, 6], [1, 2, 9]):     # 9 > L: clamped to the ring
        adj, tq, coef = gdn_oracle.adjoint_replay(state, q, k, v, g, beta, valid, np.float64)
        fwd, _ = gdn_oracle.forward_rebuild(state, q, k, v, g, beta, valid, np.float64)
        assert np.allclose(adj, fwd, rtol=1e-10, atol=1e-12)
        # split form: out = (S T0 + sum_t c_t v_t) / sqrt(K)
        G = HV // H
        split = (np.einsum("bjvk,bjk->bjv", state, tq) + np.einsum("bjt,btjv->bjv", coef, v)) / math.sqrt(K)
        assert np.allclose(split, adj, rtol=1e-10, atol=1e-12)
        for b, n in enumerate(valid):
            assert np.all(coef[b, :, min(n, L):] == 0)
        del G


def test_config0_replay_equals_recurrence():
    """Config 0: B=1, H=HV=4, K=V=128, L=4, 64 steps, zero state, fp32,
    A_log ~ U(0, ln 16), dt_bias = 0; relative L2 <= 1e-6 for every output and
    the final state (the reference reports exactly 0, REPORT.md:226)."""
    rng = np.random.default_rng(0)
    B, T, H, HV, K, V, L = 1, 64, 4, 4, 128, 128, 4
    q = _normalize(rng.standard_normal((B, T, H, K))).astype(np.float32)
    k = _normalize(rng.standard_normal((B, T, H, K))).astype(np.float32)
    v = rng.standard_normal((B, T, HV, V)).astype(np.float32)
    a_log = rng.uniform(0, math.log(16), HV)
    g = (-np.exp(a_log) * np.log1p(np.exp(rng.standard_normal((B, T, HV))))).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, HV))))).astype(np.float32)
    zero = np.zeros((B, HV, V, K), np.float32)
    base_out, base_state = gdn_oracle.baseline_decode(zero, q, k, v, g, beta)
    rep_out, rep_state, _, _ = gdn_oracle.replay_decode(zero, q, k, v, g, beta, L, None)
    for t in range(T):
        assert gdn_oracle.relative_l2(rep_out[:, t], base_out[:, t]) <= 1e-6
    assert gdn_oracle.relative_l2(rep_state, base_state) <= 1e-6
    # the adjoint form (what the kernels compute) agrees as well, per step
    ring_start = 0
    checkpoint = zero.astype(np.float64)
    for t in range(T):
        n = t - ring_start + 1
        sl = slice(ring_start, t + 1)
        out, _, _ = gdn_oracle.adjoint_replay(checkpoint, q[:, t], k[:, sl], v[:, sl], g[:, sl], beta[:, sl], [n],
                                              np.float64)
        assert gdn_oracle.relative_l2(out, base_out[:, t]) <= 1e-6
        if n == L:
            _, checkpoint = gdn_oracle.forward_rebuild(checkpoint, q[:, t], k[:, sl], v[:, sl], g[:, sl],
                                                       beta[:, sl], [n], np.float64)
            ring_start = t + 1


def test_prep_closed_forms():
    H, K, HV, V = 2, 128, 4, 128
    rng = np.random.default_rng(5)
    mixed = rng.standard_normal((3, 2 * H * K + HV * V))
    a = np.array([[0.0, 20.0, 20.5, -30.0]] * 3)
    b = np.array([[0.0, 1.0, -1.0, 50.0]] * 3)
    a_log = np.array([0.0, 0.0, math.log(2.0), 1.0])
    dt_bias = np.zeros(HV)
    q, k, v, g, beta = gdn_oracle.prep_values(mixed, a, b, a_log, dt_bias, H, K, HV, V)
    # layout [q heads | k heads | v heads]
    assert np.allclose(q[1, 1] * np.sqrt((mixed[1, K:2 * K] ** 2).sum() + 1e-6), mixed[1, K:2 * K])
    assert np.allclose(k[2, 0] * np.sqrt((mixed[2, 2 * K:3 * K] ** 2).sum() + 1e-6), mixed[2, 2 * K:3 * K])
    assert np.array_equal(v[0, 3], mixed[0, 2 * H * K + 3 * V:2 * H * K + 4 * V])
    ss = (mixed[0, :K] ** 2).sum()
    assert np.linalg.norm(q[0, 0]) == pytest.approx(math.sqrt(ss / (ss + 1e-6)), rel=1e-12)
    assert g[0, 0] == pytest.approx(-math.log(2.0))              # -exp(0) * softplus(0)
    assert g[0, 1] == pytest.approx(-math.log(1.0 + math.exp(20.0)))  # x <= 20: log(1 + exp(x))
    assert g[0, 2] == pytest.approx(-2.0 * 20.5)                  # x > 20: x, times exp(ln 2)
    assert g[0, 3] == pytest.approx(-math.e * math.exp(-30.0), rel=1e-6)   # softplus(x) ~ e^x for x << 0
    assert beta[0, 0] == 0.5 and beta[0, 3] == pytest.approx(1.0)
    assert beta[0, 1] == pytest.approx(1 / (1 + math.exp(-1)))


def test_prep_ring_writes_only_slot_pos():
    H, K, HV, V, L, B = 2, 128, 4, 128, 4, 3
    rng = np.random.default_rng(6)
    mixed = rng.standard_normal((B, 2 * H * K + HV * V)).astype(np.float32)
    a = rng.standard_normal((B, HV)).astype(np.float32)
    b = rng.standard_normal((B, HV)).astype(np.float32)
    rings = [np.full((B, L, H, K), 7.0, np.float32), np.full((B, L, HV, V), 7.0, np.float32),
             np.full((B, L, HV), 7.0, np.float32), np.full((B, L, HV), 7.0, np.float32)]
    q_out = np.zeros((B, H, K), np.float32)
    pos = np.array([0, 3, -1])                                   # -1: nothing appended
    gdn_oracle.prep_ring(mixed, a, b, np.zeros(HV), np.zeros(HV), pos, q_out, *rings)
    for r in rings:
        assert np.all(r[0, 1:] == 7.0) and np.all(r[1, :3] == 7.0) and np.all(r[2] == 7.0)
        assert not np.any(r[0, 0] == 7.0) and not np.any(r[1, 3] == 7.0)
    # stored values are bf16-rounded
    assert np.array_equal(rings[1][1, 3], gdn_oracle.bf16_round(mixed[1, 2 * H * K:].reshape(HV, V)))


def test_full_contract_cycle_equals_replay_decode():
    """The cycle (prep -> adjoint replay, flush at fill == L with vblock32
    requant) produces the same outputs as the reference's replay_decode
    (forward replay from the dequantised checkpoint, ref:189-244) fed with the
    same prepared, bf16-rounded tokens."""
    rng = np.random.default_rng(7)
    B, H, K, HV, V, L, T = 2, 2, 128, 4, 128, 4, 10
    a_log = rng.uniform(0, math.log(16), HV)
    dt_bias = np.zeros(HV)
    state = rng.standard_normal((B, HV, V, K)).astype(np.float32) * 0.05
    ck = gdn_oracle.quantize_checkpoint(state, "vblock", 32)
    mixed = rng.standard_normal((B, T, 2 * H * K + HV * V)).astype(np.float32)
    a = rng.standard_normal((B, T, HV)).astype(np.float32)
    b = rng.standard_normal((B, T, HV)).astype(np.float32)
    outs, codes, scale = gdn_oracle.full_contract_decode(ck.payload, ck.scale, mixed, a, b, a_log, dt_bias, L, H, K,
                                                         HV, V, dtype=np.float64)
    toks = [gdn_oracle.prep_values(mixed[:, t], a[:, t], b[:, t], a_log, dt_bias, H, K, HV, V) for t in range(T)]
    r = lambda x: gdn_oracle.bf16_round(np.asarray(x, np.float32))
    q = np.stack([r(t[0]) for t in toks], 1)
    k = np.stack([r(t[1]) for t in toks], 1)
    v = np.stack([r(t[2]) for t in toks], 1)
    g = np.stack([r(t[3]) for t in toks], 1)
    be = np.stack([r(t[4]) for t in toks], 1)
    deq0 = gdn_oracle.dequantize_checkpoint(ck)
    ref, _, _, _ = gdn_oracle.replay_decode(deq0, q, k, v, g, be, L, "vblock", 32, np.float64)
    assert gdn_oracle.relative_l2(outs, ref) < 1e-9
    # two flushes happened (steps 4 and 8): the checkpoint was rewritten
    assert codes.shape == ck.payload.shape and not np.array_equal(codes, ck.payload)
    assert scale.dtype == np.float16


def test_error_metrics_definition():
    e = np.array([3.0, 4.0])
    m = gdn_oracle.error_metrics(np.array([3.0, 5.0]), e)
    assert m["max_abs"] == 1.0 and m["mean_abs"] == 0.5
    assert m["relative_l2"] == pytest.approx(1.0 / 5.0)
    assert m["cosine"] == pytest.approx((9 + 20) / (5 * math.sqrt(34)))
    assert gdn_oracle.error_metrics(np.zeros(3), np.zeros(3))["relative_l2"] == 0.0
