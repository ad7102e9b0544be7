"""GPU parity under the reference's own input regime (marked `gpu`).

The reference validates its kernels on `make_inputs`
(prototype/gdn_replayssm_fp8_kernel.py:1238-1289): A_log ~ U(0,1),
dt_bias ~ U(-4,-3), so gamma = exp(g) ~ 0.95 per token, and a 0.02 N(0,1)
state. Under these gates the checkpoint's weight in the output,
lam = prod_t gamma_t, is still ~0.3 after a full 16-token ring, so the FP8
matvec S_0 T_0, the scale gather and the flush's lam scale S_0 term carry a
large share of every output and of every rebuilt state (under BASELINE's
fast-decay gates lam is ~5e-7 at fill 16, and an error there would hide
under the 2e-3 gate). Every check here runs in that regime:

- the reference's own validation protocol, `validate_once` (:1292-1357), at
  B=2 and L in {4, 8, 16, 32}: the replay of a full ring against `run_kernel`
  from the dequantised checkpoint (gate 3; the reference logs 1.654e-3 to
  1.697e-3, results/kernel_sweep_blockv_warps.log:2,24,46,68), and the
  flushed checkpoint against the reference quantiser on the fp32 rebuild
  (the reference logs 6.31e-3 to 6.89e-3 there);
- the replay at every fill 0..16, flushes at L = 4 / 16 / 64, config 1 at full
  size, the B=64 L=16 full-contract cell, the long-ring cycle, and the other
  decode-kernel shapes (V = 64 / 256, odd GQA groups), against the fp64
  oracle;
- the lam path of the flush in isolation: beta = 0 and a constant g < 0 per
  head, so the rebuilt state is lam S_0 with lam in 0.3 .. 0.9; its oracle is
  the fp32 recurrence followed by the reference quantiser.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth
import gdnr_lib
from conftest import rel_l2
from gpu_helpers import codes_np, make_replay_case, np32, oracle_replay, run_replay
from oracle import gdn_oracle

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-3
CODE_FLIP_TOL = 1e-3
H, HV, K, V = 16, 32, 128, 128


def _fp16_ulps(got, want):
    g = np.asarray(got, dtype=np.float16).view(np.uint16).astype(np.int64)
    w = np.asarray(want, dtype=np.float16).view(np.uint16).astype(np.int64)
    return np.abs(g - w)


def _make_inputs(batch, cache_len, seed=0):
    """The reference's make_inputs (kernel:1238-1289) on a seeded CPU
    generator: q, k_cache L2-normalised then bf16; v_cache bf16 N(0,1);
    g = -exp(A_log) softplus(a + dt_bias) and beta = sigmoid(N(0,1)), both
    bf16; state 0.02 N(0,1) f32."""
    gen = torch.Generator().manual_seed(seed)
    q = F.normalize(torch.randn(batch, H, K, generator=gen), dim=-1).to(torch.bfloat16)
    k_cache = F.normalize(torch.randn(batch, cache_len, H, K, generator=gen), dim=-1).to(torch.bfloat16)
    v_cache = torch.randn(batch, cache_len, HV, V, generator=gen).to(torch.bfloat16)
    a = torch.randn(batch, cache_len, HV, generator=gen)
    a_log = torch.rand(HV, generator=gen)
    dt_bias = torch.rand(HV, generator=gen) - 4.0
    g_cache = (-a_log.exp() * F.softplus(a + dt_bias)).to(torch.bfloat16)
    beta_cache = torch.sigmoid(torch.randn(batch, cache_len, HV, generator=gen)).to(torch.bfloat16)
    state = torch.randn(batch, HV, V, K, generator=gen) * 0.02
    return q, k_cache, v_cache, g_cache, beta_cache, state


# gate 3 for the output; for the flushed state, well under the reference's
# own 6.31e-3 .. 6.89e-3 (measured on MI355X: 2.7e-5 .. 4.8e-4, the code
# flips of an fp32 rebuild against an fp64 one, ~1.4e-4 of the codes)
VALIDATE_OUT_TOL = 2e-3
VALIDATE_STATE_TOL = 1e-3


@pytest.mark.parametrize("cache_len", [4, 8, 16, 32])
def test_validate_once_protocol(device, cache_len):
    """validate_once (kernel:1292-1357): quantise the state; replay a full ring
    (valid_len = L, no flush) and compare with run_kernel from the dequantised
    checkpoint; then flush, and compare the dequantised new checkpoint with
    the reference quantiser applied to run_kernel's fp32 final state."""
    batch = 2
    q, k, v, g, beta, state = _make_inputs(batch, cache_len)
    ck = gk.quantize_checkpoint(state.to(device))
    codes0, scale0 = codes_np(ck.payload).copy(), ck.scale.cpu().numpy().copy()
    direct = gdn_oracle.quantize_checkpoint(state.numpy(), "vblock", 32)
    assert np.array_equal(codes0, direct.payload)
    assert np.array_equal(scale0.view(np.uint16), direct.scale.astype(np.float16).view(np.uint16))
    dq, dk, dv, dg, db = (t.to(device) for t in (q, k, v, g, beta))
    valid = torch.full((batch,), cache_len, dtype=torch.int32, device=device)
    flush = torch.zeros(batch, dtype=torch.bool, device=device)
    out = gk.gdn_replay_fp8(ck.payload, ck.scale, dq, dk, dv, dg, db, valid, flush)
    deq = gdn_oracle.dequantize_vblock32(codes0, scale0)
    qx = np.repeat(np32(q)[:, None], cache_len, axis=1)
    ref_out, ref_state = gdn_oracle.run_kernel(deq, qx, np32(k), np32(v), np32(g), np32(beta), np.float64)
    out_err = rel_l2(np32(out), ref_out[:, -1])
    flush.fill_(True)
    gk.gdn_replay_fp8(ck.payload, ck.scale, dq, dk, dv, dg, db, valid, flush)
    got_state = gdn_oracle.dequantize_vblock32(codes_np(ck.payload), ck.scale.cpu().numpy())
    want = gdn_oracle.quantize_checkpoint(ref_state.astype(np.float32), "vblock", 32)
    state_err = rel_l2(got_state, gdn_oracle.dequantize_checkpoint(want))
    flips = float(np.mean(codes_np(ck.payload) != want.payload))
    lam = float(np.mean(np.exp(np32(g).astype(np.float64).sum(axis=1))))
    print(f"validate_once L={cache_len}: output {out_err:.4e}, flush state {state_err:.4e}, code flips {flips:.2e}, "
          f"mean lam {lam:.3f}")
    assert out_err <= VALIDATE_OUT_TOL, out_err
    assert state_err <= VALIDATE_STATE_TOL, state_err


@pytest.mark.parametrize("batch", [17, 64])
def test_replay_every_fill(device, batch):
    """Gate 3 at every ring fill 0..16, L = 16, no flush (a full ring
    replays, its query as an operand block of its own). 17 sequences, one per
    fill (one-unit workgroups, which take their products before the chain's
    flag), and 64 at fills b mod 17 (the headline's 4-unit workgroups, which
    take the flag first)."""
    valid = [b % 17 for b in range(batch)]
    plan = gdnr_lib.decode_plan(batch, H, 32, 128, 16)
    assert plan is not None and plan["units"] == (1 if batch == 17 else 4), plan
    case = make_replay_case(batch, 16, device, seed=31, valid=valid, reference_dist=True)
    out = run_replay(case)
    ref, _, _ = oracle_replay(case)
    errs = [rel_l2(np32(out)[i], ref[i]) for i in range(batch) if valid[i] > 0]
    lam = np.exp(np32(case["g"]).astype(np.float64).cumsum(axis=1)).mean(axis=(0, 2))
    print(f"replay per fill: max {max(errs):.3e}; mean lam at fills 1/4/8/16: {lam[0]:.3f} {lam[3]:.3f} {lam[7]:.3f} "
          f"{lam[15]:.3f}")
    assert max(errs) <= OUT_TOL, errs
    assert rel_l2(np32(out), ref) <= OUT_TOL
    assert lam[15] > 0.2  # the checkpoint still carries the output at a full ring


@pytest.mark.parametrize("ring_len", [4, 16, 64])
def test_flush_ring_lengths(device, ring_len):
    """Flush at L = 4 / 16 / 64 beside a partial flush, a one-token flush and a
    replay: outputs vs the fp64 oracle; codes up to rounding-boundary flips;
    scales within one fp16 ulp; the replaying sequence's checkpoint untouched."""
    case = make_replay_case(4, ring_len, device, seed=40 + ring_len, valid=[ring_len, ring_len - 1, 1, ring_len],
                            flush=[1, 1, 1, 0], reference_dist=True)
    out = run_replay(case, block_v=32)
    ref, ref_codes, ref_scale = oracle_replay(case)
    got = codes_np(case["ckpt"].payload)
    err, flips = rel_l2(np32(out), ref), float(np.mean(got[:3] != ref_codes[:3]))
    print(f"flush L={ring_len}: output {err:.3e}, code flips {flips:.2e}")
    assert err <= OUT_TOL, err
    assert flips < CODE_FLIP_TOL, flips
    assert _fp16_ulps(case["ckpt"].scale.cpu().numpy(), ref_scale).max() <= 1
    assert np.array_equal(got[3], case["codes0"][3])


def test_config1_full_size(device):
    """Config 1's shape (B=64, L=16, fills uniform in 1..16, the sequences at
    16 flushing in the same launch) in the reference regime."""
    gen = torch.Generator().manual_seed(2)
    valid = torch.randint(1, 17, (64,), generator=gen, dtype=torch.int32)
    valid[:6] = 16
    case = make_replay_case(64, 16, device, seed=50, valid=valid, flush=valid == 16, reference_dist=True)
    out = run_replay(case)
    ref, ref_codes, ref_scale = oracle_replay(case, np.float32)
    fl = (valid == 16).numpy()
    codes = codes_np(case["ckpt"].payload)
    err, flips = rel_l2(np32(out), ref), float(np.mean(codes[fl] != ref_codes[fl]))
    print(f"config 1 (reference regime): output {err:.3e}, code flips {flips:.2e}")
    assert err <= OUT_TOL, err
    assert flips < CODE_FLIP_TOL, flips
    ulps = _fp16_ulps(case["ckpt"].scale.cpu().numpy()[fl], ref_scale[fl])
    assert ulps.max() <= 1 and ulps.mean() < 0.01, (ulps.max(), ulps.mean())
    assert np.array_equal(codes[~fl], case["codes0"][~fl])
    assert np.array_equal(case["ckpt"].scale.cpu().numpy()[~fl].view(np.uint16),
                          case["scale0"][~fl].view(np.uint16))


def _cycle(batch, window, seed, device, steps, phase, idx=None, shape=None):
    """A full-contract cycle (one fused launch per step; fill (phase + s) % L + 1,
    flush at fill L) in the reference regime; returns (got outputs, oracle
    outputs, got codes, oracle codes, got scales, oracle scales) of the
    sequences idx (default all; sequences are independent)."""
    shape = shape or synth.Shape(batch)
    gen = synth.generator(seed, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device, reference_dist=True)
    state = synth.warm_state(shape, 0, gen, device, a_log, dt_bias, reference_dist=True)
    mixed, a, b = synth.raw_step_inputs(shape, steps, gen, device)
    ck = gk.quantize_checkpoint(state)
    codes0, scale0 = codes_np(ck.payload).copy(), ck.scale.cpu().numpy().copy()
    q_out = torch.zeros(batch, shape.heads, shape.key_dim, dtype=torch.bfloat16, device=device)
    rings = [torch.zeros(batch, window, shape.heads, shape.key_dim, dtype=torch.bfloat16, device=device),
             torch.zeros(batch, window, shape.value_heads, shape.value_dim, dtype=torch.bfloat16, device=device),
             torch.zeros(batch, window, shape.value_heads, dtype=torch.bfloat16, device=device),
             torch.zeros(batch, window, shape.value_heads, dtype=torch.bfloat16, device=device)]
    phase_t = torch.as_tensor(phase, dtype=torch.int32, device=device)
    outs = []
    for step in range(steps):
        fill = (phase_t + step) % window + 1
        outs.append(np32(gk.gdn_prep_replay_fp8(mixed[:, step].contiguous(), a[:, step].contiguous(),
                                                b[:, step].contiguous(), a_log, dt_bias, fill - 1, ck.payload,
                                                ck.scale, q_out, *rings, fill, fill == window)))
    idx = np.arange(batch) if idx is None else np.asarray(idx)
    ref, ref_codes, ref_scale = gdn_oracle.full_contract_decode(
        codes0[idx], scale0[idx], np32(mixed)[idx], np32(a)[idx], np32(b)[idx], np32(a_log), np32(dt_bias), window,
        shape.heads, shape.key_dim, shape.value_heads, shape.value_dim, phase=np.asarray(phase)[idx],
        dtype=np.float64)
    return (np.stack(outs, axis=1)[idx], ref, codes_np(ck.payload)[idx], ref_codes, ck.scale.cpu().numpy()[idx],
            ref_scale)


@pytest.mark.parametrize("batch,window", [(64, 16), (8, 4)])
def test_full_contract_cell(device, batch, window):
    """Config 2's headline cell (and a small one) over one ring cycle plus two
    steps with spread phases (every sequence flushes once), all sequences
    against the oracle's full-contract cycle (prep, replays, flushes,
    requantisation); at B=64 one sequence of each phase and a few more."""
    phase = np.arange(batch) % window
    idx = None if batch <= 8 else np.array(sorted(set(range(window)) | {batch // 2 + 3, batch - 2, batch - 1}))
    got, ref, codes, ref_codes, scale, ref_scale = _cycle(batch, window, 60 + batch, device, window + 2, phase, idx)
    err, flips = rel_l2(got, ref), float(np.mean(codes != ref_codes))
    print(f"full contract B={batch} L={window}: output {err:.3e}, code flips {flips:.2e}")
    assert err <= OUT_TOL, err
    assert flips < CODE_FLIP_TOL, flips
    assert _fp16_ulps(scale, ref_scale).max() <= 1


@pytest.mark.parametrize("window", [32, 64])
def test_long_ring_cycle(device, window):
    """The long-ring path over one cycle with mixed phases in the reference regime."""
    phase = np.array([0, window // 2, window - 1])
    got, ref, codes, ref_codes, scale, ref_scale = _cycle(3, window, 70 + window, device, window + 1, phase)
    err, flips = rel_l2(got, ref), float(np.mean(codes != ref_codes))
    print(f"long ring L={window}: output {err:.3e}, code flips {flips:.2e}")
    assert err <= OUT_TOL, err
    assert flips < CODE_FLIP_TOL, flips
    assert _fp16_ulps(scale, ref_scale).max() <= 1


OTHER_SHAPES = {
    # id: (batch, value_heads, value_dim[, ring length, activation dtype])  (H = 16 key heads; L = 16, bf16 when absent)
    "V64_G2_B64": (64, 32, 64),
    "V256_G1_B32": (32, 16, 256),
    "V256_G1_B64": (64, 16, 256),
    "V256_G2_B64": (64, 32, 256),
    "V128_G1_B16": (16, 16, 128),
    "V128_G1_B64": (64, 16, 128),
    # rings of 16-token chunks: V = 64 and 128, G = 1 and 2, up to the decode kernel's batch limit, and f16
    "L48_V64_G2_B8": (8, 32, 64, 48),
    "L64_V128_G1_B16": (16, 16, 128, 64),
    "L32_V128_G2_B16": (16, 32, 128, 32),
    "L64_V128_G2_B8_f16": (8, 32, 128, 64, torch.float16),
    "L16_V128_G2_B8_f16": (8, 32, 128, 16, torch.float16),
}


@pytest.mark.parametrize("case_id", list(OTHER_SHAPES))
def test_other_decode_shapes(device, case_id):
    """The decode kernel's other instantiations (V = 64 / 256, odd GQA groups,
    small and large batches), alternate sequences flushing so that partner
    units help: outputs vs the fp64 oracle, codes to rounding-boundary flips,
    scales within one fp16 ulp, replaying sequences untouched."""
    batch, value_heads, value_dim, *rest = OTHER_SHAPES[case_id]
    ring = rest[0] if rest else 16
    act = rest[1] if len(rest) > 1 else torch.bfloat16
    plan = gdnr_lib.decode_plan(batch, H, value_heads, value_dim, ring, act=act)
    assert plan is not None
    valid = np.where(np.arange(batch) % 2 == 0, ring, 1 + (7 * np.arange(batch)) % (ring - 1)).astype(np.int32)
    case = make_replay_case(batch, ring, device, seed=80 + batch + ring, value_heads=value_heads, value_dim=value_dim,
                            dtype=act, valid=valid, flush=valid == ring, reference_dist=True)
    out = run_replay(case, block_v=min(128, value_dim))
    ref, ref_codes, ref_scale = oracle_replay(case, np.float32)
    fl = valid == ring
    codes = codes_np(case["ckpt"].payload)
    err, flips = rel_l2(np32(out), ref), float(np.mean(codes[fl] != ref_codes[fl]))
    print(f"{case_id}: output {err:.3e}, code flips {flips:.2e}")
    assert err <= OUT_TOL, err
    assert flips < CODE_FLIP_TOL, flips
    assert _fp16_ulps(case["ckpt"].scale.cpu().numpy()[fl], ref_scale[fl]).max() <= 1
    assert np.array_equal(codes[~fl], case["codes0"][~fl])


LAMBDA_FLIP_TOL = 1e-4


@pytest.mark.parametrize("ring_len,regime", [(4, "mid"), (16, "mid"), (64, "mid"), (16, "tiny"), (64, "tiny")])
def test_lambda_path_flush(device, ring_len, regime):
    """beta = 0 on every token and a constant g_h < 0 per (sequence, head), so
    the flush rebuilds lam S_0 with lam = exp(L g_h): in 0.3 .. 0.9 ("mid"),
    or log-uniform in 1e-28 .. 1e-6 ("tiny": lam scale on both sides of
    2^-64, where the one-chunk decode rebuild stops folding lam scale into
    the quotient and forms (lam scale) x code instead). The oracle is the
    fp32 recurrence S <- exp(g) S token by token (ref:155-161), then the
    reference quantiser. Codes may differ only where the two roundings
    straddle an e4m3 rounding boundary (< 1e-4 of the codes); scales within
    one fp16 ulp. B = 64 with alternate sequences flushing (helpers rebuild
    some vblocks)."""
    batch = 64
    valid = np.where(np.arange(batch) % 2 == 0, ring_len, 1).astype(np.int32)
    case = make_replay_case(batch, ring_len, device, seed=90 + ring_len, valid=valid, flush=valid == ring_len,
                            reference_dist=True)
    gen = torch.Generator().manual_seed(ring_len)
    if regime == "mid":
        lam = torch.rand(batch, 1, HV, generator=gen) * 0.6 + 0.3
    else:
        lam = 10.0 ** (torch.rand(batch, 1, HV, generator=gen, dtype=torch.float64) * -22.0 - 6.0)
    g = (lam.log() / ring_len).expand(batch, ring_len, HV).to(torch.bfloat16)
    case["g"] = g.contiguous().to(device)
    case["beta"] = torch.zeros_like(case["beta"])
    out = run_replay(case)
    ref, ref_codes, ref_scale = oracle_replay(case, np.float32)
    fl = valid == ring_len
    codes = codes_np(case["ckpt"].payload)
    flips = float(np.mean(codes[fl] != ref_codes[fl]))
    ulps = _fp16_ulps(case["ckpt"].scale.cpu().numpy()[fl], ref_scale[fl])
    realised = np.exp(np32(case["g"]).astype(np.float64).sum(axis=1))[fl]
    print(f"lam path L={ring_len} {regime}: lam {realised.min():.3g}..{realised.max():.3g}, code flips {flips:.2e}, "
          f"scale ulps max {ulps.max()} (mean {ulps.mean():.2e})")
    if regime == "mid":
        assert realised.min() > 0.25 and realised.max() < 0.95
    else:
        assert realised.min() < 1e-25 and realised.max() > 1e-9
    assert flips < LAMBDA_FLIP_TOL, flips
    assert ulps.max() <= 1
    assert rel_l2(np32(out), ref) <= OUT_TOL
    assert np.array_equal(codes[~fl], case["codes0"][~fl])


# measured on MI355X with these seeds (state drift mean / at step 4096 /
# output drift max): L=4 0.0380 / 0.0356 / 0.0442, L=16 0.0169 / 0.0102 /
# 0.0281, L=64 0.0064 / 0.00088 / 0.0261; the bounds sit ~25% above
DRIFT_BOUNDS = {
    # L: (state drift mean, state drift at 4096, output drift max)
    4: (0.048, 0.045, 0.055),
    16: (0.021, 0.013, 0.035),
    64: (0.008, 0.0011, 0.033),
}


@pytest.mark.parametrize("window", [4, 16, 64])
def test_long_sequence_drift(device, window):
    """Config 3 in the reference regime (B=8, 4096 steps, fresh inputs every
    step): the reference's drift metric (the state replayed from the device's
    checkpoint over the ring, against the exact fp32 recurrence on the same
    ring values, every step; gdn_replayssm_drift) stays near the levels
    measured here and does not grow from step 512 to 4096 (measured
    1.00 .. 1.07). Under these synthetic gates the state forgets the
    checkpoint within a few rings, so the error each flush injects decays
    instead of accumulating as the sqrt(flushes) law the reference found on
    Qwen3.5's long-memory heads (REPORT.md:294-311, which would give
    sqrt(4096 / 512) = 2.8)."""
    from gdn_replayssm_drift import drift_study

    d = drift_study(window, device, steps=4096, batch=8, regime="reference", seed=700 + window)
    print(f"drift L={window}: " + ", ".join(f"{k} {v:.4g}" for k, v in d.items() if isinstance(v, float)))
    mean_max, last_max, out_max = DRIFT_BOUNDS[window]
    assert d["state_drift_mean"] < mean_max, d
    assert d["state_drift_at_4096"] < last_max, d
    assert d["output_drift_max"] < out_max, d
    assert d["growth_512_to_last"] < 1.25, d
