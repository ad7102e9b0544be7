"""GPU parity of the HIP path against the CPU oracle (marked `gpu`).

Gates (tolerances written here, from the measurement plan of this build):
  (1) full-precision replay vs the per-token recurrence: rel-L2 <= 1e-6
      (f32 activations, exact checkpoint);
  (2) checkpoint codes and scales bit-exact vs the reference quantiser
      (ref:36-37,40-106) given the identical fp32 state;
  (3) replay output rel-L2 <= 2e-3 vs the fp32/fp64 oracle started from the
      same dequantised checkpoint (bf16 output rounding floor ~1.7e-3).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth
from conftest import rel_l2
from gpu_helpers import c_quantize, codes_np, make_replay_case, np32, oracle_replay, run_replay
from oracle import gdn_oracle

pytestmark = pytest.mark.gpu

OUT_TOL = 2e-3


def test_fp8_decode_all_codes(device):
    """Every e4m3fn code decodes on the device to the OCP value (scale 1)."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).repeat(32 * 128 // 256)
    payload = codes.view(1, 1, 32, 128).to(device).view(torch.float8_e4m3fn)
    scale = torch.ones(1, 1, 1, dtype=torch.float16, device=device)
    ck = gk.QuantizedCheckpoint(payload, scale, "vblock", 32, 0.0)
    got = np32(gk.dequantize_checkpoint(ck)).ravel()
    want = gdn_oracle.e4m3fn_decode(codes.numpy())
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _edge_state(device):
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(2, 4, 128, 128, generator=gen) * 0.02
    x[0, 0, :32] = 0.0                                 # amax == 0 -> scale 1, codes 0
    x[0, 0, 32:64] = 3e-6 * torch.randn(32, 128, generator=gen)   # fp16 scale underflows
    x[0, 1, :32] = -0.0                                # negative zeros
    x[0, 1, 32:64, 5] = 1.0                            # power-of-two amax, rest zero
    x[0, 2, :32] = torch.linspace(-448, 448, 32 * 128).view(32, 128)  # scale exactly 1
    x[1, 0, :32] *= 1e4                                # large magnitudes
    x[1, 1, :32] = torch.randint(-2000, 2000, (32, 128), generator=gen).float() / 256.0  # many ties
    x[1, 2, 64:96] = 1e-30 * torch.randn(32, 128, generator=gen)  # subnormal fp32 scale
    x[1, 3, :32] = _near_midpoint_block(gen)           # quotients within a few ulp of fp8 midpoints
    nan_block = torch.full((32, 128), 0.25)            # NaN amax: scale 1, NaN codes keep their sign
    nan_block[4, 4], nan_block[5, 5], nan_block[0, 1] = float("nan"), -float("nan"), 1000.0
    x[1, 3, 32:64] = nan_block
    x[1, 3, 64:96] = 1e-25 * torch.randn(32, 128, generator=gen)  # scale below 2^-64: division path
    x[0, 3, :32] = torch.arange(-2048, 2048).float().view(32, 128) * 2.0 ** -11  # fp8 subnormal ties
    x[0, 3, 0, 0] = 448.0                              # (scale exactly 1)
    return x.to(device)


def _near_midpoint_block(gen):
    """A 32 x 128 block whose quotients x / s land within +-3 fp32 ulp of
    e4m3fn rounding midpoints (and a few on fp8 values), s = amax / 448 with
    a non-power-of-two amax: the quotients the fast quantiser path must round
    exactly as the division does."""
    amax = np.float32(1.2345)
    s = np.float32(amax / np.float32(448.0))
    exps = torch.randint(-6, 9, (32 * 128,), generator=gen).numpy()
    mant = torch.randint(0, 8, (32 * 128,), generator=gen).numpy()
    mid = (1.0 + (2 * mant + 1) / 16.0) * np.exp2(exps.astype(np.float64))  # midpoints of the fp8 grid
    mid = np.minimum(mid, 440.0)
    ulps = torch.randint(-3, 4, (32 * 128,), generator=gen).numpy()
    q = mid * (1.0 + ulps * 2.0 ** -23)
    sign = np.where(torch.rand(32 * 128, generator=gen).numpy() < 0.5, -1.0, 1.0)
    x = np.float32(sign * q * np.float64(s))
    x = np.clip(x, -amax, amax)
    x[0] = amax
    return torch.from_numpy(x.reshape(32, 128).astype(np.float32))


@pytest.mark.parametrize("kind", ["random", "edge"])
def test_quantizer_bit_exact(device, kind):
    """Gate (2): device quantiser == C restatement of the reference quantiser."""
    if kind == "random":
        shape = synth.Shape(3)
        gen = synth.generator(1, device)
        a_log, dt_bias = synth.gating_params(shape, gen, device)
        state = synth.warm_state(shape, 64, gen, device, a_log, dt_bias)
    else:
        state = _edge_state(device)
    ck = gk.quantize_checkpoint(state)
    codes, scale, sat = c_quantize(state)
    assert np.array_equal(ck.scale.cpu().numpy().view(np.uint16), scale.view(np.uint16))
    got = codes_np(ck.payload)
    assert np.array_equal(got, codes)
    assert ck.saturation_fraction == pytest.approx(sat.sum() / state.numel())
    # and the numpy restatement agrees with both
    nq = gdn_oracle.quantize_checkpoint(np32(state), "vblock", 32)
    assert np.array_equal(nq.payload, got)


@pytest.mark.parametrize("block_v", [32, 64, 128])
def test_replay_matches_oracle(device, block_v):
    """Gate (3), mixed ring fills (0..L) including empty and full rings."""
    case = make_replay_case(6, 16, device, seed=3, valid=[0, 1, 5, 9, 15, 16])
    out = run_replay(case, block_v=block_v)
    ref, _, _ = oracle_replay(case)
    err = rel_l2(np32(out), ref)
    assert err <= OUT_TOL, err
    # bf16 rounding is the only loss: compare with the rounded oracle too
    assert rel_l2(np32(out), gdn_oracle.bf16_round(ref.astype(np.float32))) < 2e-4


def test_replay_block_v_and_split_identical(device):
    """The tilings (one decode kernel) give bit-identical outputs, and so do
    the two precompute variants of the two-launch split; the split (T_0 in
    f32, then S_0 T_0) and the one-launch decode (S_0 X_t for the 16 X rows,
    weighted by the chain's alpha) sum in different orders and differ by at
    most one bf16 ulp."""
    case = make_replay_case(4, 8, device, seed=4)
    outs = [run_replay(case, block_v=bv) for bv in (32, 64, 128)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    B, L = 4, 8
    tq = torch.empty(B, 32, 128, dtype=torch.float32, device=device)
    coef = torch.zeros(B, 32, L, dtype=torch.float32, device=device)
    split = []
    for grouped in (True, False):
        split.append(gk.gdn_replay_fp8_split(case["ckpt"].payload, case["ckpt"].scale, case["q"], case["k"],
                                             case["v"], case["g"], case["beta"], case["valid"], tq, coef,
                                             block_v=128, precompute_grouped=grouped))
    assert torch.equal(split[1], split[0])
    fused, two = np32(outs[0]).ravel(), np32(split[0]).ravel()
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(two), 1e-30))) - 7)  # bf16 spacing at |two|
    assert np.all(np.abs(fused - two) <= ulp), np.max(np.abs(fused - two) / ulp)
    assert np.mean(fused != two) < 0.01
    _, tq_ref, coef_ref = gdn_oracle.adjoint_replay(
        gdn_oracle.dequantize_vblock32(codes_np(case["ckpt"].payload), case["ckpt"].scale.cpu().numpy()),
        np32(case["q"]), np32(case["k"]), np32(case["v"]), np32(case["g"]), np32(case["beta"]),
        case["valid"].cpu().numpy(), np.float64)
    assert rel_l2(np32(tq), tq_ref) < 1e-5
    assert rel_l2(np32(coef), coef_ref) < 1e-5


def test_replay_full_size_config1(device):
    """Config 1 as defined: B=64, Qwen3.5-4B layer, L=16, fills uniform in
    1..16, the sequences at fill 16 flushing in the same launch (rebuild,
    emit from the rebuilt state, requantise in place)."""
    gen = torch.Generator(device="cpu").manual_seed(1)
    valid = torch.randint(1, 17, (64,), generator=gen, dtype=torch.int32)
    valid[:4] = 16  # at least four flushing sequences
    case = make_replay_case(64, 16, device, seed=0, warmup=256, valid=valid, flush=valid == 16)
    out = run_replay(case, block_v=128)
    ref, ref_codes, ref_scale = oracle_replay(case, np.float32)
    err = rel_l2(np32(out), ref)
    assert err <= OUT_TOL, err
    fl = (valid == 16).numpy()
    codes = codes_np(case["ckpt"].payload)
    assert np.mean(codes[fl] != ref_codes[fl]) < 1e-3
    assert np.array_equal(codes[~fl], case["codes0"][~fl])  # replays leave their checkpoints alone
    # scales: the flushing sequences' within one fp16 ulp of the oracle's
    # (the rebuilt amax may round to the neighbouring fp16 value), rarely
    # off; the replaying sequences' untouched
    got_s = case["ckpt"].scale.cpu().numpy()
    ulps = np.abs(got_s[fl].view(np.uint16).astype(np.int64)
                  - ref_scale[fl].astype(np.float16).view(np.uint16).astype(np.int64))
    assert ulps.max() <= 1 and ulps.mean() < 0.01, (ulps.max(), ulps.mean())
    assert np.array_equal(got_s[~fl].view(np.uint16), case["scale0"][~fl].view(np.uint16))


@pytest.mark.parametrize("ring_len,block_v", [(4, 32), (16, 128), (64, 64)])
def test_flush_matches_oracle(device, ring_len, block_v):
    """Flush: output from the rebuilt fp32 state, then in-place requantisation.
    Codes equal the oracle's except where fp32 summation order moves a value
    across a rounding boundary (then by one code)."""
    batch = 4
    case = make_replay_case(batch, ring_len, device, seed=5, valid=[ring_len, ring_len - 1, 1, 0][:batch],
                            flush=[1, 1, 1, 0])
    before = codes_np(case["ckpt"].payload).copy()
    out = run_replay(case, block_v=block_v)
    ref_out, ref_codes, ref_scale = oracle_replay(case)
    assert rel_l2(np32(out), ref_out) <= OUT_TOL
    got = codes_np(case["ckpt"].payload)
    assert np.array_equal(got[3], before[3])           # flush == 0 leaves the checkpoint alone
    mismatch = np.mean(got != ref_codes)
    assert mismatch < 1e-3, mismatch
    deq = gdn_oracle.dequantize_vblock32(got, case["ckpt"].scale.cpu().numpy())
    deq_ref = gdn_oracle.dequantize_vblock32(ref_codes, ref_scale)
    assert rel_l2(deq, deq_ref) < 2e-3
    assert np.mean(case["ckpt"].scale.cpu().numpy() != ref_scale) < 0.02


@pytest.mark.parametrize("ring_len,block_v", [(4, 32), (16, 64), (64, 128)])
def test_flush_output_equals_replay_output(device, ring_len, block_v):
    """Invariant: the adjoint replay (flush = 0) and the forward rebuild
    (flush = 1) compute the same o = S q from the same checkpoint and ring, for
    every ring fill 0..L; only fp32 summation order differs."""
    valid = sorted(set([0, 1, 2, ring_len // 2, ring_len - 1, ring_len]))
    case = make_replay_case(len(valid), ring_len, device, seed=8, valid=valid, flush=[0] * len(valid))
    replay_out = np32(run_replay(case, block_v=block_v))
    case["flush"] = torch.ones(len(valid), dtype=torch.bool, device=device)
    flush_out = np32(run_replay(case, block_v=block_v))
    for i in range(len(valid)):
        assert rel_l2(flush_out[i], replay_out[i]) < 2e-3, (valid[i], rel_l2(flush_out[i], replay_out[i]))


@pytest.mark.parametrize("act", [torch.float16, torch.float32])
def test_replay_other_dtypes(device, act):
    case = make_replay_case(3, 8, device, seed=6, dtype=act)
    out = run_replay(case, block_v=64)
    assert out.dtype == act
    ref, _, _ = oracle_replay(case)
    assert rel_l2(np32(out), ref) <= (OUT_TOL if act == torch.float16 else 1e-5)


def test_full_precision_replay_vs_recurrence(device):
    """Gate (1) on the device: f32 activations and an exact (zero) checkpoint,
    so the adjoint replay must equal the per-token recurrence to 1e-6."""
    shape = synth.Shape(2, 4, 4)
    gen = synth.generator(11, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    L = 4
    q, k, v, g, beta = synth.token_inputs(shape, L, gen, device, a_log, dt_bias)
    zero = torch.zeros(2, 4, 128, 128, device=device)
    ck = gk.quantize_checkpoint(zero)
    flush = torch.zeros(2, dtype=torch.bool, device=device)
    for fill in range(1, L + 1):
        valid = torch.full((2,), fill, dtype=torch.int32, device=device)
        out = gk.gdn_replay_fp8(ck.payload, ck.scale, q[:, fill - 1].contiguous(), k, v, g, beta, valid, flush,
                                block_v=32)
        qs = np.repeat(np32(q)[:, fill - 1:fill], fill, axis=1)
        ref, _ = gdn_oracle.baseline_decode(np.zeros((2, 4, 128, 128)), qs, np32(k)[:, :fill], np32(v)[:, :fill],
                                            np32(g)[:, :fill], np32(beta)[:, :fill], np.float64)
        assert rel_l2(np32(out), ref[:, -1]) <= 1e-6


def test_prep_matches_oracle(device):
    shape = synth.Shape(8)
    gen = synth.generator(12, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    mixed, a, b = synth.raw_step_inputs(shape, 1, gen, device)
    mixed, a, b = mixed[:, 0].contiguous(), a[:, 0].contiguous(), b[:, 0].contiguous()
    L = 4
    pos = torch.tensor([0, 1, 2, 3, 3, 2, 1, 0], dtype=torch.int32, device=device)
    q_out = torch.zeros(8, 16, 128, dtype=torch.bfloat16, device=device)
    rings = [torch.zeros(8, L, 16, 128, dtype=torch.bfloat16, device=device),
             torch.zeros(8, L, 32, 128, dtype=torch.bfloat16, device=device),
             torch.zeros(8, L, 32, dtype=torch.bfloat16, device=device),
             torch.zeros(8, L, 32, dtype=torch.bfloat16, device=device)]
    gk.gdn_prep_ring(mixed, a, b, a_log, dt_bias, pos, q_out, *rings)
    oq = np.zeros((8, 16, 128), np.float32)
    orings = [np.zeros(r.shape, np.float32) for r in rings]
    gdn_oracle.prep_ring(np32(mixed), np32(a), np32(b), np32(a_log), np32(dt_bias), pos.cpu().numpy(), oq, *orings)
    for got, want in zip([q_out, *rings], [oq, *orings]):
        got = np32(got)
        # fp32 math vs the float64 formula: equal after bf16 rounding except near ties (one bf16 ulp)
        ulp = np.abs(want) * 2.0 ** -7 + 1e-30
        assert np.all(np.abs(got - want) <= ulp)
        assert np.mean(got != want) < 0.01


@pytest.mark.parametrize("gate_dtype", [torch.bfloat16, torch.float32])
def test_fused_step_equals_prep_then_replay(device, gate_dtype):
    """gdn_prep_replay_fp8 == gdn_prep_ring + gdn_replay_fp8, bit for bit,
    on buffers that also receive identical ring appends."""
    shape = synth.Shape(5)
    L = 8
    gen = synth.generator(13, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 16, gen, device, a_log, dt_bias)
    mixed, a, b = synth.raw_step_inputs(shape, 1, gen, device, gate_dtype=gate_dtype)
    mixed, a, b = mixed[:, 0].contiguous(), a[:, 0].contiguous(), b[:, 0].contiguous()
    _, k, v, g, beta = synth.ring_inputs(shape, L, gen, device, a_log, dt_bias)
    pos = torch.tensor([0, 3, 7, 5, 2], dtype=torch.int32, device=device)
    valid = pos + 1
    valid[3] = 3   # new token outside the replayed prefix
    flush = torch.tensor([0, 0, 1, 0, 1], dtype=torch.bool, device=device)
    results = []
    for fused in (False, True):
        ck = gk.quantize_checkpoint(state)
        q_out = torch.zeros(5, 16, 128, dtype=torch.bfloat16, device=device)
        rk, rv, rg, rb = k.clone(), v.clone(), g.clone(), beta.clone()
        if fused:
            out = gk.gdn_prep_replay_fp8(mixed, a, b, a_log, dt_bias, pos, ck.payload, ck.scale, q_out, rk, rv, rg,
                                         rb, valid, flush, block_v=128)
        else:
            gk.gdn_prep_ring(mixed, a, b, a_log, dt_bias, pos, q_out, rk, rv, rg, rb)
            out = gk.gdn_replay_fp8(ck.payload, ck.scale, q_out, rk, rv, rg, rb, valid, flush, block_v=128)
        results.append([out, q_out, rk, rv, rg, rb, ck.payload.view(torch.uint8), ck.scale])
    for x, y in zip(*results):
        assert torch.equal(x, y)


def test_cycle_matches_oracle(device):
    """Config 2 semantics over two whole ring cycles (L=4) with mixed ring
    phases: prep + replay every step, flush + requantise at the ring end."""
    shape = synth.Shape(4)
    L, steps = 4, 9
    gen = synth.generator(14, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 64, gen, device, a_log, dt_bias)
    mixed, a, b = synth.raw_step_inputs(shape, steps, gen, device)
    phase = np.array([0, 1, 2, 3])
    ck = gk.quantize_checkpoint(state)
    codes0, scale0 = codes_np(ck.payload).copy(), ck.scale.cpu().numpy().copy()
    q_out = torch.zeros(4, 16, 128, dtype=torch.bfloat16, device=device)
    rings = [torch.zeros(4, L, 16, 128, dtype=torch.bfloat16, device=device),
             torch.zeros(4, L, 32, 128, dtype=torch.bfloat16, device=device),
             torch.zeros(4, L, 32, dtype=torch.bfloat16, device=device),
             torch.zeros(4, L, 32, dtype=torch.bfloat16, device=device)]
    outs = []
    for step in range(steps):
        fill = torch.as_tensor((phase + step) % L + 1, dtype=torch.int32, device=device)
        outs.append(np32(gk.gdn_prep_replay_fp8(mixed[:, step].contiguous(), a[:, step].contiguous(),
                                                b[:, step].contiguous(), a_log, dt_bias, fill - 1, ck.payload,
                                                ck.scale, q_out, *rings, fill, fill == L)))
    ref, ref_codes, _ = gdn_oracle.full_contract_decode(codes0, scale0, np32(mixed), np32(a), np32(b), np32(a_log),
                                                        np32(dt_bias), L, 16, 128, 32, 128, phase=phase,
                                                        dtype=np.float64)
    got = np.stack(outs, axis=1)
    assert rel_l2(got, ref) <= OUT_TOL
    assert np.mean(codes_np(ck.payload) != ref_codes) < 1e-3


@pytest.mark.parametrize("block_v", [32, 64, 128])
def test_strided_views_equal_contiguous(device, block_v):
    """Outer strides are free, as in the reference's wrappers: a checkpoint
    whose rows sit 192 bytes apart (a view of a padded buffer), scales and
    rings that are slices of larger buffers give bit-identical outputs and
    requantised checkpoints to contiguous copies, and the padding is never
    written. Fills 1..16 plus two flushes (L=16)."""
    B, L = 8, 16
    valid = [1, 4, 7, 9, 12, 15, 16, 16]
    flush = [False] * 6 + [True, True]
    case = make_replay_case(B, L, device, seed=21, valid=valid, flush=flush)
    ck = case["ckpt"]
    pad_payload = torch.full((B, 32, 128, 192), 0x55, dtype=torch.uint8, device=device)
    pay_view = pad_payload[..., :128].view(torch.float8_e4m3fn)
    pay_view.copy_(ck.payload)
    pad_scale = torch.zeros(B, 32, 8, dtype=torch.float16, device=device)
    sc_view = pad_scale[..., :4]
    sc_view.copy_(ck.scale)

    def ring_view(x):
        big = torch.zeros(x.shape[0], 2 * L, *x.shape[2:], dtype=x.dtype, device=device)
        big[:, :L].copy_(x)
        return big[:, :L]

    k, v, g, beta = (ring_view(case[n]) for n in ("k", "v", "g", "beta"))
    out_view = gk.gdn_replay_fp8(pay_view, sc_view, case["q"], k, v, g, beta, case["valid"], case["flush"],
                                 block_v=block_v)
    payload_c, scale_c = ck.payload.clone(), ck.scale.clone()
    out_c = gk.gdn_replay_fp8(payload_c, scale_c, case["q"], case["k"], case["v"], case["g"], case["beta"],
                              case["valid"], case["flush"], block_v=block_v)
    assert torch.equal(out_view, out_c)
    assert torch.equal(pay_view.view(torch.uint8), payload_c.view(torch.uint8))
    assert torch.equal(sc_view, scale_c)
    assert bool((pad_payload[..., 128:] == 0x55).all())
    assert bool((pad_scale[..., 4:] == 0).all())
