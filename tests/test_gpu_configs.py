"""GPU parity of the full-contract path on the remaining BASELINE configs
(marked `gpu`): the batch x ring-length sweep, the long-sequence drift run
and the large-batch stacked-layer stress.

Sequences are independent, so each large run is checked against the fp64
oracle on a few sampled sequences (the oracle restates the reference's
replay semantics, prototype/gdn_replay_fp8_reference.py:189-244, and the
full-contract cycle, prototype/bench_gdn_full_contract.py:225-308).
Tolerances: output rel-L2 <= 2e-3 vs the oracle started from the same
checkpoint; requantised codes equal up to rounding-boundary flips (< 1e-3 of
the codes); the drift run is measured against an exact fp32 recurrence.
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


def _rings(batch, window, dtype, device, shape):
    return [torch.zeros(batch, window, shape.heads, shape.key_dim, dtype=dtype, device=device),
            torch.zeros(batch, window, shape.value_heads, shape.value_dim, dtype=dtype, device=device),
            torch.zeros(batch, window, shape.value_heads, dtype=dtype, device=device),
            torch.zeros(batch, window, shape.value_heads, dtype=dtype, device=device)]


def _run_cycle(ck, mixed, a, b, a_log, dt_bias, window, phase, steps, block_v, device):
    """Full-contract steps (one fused launch each), ring fill ((phase + s) % L) + 1,
    flush at fill L; returns outputs [B, steps, HV, V] as float32 numpy."""
    batch = mixed.shape[0]
    shape = synth.Shape(batch)
    q_out = torch.zeros(batch, shape.heads, shape.key_dim, dtype=mixed.dtype, device=device)
    rings = _rings(batch, window, mixed.dtype, device, shape)
    phase_t = torch.as_tensor(phase, dtype=torch.int32, device=device)
    outs = []
    for step in range(steps):
        fill = (phase_t + step) % window + 1
        outs.append(gk.gdn_prep_replay_fp8(mixed[:, step], a[:, step], b[:, step], a_log, dt_bias, fill - 1,
                                           ck.payload, ck.scale, q_out, *rings, fill, fill == window,
                                           block_v=block_v))
    return np32(torch.stack(outs, dim=1))


def _oracle_on(idx, codes0, scale0, mixed, a, b, a_log, dt_bias, window, phase):
    """fp64 oracle of the cycle for the sequences in idx."""
    shape = synth.Shape(1)
    return gdn_oracle.full_contract_decode(codes0[idx], scale0[idx], np32(mixed[idx]), np32(a[idx]), np32(b[idx]),
                                           np32(a_log), np32(dt_bias), window, shape.heads, shape.key_dim,
                                           shape.value_heads, shape.value_dim, phase=phase[idx], dtype=np.float64)


@pytest.mark.parametrize("window", [4, 8, 16])
@pytest.mark.parametrize("batch", [8, 16, 32, 64])
def test_full_contract_sweep(device, batch, window):
    """Config 2: batch in {8, 16, 32, 64} x L in {4, 8, 16}, steady-state ring
    phases (fills spread over 1..L), a little over one ring cycle so every
    sequence flushes once; sampled sequences against the oracle."""
    shape = synth.Shape(batch)
    gen = synth.generator(1000 + 10 * batch + window, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 32, gen, device, a_log, dt_bias)
    steps = window + 2
    mixed, a, b = synth.raw_step_inputs(shape, steps, gen, device)
    phase = np.arange(batch) % window
    ck = gk.quantize_checkpoint(state)
    codes0, scale0 = codes_np(ck.payload).copy(), ck.scale.cpu().numpy().copy()
    got = _run_cycle(ck, mixed, a, b, a_log, dt_bias, window, phase, steps, 128, device)
    idx = np.array(sorted({0, batch // 2 + 1, batch - 1}))
    ref, ref_codes, ref_scale = _oracle_on(idx, codes0, scale0, mixed, a, b, a_log, dt_bias, window, phase)
    assert rel_l2(got[idx], ref) <= OUT_TOL
    assert np.mean(codes_np(ck.payload)[idx] != ref_codes) < CODE_FLIP_TOL
    # scales: the rebuilt amax may round to the neighbouring fp16 value
    got_s = ck.scale.cpu().numpy()[idx].astype(np.float16).view(np.uint16).astype(np.int64)
    ref_s = np.asarray(ref_scale, dtype=np.float16).view(np.uint16).astype(np.int64)
    assert np.abs(got_s - ref_s).max() <= 1


DRIFT_MAX = 0.035   # measured 0.0263-0.0265 at every probe, L = 4, 16 and 64
OUT_DRIFT_MAX = 3e-3  # measured 1.69e-3 - 1.92e-3 against the exact fp32 recurrence


@pytest.mark.parametrize("window", [4, 16, 64])
def test_long_sequence_drift(device, window):
    """Config 3: batch 8, 4096 consecutive full-contract steps with fresh
    seeded inputs, L in {4, 16, 64}.

    Alongside, an exact fp32 recurrence (S <- e^g S; S += beta (v - S k) k^T,
    ref:155-161) consumes the same ring values the kernel appended. After the
    flushes at steps 128, 512, 2048 and 4096 the checkpoint is the whole
    state: its relative drift from the fp32 state must stay at the
    one-quantisation level (the e4m3 step is 2^-3 relative; the decay forgets
    older errors), and must not grow with the number of flushes. The fp32
    recurrence itself is pinned to the oracle's run_kernel (ref:137-163) on
    sequence 0 over the first 128 steps, and sequence 0's outputs and
    checkpoint after 128 steps to the oracle's own full-contract cycle (its
    prep from the raw inputs, replays, flushes and requantisation)."""
    shape = synth.Shape(8)
    steps = 4096
    gen = synth.generator(77 + window, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    mixed, a, b = synth.raw_step_inputs(shape, steps, gen, device)
    state = torch.zeros(8, shape.value_heads, shape.value_dim, shape.key_dim, device=device)
    ck = gk.quantize_checkpoint(state)
    codes0, scale0 = codes_np(ck.payload).copy(), ck.scale.cpu().numpy().copy()
    q_out = torch.zeros(8, shape.heads, shape.key_dim, dtype=torch.bfloat16, device=device)
    k_ring, v_ring, g_ring, b_ring = _rings(8, window, torch.bfloat16, device, shape)
    exact = state.clone()
    G = shape.group
    drift, out_err = {}, []
    pin = 128
    seq0 = {"q": [], "k": [], "v": [], "g": [], "beta": [], "out": []}
    for step in range(steps):
        fill = torch.full((8,), step % window + 1, dtype=torch.int32, device=device)
        out = gk.gdn_prep_replay_fp8(mixed[:, step], a[:, step], b[:, step], a_log, dt_bias, fill - 1, ck.payload,
                                     ck.scale, q_out, k_ring, v_ring, g_ring, b_ring, fill, fill == window)
        pos = step % window
        if step < pin:
            for key, t in (("q", q_out), ("k", k_ring[:, pos]), ("v", v_ring[:, pos]), ("g", g_ring[:, pos]),
                           ("beta", b_ring[:, pos]), ("out", out)):
                seq0[key].append(np32(t[0]))
        q = q_out.float().repeat_interleave(G, dim=1)
        k = k_ring[:, pos].float().repeat_interleave(G, dim=1)
        exact.mul_(g_ring[:, pos].float().exp()[..., None, None])
        r = (exact * k[:, :, None, :]).sum(-1)
        exact.add_(((v_ring[:, pos].float() - r) * b_ring[:, pos].float()[..., None])[..., None] * k[:, :, None, :])
        o_exact = (exact * q[:, :, None, :]).sum(-1) * shape.key_dim ** -0.5
        if step % 64 == 63:
            out_err.append(rel_l2(np32(out), np32(o_exact)))
        if step + 1 == pin:
            exact_pin, codes_pin = np32(exact[0]), codes_np(ck.payload)[0].copy()
        if step + 1 in (128, 512, 2048, 4096):
            got = gk.dequantize_checkpoint(ck)
            drift[step + 1] = rel_l2(np32(got), np32(exact))
    print(f"L={window}: state drift {drift}, output error max {max(out_err):.3e}")
    assert all(d < DRIFT_MAX for d in drift.values()), drift
    assert drift[4096] < 1.15 * drift[128], drift
    assert max(out_err) < OUT_DRIFT_MAX, max(out_err)
    # the fp32 recurrence of this test against the oracle's (fp64), sequence 0
    stack = {key: np.stack(vals)[None] for key, vals in seq0.items()}
    _, ref_state = gdn_oracle.run_kernel(np.zeros((1,) + exact_pin.shape), stack["q"], stack["k"], stack["v"],
                                         stack["g"], stack["beta"], np.float64)
    assert rel_l2(exact_pin, ref_state[0]) < 1e-5
    # sequence 0 against the oracle's full-contract cycle from the raw inputs
    ref_out, ref_codes, _ = gdn_oracle.full_contract_decode(
        codes0[:1], scale0[:1], np32(mixed[:1, :pin]), np32(a[:1, :pin]), np32(b[:1, :pin]), np32(a_log),
        np32(dt_bias), window, shape.heads, shape.key_dim, shape.value_heads, shape.value_dim, dtype=np.float64)
    assert rel_l2(stack["out"], ref_out) <= OUT_TOL
    assert np.mean(codes_pin != ref_codes[0]) < CODE_FLIP_TOL


@pytest.mark.parametrize("block_v", [32, 64, 128])
def test_large_batch_stacked_layers(device, block_v):
    """Config 4: batch 512, 24 stacked GDN layers (independent seeded inputs
    per layer), L=8, one whole ring cycle per layer back to back; every
    layer's checkpoint and rings stay resident. Sampled (layer, sequence)
    pairs are checked against the oracle; the results for each layer are the
    same for every block_v (a hash of outputs and codes per layer)."""
    layers, batch, window = 24, 512, 8
    shape = synth.Shape(batch)
    phase = np.arange(batch) % window
    digests = []
    checked = {3: [0, 257], 17: [511]}
    for layer in range(layers):
        gen = synth.generator(5000 + layer, device)
        a_log, dt_bias = synth.gating_params(shape, gen, device)
        state = synth.warm_state(shape, 8, gen, device, a_log, dt_bias)
        ck = gk.quantize_checkpoint(state)
        del state
        codes0, scale0 = (codes_np(ck.payload).copy(), ck.scale.cpu().numpy().copy()) if layer in checked else (None,
                                                                                                               None)
        mixed, a, b = synth.raw_step_inputs(shape, window, gen, device)
        got = _run_cycle(ck, mixed, a, b, a_log, dt_bias, window, phase, window, block_v, device)
        digests.append((float(np.abs(got).sum()), int(ck.payload.view(torch.uint8).sum().item())))
        if layer in checked:
            idx = np.array(checked[layer])
            ref, ref_codes, _ = _oracle_on(idx, codes0, scale0, mixed, a, b, a_log, dt_bias, window, phase)
            assert rel_l2(got[idx], ref) <= OUT_TOL
            assert np.mean(codes_np(ck.payload)[idx] != ref_codes) < CODE_FLIP_TOL
        del ck, mixed, a, b
    key = "stacked_layer_digests"
    store = test_large_batch_stacked_layers.__dict__.setdefault(key, {})
    store[block_v] = digests
    for other, ref_digests in store.items():
        assert ref_digests == digests, f"block_v={block_v} differs from block_v={other}"


def test_captured_inputs_drive_the_cycle(device, tmp_path):
    """Real-trace mode (gdn_replayssm_capture, the capture format of
    prototype/qwen35_capture_raw.py:100-130 as read by
    bench_gdn_full_contract.py:83-110): a batch-1 record of one layer,
    written and loaded back, replicated over 4 sequences, drives 10 steps of
    the L=4 cycle. Every sequence gives the same outputs; they match the fp64
    oracle of the cycle to rel-L2 <= 2e-3 and the record's production_out
    (stored in bf16, so two bf16 roundings apart) to 3e-3."""
    import gdn_replayssm_capture as cap

    T, L, batch = 10, 4, 4
    shape1 = synth.Shape(1)
    gen = synth.generator(71, device)
    a_log, dt_bias = synth.gating_params(shape1, gen, device)
    state = synth.warm_state(shape1, 32, gen, device, a_log, dt_bias)
    mixed, a, b = synth.raw_step_inputs(shape1, T, gen, device, gate_dtype=torch.float32)
    ck1 = gk.quantize_checkpoint(state)
    ref = gdn_oracle.full_contract_decode(codes_np(ck1.payload), ck1.scale.cpu().numpy(), np32(mixed), np32(a), np32(b),
                                          np32(a_log), np32(dt_bias), L, shape1.heads, shape1.key_dim,
                                          shape1.value_heads, shape1.value_dim, dtype=np.float64)[0][0]
    record = {
        "mixed_qkv": [mixed[:, t].cpu() for t in range(T)],
        "a": [a[:, t].cpu() for t in range(T)],
        "b": [b[:, t].cpu() for t in range(T)],
        "production_out": [torch.from_numpy(ref[t].reshape(1, -1)).to(torch.bfloat16) for t in range(T)],
        "state": state.cpu(),
        "a_log": a_log.cpu(),
        "dt_bias": dt_bias.cpu(),
        "scale": shape1.key_dim ** -0.5,
        "use_qk_l2norm_in_kernel": True,
    }
    path = tmp_path / "capture.pt"
    cap.save_capture(path, {5: record})
    inp = cap.captured_inputs(cap.load_capture(path), batch=batch, layer=5, steps=T, device=device)
    ck = gk.quantize_checkpoint(inp["state"])
    outs = _run_cycle(ck, inp["mixed_qkv"], inp["a"], inp["b"], inp["a_log"], inp["dt_bias"], L,
                      np.zeros(batch, dtype=np.int64), T, 128, device)
    prod = np32(inp["production_out"]).reshape(T, shape1.value_heads, shape1.value_dim)
    for bi in range(batch):
        assert np.array_equal(outs[bi], outs[0])
    assert rel_l2(outs[0], ref) <= OUT_TOL
    assert rel_l2(outs[0], prod) <= 3e-3
