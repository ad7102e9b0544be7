"""Long-sequence drift of the FP8 checkpoint.

The study the reference makes on captured Qwen3.5 inputs
(prototype/qwen35_drift_study.py:355-418), run here on the device path with
seeded synthetic inputs: `steps` consecutive full-contract decode steps
(gdn_prep_replay_fp8: prep, replay, flush and in-place requantisation at
fill L), beside an exact fp32 recurrence (S <- e^g S; S += beta (v - S k) k^T,
prototype/gdn_replay_fp8_reference.py:155-161) that consumes the same ring
values the device appended (q_out and the k, v, g, beta slots).

State drift follows the reference's definition: at every step, the state
reconstructed from the current checkpoint (the device's, dequantised) by an
fp32 replay of the ring tokens appended since it was written, against the
exact state -- at a flush step that is the rebuilt state before it is
requantised. Output drift is the step's output against the exact
recurrence's. The reference reports the drift at steps 64 .. 4096 (index
probe - 1), its mean over all steps and its growth from step 512 to the last
(:402-418); its finding is drift ~ 1% x sqrt(flushes) (REPORT.md:294-311), so
`per_flush` = mean drift / sqrt(flushes) is reported beside it.
"""

from __future__ import annotations

import math

import torch

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth


@torch.no_grad()
def drift_study(window: int, device, steps: int = 4096, batch: int = 8, regime: str = "reference", seed: int = 0,
                probes=(64, 128, 256, 512, 1024, 2048, 4096)) -> dict:
    """Run the study for one ring length. regime "reference": the reference's
    make_inputs gates (A_log ~ U(0,1), dt_bias ~ U(-4,-3)) and its 0.02 N(0,1)
    initial state (prototype/gdn_replayssm_fp8_kernel.py:1238-1289); regime
    "baseline": BASELINE's gates (A_log ~ U(0, ln 16), dt_bias = 0) from a
    zero state. Returns the drift summary (floats)."""
    if regime not in ("reference", "baseline"):
        raise ValueError(f"unknown regime {regime!r}")
    ref = regime == "reference"
    shape = synth.Shape(batch)
    HV, K, V, G = shape.value_heads, shape.key_dim, shape.value_dim, shape.group
    gen = synth.generator(seed, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device, reference_dist=ref)
    if ref:
        state0 = synth.warm_state(shape, 0, gen, device, a_log, dt_bias, reference_dist=True)
    else:
        state0 = torch.zeros(batch, HV, V, K, device=device)
    mixed, a_raw, b_raw = synth.raw_step_inputs(shape, steps, gen, device)
    bf = dict(dtype=torch.bfloat16, device=device)
    ck = gk.quantize_checkpoint(state0, saturation=False)
    q_out = torch.zeros(batch, shape.heads, K, **bf)
    k_r, v_r = torch.zeros(batch, window, shape.heads, K, **bf), torch.zeros(batch, window, HV, V, **bf)
    g_r, b_r = torch.zeros(batch, window, HV, **bf), torch.zeros(batch, window, HV, **bf)
    exact = state0.clone()
    recon = gk.dequantize_checkpoint(ck)
    out = torch.empty(batch, HV, V, **bf)
    state_err = torch.empty(steps, device=device, dtype=torch.float64)
    out_err = torch.empty(steps, device=device, dtype=torch.float64)
    scale = K ** -0.5

    def rel(a, b):
        return torch.linalg.vector_norm((a - b).double()) / torch.linalg.vector_norm(b.double()).clamp_min(1e-30)

    for step in range(steps):
        pos = step % window
        fill = torch.full((batch,), pos + 1, dtype=torch.int32, device=device)
        gk.gdn_prep_replay_fp8(mixed[:, step], a_raw[:, step], b_raw[:, step], a_log, dt_bias, fill - 1, ck.payload,
                               ck.scale, q_out, k_r, v_r, g_r, b_r, fill, fill == window, out=out)
        k = k_r[:, pos].float().repeat_interleave(G, dim=1)[:, :, None, :]
        decay = g_r[:, pos].float().exp()[..., None, None]
        beta = b_r[:, pos].float()[..., None]
        v = v_r[:, pos].float()
        for s in (exact, recon):
            s.mul_(decay)
            s.add_(((v - (s * k).sum(-1)) * beta)[..., None] * k)
        o_exact = (exact * q_out.float().repeat_interleave(G, dim=1)[:, :, None, :]).sum(-1) * scale
        state_err[step] = rel(recon, exact)
        out_err[step] = rel(out.float(), o_exact)
        if pos + 1 == window:
            recon = gk.dequantize_checkpoint(ck)  # the checkpoint the flush just wrote
    drift = state_err.cpu().tolist()
    odrift = out_err.cpu().tolist()
    flushes = steps // window
    mean = sum(drift) / steps
    res = {
        "regime": regime,
        "window": window,
        "steps": steps,
        "flushes": flushes,
        "state_drift_mean": mean,
        "state_drift_max": max(drift),
        "state_drift_last": drift[-1],
        "output_drift_mean": sum(odrift) / steps,
        "output_drift_max": max(odrift),
        "per_flush": mean / math.sqrt(flushes) if flushes else None,
        "growth_512_to_last": drift[-1] / drift[511] if steps > 512 and drift[511] else None,
    }
    for p in probes:
        if p - 1 < steps:
            res[f"state_drift_at_{p}"] = drift[p - 1]
    return res
