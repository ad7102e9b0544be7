"""Shared helpers of the GPU parity tests: build device inputs with the
synthetic generator and hand the same values to the CPU oracle."""

from __future__ import annotations

import numpy as np
import torch

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth
from oracle import fp8_quant, gdn_oracle

STORAGE = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def codes_np(payload: torch.Tensor) -> np.ndarray:
    return payload.detach().view(torch.uint8).cpu().numpy()


def make_replay_case(batch, ring_len, device, seed=0, heads=16, value_heads=32, dtype=torch.bfloat16,
                     warmup=32, valid=None, flush=None, reference_dist=False, value_dim=128):
    """Checkpoint (device-quantised), ring, q, valid_len, flush for one replay
    call. reference_dist: the reference's own input regime (A_log ~ U(0,1),
    dt_bias ~ U(-4,-3): gamma ~ 0.95 per token; state 0.02 N(0,1);
    prototype/gdn_replayssm_fp8_kernel.py:1238-1289) instead of BASELINE's."""
    shape = synth.Shape(batch, heads, value_heads, value_dim=value_dim)
    gen = synth.generator(seed, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device, reference_dist=reference_dist)
    state = synth.warm_state(shape, warmup, gen, device, a_log, dt_bias, reference_dist=reference_dist)
    ckpt = gk.quantize_checkpoint(state)
    q, k, v, g, beta = synth.ring_inputs(shape, ring_len, gen, device, a_log, dt_bias, dtype)
    if valid is None:
        valid = torch.randint(1, ring_len + 1, (batch,), generator=gen, device=device, dtype=torch.int32)
    else:
        valid = torch.as_tensor(valid, dtype=torch.int32, device=device)
    if flush is None:
        flush = torch.zeros(batch, dtype=torch.bool, device=device)
    else:
        flush = torch.as_tensor(flush, dtype=torch.bool, device=device)
    # host snapshot of the checkpoint as created: a flush rewrites ckpt in place
    codes0 = codes_np(ckpt.payload).copy()
    scale0 = ckpt.scale.cpu().numpy().copy()
    return dict(state=state, ckpt=ckpt, codes0=codes0, scale0=scale0, q=q, k=k, v=v, g=g, beta=beta, valid=valid,
                flush=flush)


def oracle_replay(case, dtype=np.float64):
    """Oracle output (float) and new codes/scale for a replay call on `case`,
    started from the checkpoint as it was when the case was made."""
    return gdn_oracle.replay_step(case["codes0"], case["scale0"],
                                  np32(case["q"]), np32(case["k"]), np32(case["v"]), np32(case["g"]),
                                  np32(case["beta"]), case["valid"].cpu().numpy(), case["flush"].cpu().numpy(),
                                  dtype)


def run_replay(case, block_v=128, out=None):
    return gk.gdn_replay_fp8(case["ckpt"].payload, case["ckpt"].scale, case["q"], case["k"], case["v"],
                             case["g"], case["beta"], case["valid"], case["flush"], block_v=block_v, out=out)


def c_quantize(state: torch.Tensor):
    codes, scale, sat = fp8_quant.quantize_vblock32(np32(state))
    return codes, scale, sat
