"""Seeded synthetic inputs for the ReplaySSM GDN decode path.

Distributions follow the measurement configs of this build (Qwen3.5-4B GDN
layer shape H=16, HV=32, K=V=128):
  q, k ~ N(0,1) then L2-normalised; v, a, b ~ N(0,1); A_log ~ U(0, ln 16);
  dt_bias = 0; g = -exp(A_log) softplus(a + dt_bias); beta = sigmoid(b);
  the recurrent state is produced by ``warmup`` recurrence steps from zero.
The reference's own benches use A_log ~ U(0,1), dt_bias ~ U(-4,-3) and a
0.02 N(0,1) state (prototype/gdn_replayssm_fp8_kernel.py:1238-1289);
``reference_dist=True`` selects those.

Everything is generated with torch on the requested device from one seeded
generator, so a (seed, device) pair always yields the same tensors.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

QWEN35_4B = dict(heads=16, value_heads=32, key_dim=128, value_dim=128)


@dataclass
class Shape:
    batch: int
    heads: int = 16
    value_heads: int = 32
    key_dim: int = 128
    value_dim: int = 128

    @property
    def group(self) -> int:
        return self.value_heads // self.heads

    @property
    def mixed_width(self) -> int:
        return 2 * self.heads * self.key_dim + self.value_heads * self.value_dim


def generator(seed: int, device) -> torch.Generator:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return gen


def gating_params(shape: Shape, gen: torch.Generator, device, reference_dist: bool = False):
    """A_log [HV] and dt_bias [HV], float32."""
    if reference_dist:
        a_log = torch.rand(shape.value_heads, generator=gen, device=device)
        dt_bias = torch.rand(shape.value_heads, generator=gen, device=device) - 4.0
    else:
        a_log = torch.rand(shape.value_heads, generator=gen, device=device) * math.log(16.0)
        dt_bias = torch.zeros(shape.value_heads, device=device)
    return a_log, dt_bias


def gate(a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor, dt_bias: torch.Tensor):
    """g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b) (float32)."""
    g = -a_log.float().exp() * F.softplus(a.float() + dt_bias.float())
    return g, torch.sigmoid(b.float())


def token_inputs(shape: Shape, steps: int, gen: torch.Generator, device, a_log, dt_bias):
    """Normalised per-token recurrence inputs, float32:
    q, k [B,T,H,K]; v [B,T,HV,V]; g, beta [B,T,HV]."""
    B, H, HV, K, V = shape.batch, shape.heads, shape.value_heads, shape.key_dim, shape.value_dim
    q = F.normalize(torch.randn(B, steps, H, K, generator=gen, device=device), dim=-1)
    k = F.normalize(torch.randn(B, steps, H, K, generator=gen, device=device), dim=-1)
    v = torch.randn(B, steps, HV, V, generator=gen, device=device)
    a = torch.randn(B, steps, HV, generator=gen, device=device)
    b = torch.randn(B, steps, HV, generator=gen, device=device)
    g, beta = gate(a, b, a_log, dt_bias)
    return q, k, v, g, beta


@torch.no_grad()
def warm_state(shape: Shape, warmup: int, gen: torch.Generator, device, a_log, dt_bias,
               chunk: int = 32, reference_dist: bool = False) -> torch.Tensor:
    """[B,HV,V,K] float32 state after ``warmup`` gated-delta-rule steps from 0
    (S *= exp(g); S += beta (v - S k) k^T), inputs drawn in chunks of steps.
    With reference_dist the state is 0.02 N(0,1) instead."""
    B, HV, V, K, G = shape.batch, shape.value_heads, shape.value_dim, shape.key_dim, shape.group
    if reference_dist:
        return torch.randn(B, HV, V, K, generator=gen, device=device) * 0.02
    state = torch.zeros(B, HV, V, K, device=device)
    done = 0
    while done < warmup:
        n = min(chunk, warmup - done)
        _, k, v, g, beta = token_inputs(shape, n, gen, device, a_log, dt_bias)
        k = k.repeat_interleave(G, dim=2)
        for t in range(n):
            state.mul_(g[:, t].exp()[..., None, None])
            r = (state * k[:, t][:, :, None, :]).sum(-1)
            state.add_(((v[:, t] - r) * beta[:, t][..., None])[..., None] * k[:, t][:, :, None, :])
        done += n
    return state


def raw_step_inputs(shape: Shape, steps: int, gen: torch.Generator, device, dtype=torch.bfloat16,
                    gate_dtype=torch.bfloat16):
    """Raw full-contract inputs: mixed_qkv [B,T,2HK+HV*V] (q|k|v heads, N(0,1)),
    a, b [B,T,HV] ~ N(0,1)."""
    B, HV = shape.batch, shape.value_heads
    mixed = torch.randn(B, steps, shape.mixed_width, generator=gen, device=device).to(dtype)
    a = torch.randn(B, steps, HV, generator=gen, device=device).to(gate_dtype)
    b = torch.randn(B, steps, HV, generator=gen, device=device).to(gate_dtype)
    return mixed, a, b


def ring_inputs(shape: Shape, ring_len: int, gen: torch.Generator, device, a_log, dt_bias, dtype=torch.bfloat16):
    """A filled ring in storage dtype: q [B,H,K], k [B,L,H,K], v [B,L,HV,V], g, beta [B,L,HV]."""
    q, k, v, g, beta = token_inputs(shape, ring_len, gen, device, a_log, dt_bias)
    return q[:, -1].to(dtype), k.to(dtype), v.to(dtype), g.to(dtype), beta.to(dtype)
