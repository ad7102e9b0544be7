"""torch-CPU restatement of the reference's host decode path -- the CPU
baseline that bench.py times beside the GPU.

TEST / BASELINE INFRASTRUCTURE ONLY: imported by bench.py's cpu_baseline leg
and by tests/ (which check it against gdn_oracle); never by the product.

It runs the same per-step algorithm as the reference's fp32 path
(prototype/gdn_replay_fp8_reference.py), in fp32 torch ops on the host cores:
  prep       q,k L2-normalised, g = -exp(A_log) softplus_20(a + dt_bias),
             beta = sigmoid(b), appended to the ring       (kernel:504-562)
  replay     dequantise the vblock32 checkpoint             (ref:109-134)
             forward recurrence over the ring tokens         (ref:137-163)
             emit the last token's output                    (ref:208-217)
  flush      when the ring holds L tokens: requantise the
             rebuilt state, restart the ring                 (ref:218-229, :40-106)
"""

from __future__ import annotations

import torch

FP8_MAX = 448.0
VBLOCK = 32


def dequantize_vblock32(codes: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """codes [B,HV,V,K] float8_e4m3fn, scale [B,HV,V/32] fp16 -> fp32 state."""
    B, HV, V, K = codes.shape
    values = codes.float().view(B, HV, V // VBLOCK, VBLOCK, K)
    return (values * scale.float()[..., None, None]).view(B, HV, V, K)


def quantize_vblock32(state: torch.Tensor):
    """fp32 state -> (codes fp8, scale fp16): scale = fp16(amax/448) (1 where
    amax is not > 0); codes = e4m3fn(clamp(state / (amax/448), +-448))."""
    B, HV, V, K = state.shape
    blocks = state.view(B, HV, V // VBLOCK, VBLOCK, K)
    amax = blocks.abs().amax(dim=(-2, -1), keepdim=True)
    s32 = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    codes = (blocks / s32).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn).view(B, HV, V, K)
    return codes, s32.view(B, HV, V // VBLOCK).to(torch.float16)


def forward_replay(state, q, k_ring, v_ring, g_ring, beta_ring, n):
    """Forward recurrence of ring tokens [0, n) from ``state`` (modified in
    place); returns (o of the last token [B,HV,V], rebuilt state)."""
    B, HV, V, K = state.shape
    G = HV // q.shape[1]
    qq = q.float().repeat_interleave(G, dim=1)
    for t in range(n):
        kk = k_ring[:, t].float().repeat_interleave(G, dim=1)
        state.mul_(torch.exp(g_ring[:, t].float())[..., None, None])
        retrieved = torch.einsum("bjvk,bjk->bjv", state, kk)
        correction = (v_ring[:, t].float() - retrieved) * beta_ring[:, t].float()[..., None]
        state.add_(correction[..., None] * kk[:, :, None, :])
    return torch.einsum("bjvk,bjk->bjv", state, qq) * (K ** -0.5), state


class HostDecoder:
    """Full-contract decode steps for a batch whose sequences share one ring
    phase (the reference's cycle, prototype/bench_gdn_full_contract.py:225-308)."""

    def __init__(self, codes, scale, a_log, dt_bias, heads, window, ring_dtype=torch.bfloat16):
        B, HV, V, K = codes.shape
        self.codes, self.scale = codes.clone(), scale.clone()
        self.a_log, self.dt_bias = a_log.float(), dt_bias.float()
        self.H, self.HV, self.K, self.V, self.L = heads, HV, K, V, window
        self.k_ring = torch.zeros(B, window, heads, K, dtype=ring_dtype)
        self.v_ring = torch.zeros(B, window, HV, V, dtype=ring_dtype)
        self.g_ring = torch.zeros(B, window, HV, dtype=ring_dtype)
        self.beta_ring = torch.zeros(B, window, HV, dtype=ring_dtype)
        self.fill = 0

    def prep(self, mixed, a, b):
        H, HV, K, V = self.H, self.HV, self.K, self.V
        x = mixed.float()
        q = x[:, :H * K].view(-1, H, K)
        k = x[:, H * K:2 * H * K].view(-1, H, K)
        v = mixed[:, 2 * H * K:2 * H * K + HV * V].view(-1, HV, V)
        q = q / torch.sqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        k = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
        xg = a.float() + self.dt_bias
        softplus = torch.where(xg <= 20.0, torch.log(1.0 + torch.exp(xg)), xg)
        g = -torch.exp(self.a_log) * softplus
        beta = torch.sigmoid(b.float())
        pos = self.fill
        dt = self.k_ring.dtype
        self.k_ring[:, pos] = k.to(dt)
        self.v_ring[:, pos] = v.to(dt)
        self.g_ring[:, pos] = g.to(dt)
        self.beta_ring[:, pos] = beta.to(dt)
        self.fill += 1
        return q.to(dt)

    def step(self, mixed, a, b):
        q = self.prep(mixed, a, b)
        state = dequantize_vblock32(self.codes, self.scale)
        out, rebuilt = forward_replay(state, q, self.k_ring, self.v_ring, self.g_ring, self.beta_ring, self.fill)
        if self.fill == self.L:
            self.codes, self.scale = quantize_vblock32(rebuilt)
            self.fill = 0
        return out
