"""Slot-indexed ReplaySSM state for a decode batch that changes from step to
step: the caller's side of the decode step.

The reference sequences the full-contract step on the host
(prototype/bench_gdn_full_contract.py:113-154,225-308): ring slot
pos = position, replay with valid_len = fill, flush when the ring is full,
ring restarted after it. vLLM keeps per-sequence recurrent state in cache
slots addressed by ssm_state_indices, with slot 0 the null block
(findings.md:35-56; the model hook prototype/qwen35_replay_ab.py:61-75,234-292).
ReplaySSMCache combines the two:

  * checkpoint, scale and the k/v/g/beta rings are [S, ...] device tensors,
    one row per slot, row 0 the null slot;
  * the ring fill of every slot lives on the host (the caller knows how many
    tokens each sequence has appended), so building a step's metadata needs
    no device round trip;
  * step() takes the batch's slots (host ints; 0 marks a padding entry),
    derives pos = fill, valid_len = fill + 1, flush = (valid_len == L), runs
    ONE fused launch (gdn_prep_replay_fp8 with state_indices), and advances
    the fills: 0 after a flush (the ring restarts), fill + 1 otherwise.
    Padding entries append nothing (pos -1), replay nothing (valid_len 0)
    and never flush, so the null slot is never written.
"""

from __future__ import annotations

import numpy as np
import torch

import gdn_replayssm_fp8_kernel as gk

FP8_DTYPE = torch.float8_e4m3fn


class ReplaySSMCache:
    """ReplaySSM checkpoints and rings for ``num_slots`` sequences (slots
    1..num_slots; slot 0 is the null slot) of one GDN layer."""

    def __init__(self, num_slots: int, window: int, heads: int = 16, value_heads: int = 32, key_dim: int = 128,
                 value_dim: int = 128, dtype: torch.dtype = torch.bfloat16, device="cuda"):
        if num_slots < 1:
            raise ValueError("num_slots must be at least 1")
        if not 1 <= window <= 64:
            raise ValueError("the slot-indexed step takes rings of 1 to 64 tokens")
        if value_heads % heads or value_dim % gk.VBLOCK:
            raise ValueError("value_heads must be a multiple of heads and value_dim of 32")
        self.window, self.heads, self.value_heads = window, heads, value_heads
        self.key_dim, self.value_dim, self.dtype = key_dim, value_dim, dtype
        self.device = torch.device(device)
        S = num_slots + 1
        self.payload = torch.zeros(S, value_heads, value_dim, key_dim, dtype=FP8_DTYPE, device=self.device)
        self.scale = torch.ones(S, value_heads, value_dim // gk.VBLOCK, dtype=torch.float16, device=self.device)
        self.k_ring = torch.zeros(S, window, heads, key_dim, dtype=dtype, device=self.device)
        self.v_ring = torch.zeros(S, window, value_heads, value_dim, dtype=dtype, device=self.device)
        self.g_ring = torch.zeros(S, window, value_heads, dtype=dtype, device=self.device)
        self.beta_ring = torch.zeros(S, window, value_heads, dtype=dtype, device=self.device)
        self.fill = np.zeros(S, dtype=np.int64)  # tokens in each slot's ring since its last flush

    @property
    def num_slots(self) -> int:
        return self.fill.shape[0] - 1

    def _check_slot(self, slot: int) -> None:
        if not 1 <= slot <= self.num_slots:
            raise ValueError(f"slot {slot} outside 1..{self.num_slots}")

    def load_state(self, slot: int, state: torch.Tensor) -> None:
        """Start a sequence in ``slot`` from an fp32 state [HV, V, K] (a
        prefill's final state): quantised to the slot's checkpoint, empty ring."""
        self._check_slot(slot)
        ck = gk.quantize_checkpoint(state.reshape(1, *state.shape).float().to(self.device), saturation=False)
        self.payload[slot].copy_(ck.payload[0])
        self.scale[slot].copy_(ck.scale[0])
        self.fill[slot] = 0

    def release(self, slot: int) -> None:
        """End the sequence in ``slot``: its ring restarts; the slot is free."""
        self._check_slot(slot)
        self.fill[slot] = 0

    def metadata(self, slots) -> tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
        """(slots, pos, valid_len, flush) of one step for the batch ``slots``
        (0 = padding), from the host-side ring fills."""
        slots = np.asarray(slots, dtype=np.int64)
        if slots.ndim != 1:
            raise ValueError("slots must be one-dimensional")
        if ((slots < 0) | (slots > self.num_slots)).any():
            raise ValueError(f"slots outside 0..{self.num_slots}")
        live = slots[slots != 0]
        if np.unique(live).size != live.size:
            raise ValueError("a non-null slot appears twice in the batch")
        pad = slots == 0
        fill = self.fill[slots]
        pos = np.where(pad, -1, fill)
        valid = np.where(pad, 0, fill + 1)
        flush = ~pad & (valid == self.window)
        return slots, pos, valid, flush

    def step(self, slots, mixed_qkv: torch.Tensor, a: torch.Tensor, b: torch.Tensor, a_log: torch.Tensor,
             dt_bias: torch.Tensor, block_v: int = 128, q_out: torch.Tensor | None = None,
             out: torch.Tensor | None = None) -> torch.Tensor:
        """One full-contract decode step of the batch: batch entry i is the
        sequence in slot slots[i] (0 = padding; its output is meaningless).
        mixed_qkv [B, 2HK + HV V], a, b [B, HV]; returns out [B, HV, V]."""
        slots, pos, valid, flush = self.metadata(slots)
        batch = slots.shape[0]
        if mixed_qkv.shape[0] != batch:
            raise ValueError(f"mixed_qkv has {mixed_qkv.shape[0]} rows for a batch of {batch}")
        meta = torch.from_numpy(np.stack([slots, pos, valid, flush.astype(np.int64)]).astype(np.int32))
        meta = meta.pin_memory().to(self.device, non_blocking=True)
        if q_out is None:
            q_out = torch.empty(batch, self.heads, self.key_dim, dtype=self.dtype, device=self.device)
        result = gk.gdn_prep_replay_fp8(mixed_qkv, a, b, a_log, dt_bias, meta[1], self.payload, self.scale, q_out,
                                        self.k_ring, self.v_ring, self.g_ring, self.beta_ring, meta[2],
                                        meta[3].bool(), block_v=block_v, out=out, state_indices=meta[0])
        live = slots != 0
        self.fill[slots[live]] = np.where(flush, 0, valid)[live]
        return result
