"""Byte model of the ReplaySSM GDN decode path (HBM bytes per call).

Two accountings:

* ``algorithmic``: every compulsory tensor element counted once per call
  (checkpoint codes + scales, query, the ``fill`` ring tokens, output; a
  flush also writes the checkpoint back). This is the figure the roofline
  fraction is computed from:
      C = B*HV*V*K (fp8)       S = B*HV*(V/32)*2       Q = B*H*K*2
      O = B*HV*V*2             R = B*(H*K*2 + HV*V*2 + HV*2*2) per ring token
      replay(l) = C + S + Q + l*R + O
      flush(L)  = 2C + 2S + Q + L*R + O
      prep      = B*(2HK + HV*V)*2 + 2*B*HV*sizeof(a) + HV*8 + B*4 + Q + R
      full-contract per step = [sum_{l=1}^{L-1} replay(l) + flush(L) + L*prep] / L
* ``reference``: the reference's own per-call accounting, restated from
  prototype/bench_gdn_replayssm.py:45-87 (``traffic_bytes``: ring always
  full, no output term, query/keys re-read per V tile in ``replay_actual``),
  kept so ratios can be quoted on the reference's terms.

The bf16 read-modify-write comparison is B*HV*V*K*2*2 bytes per step
(state read + write, prototype/bench_gdn_replayssm.py:82).
"""

from __future__ import annotations

from dataclasses import dataclass

VBLOCK = 32


@dataclass(frozen=True)
class LayerShape:
    batch: int
    heads: int = 16          # H, key heads
    value_heads: int = 32    # HV
    key_dim: int = 128       # K
    value_dim: int = 128     # V
    act_bytes: int = 2       # q / ring / out storage (bf16)
    gate_bytes: int = 2      # a, b raw gating inputs (bf16)

    @property
    def checkpoint(self) -> int:
        return self.batch * self.value_heads * self.value_dim * self.key_dim

    @property
    def scales(self) -> int:
        return self.batch * self.value_heads * (self.value_dim // VBLOCK) * 2

    @property
    def query(self) -> int:
        return self.batch * self.heads * self.key_dim * self.act_bytes

    @property
    def output(self) -> int:
        return self.batch * self.value_heads * self.value_dim * self.act_bytes

    @property
    def ring_token(self) -> int:
        """k + v + g + beta of one token for the whole batch."""
        return self.batch * (self.heads * self.key_dim * self.act_bytes
                             + self.value_heads * self.value_dim * self.act_bytes
                             + self.value_heads * 2 * self.act_bytes)

    @property
    def mixed_row(self) -> int:
        return (2 * self.heads * self.key_dim + self.value_heads * self.value_dim) * self.act_bytes


def replay_bytes(s: LayerShape, fill: int, flush: bool) -> int:
    """Algorithmic bytes of one gdn_replay_fp8 call with ring fill ``fill``."""
    base = s.query + fill * s.ring_token + s.output
    if flush:
        return 2 * s.checkpoint + 2 * s.scales + base
    return s.checkpoint + s.scales + base


def prep_bytes(s: LayerShape) -> int:
    """Algorithmic bytes of one gdn_prep_ring call: mixed_qkv row, a, b,
    A_log + dt_bias (f32), pos (i32) read; q_out and one ring slot written."""
    return (s.batch * s.mixed_row + 2 * s.batch * s.value_heads * s.gate_bytes + s.value_heads * 8
            + s.batch * 4 + s.query + s.ring_token)


def cycle_bytes_per_step(s: LayerShape, window: int, with_prep: bool = True) -> float:
    """Full-contract (with_prep) or core bytes per decode step, averaged over
    one ring cycle: fills 1..window-1 replay, fill == window flushes."""
    total = sum(replay_bytes(s, fill, False) for fill in range(1, window)) + replay_bytes(s, window, True)
    if with_prep:
        total += window * prep_bytes(s)
    return total / window


def bf16_rmw_bytes(s: LayerShape) -> int:
    """State bytes of a bf16 read-modify-write decode step."""
    return s.batch * s.value_heads * s.value_dim * s.key_dim * 2 * 2


def reference_traffic(s: LayerShape, window: int, block_v: int) -> dict:
    """The reference's accounting (prototype/bench_gdn_replayssm.py:45-87)."""
    tiles = s.value_dim // block_v
    checkpoint = s.checkpoint
    scales = s.batch * s.value_heads * tiles * 2
    query = s.query
    ring_key = s.batch * window * s.heads * s.key_dim * 2
    ring_value = s.batch * window * s.value_heads * s.value_dim * 2
    ring_scalars = s.batch * window * s.value_heads * 4
    return {
        "replay_logical": checkpoint + scales + query + ring_key + ring_value + ring_scalars,
        "replay_actual": checkpoint + scales + tiles * (query + ring_key) + ring_value + ring_scalars,
        "flush_actual": 2 * checkpoint + 2 * scales + tiles * ring_key + ring_value + ring_scalars,
        "bf16_baseline": bf16_rmw_bytes(s),
    }
