"""GPU parity of the slot-indexed full-contract step (gdnr_prep_replay_fp8_slots)
and of the host cache that drives it (gdn_replayssm_cache.ReplaySSMCache),
marked `gpu`.

- The slot path is the direct path with other addresses: on the same data it
  gives bit-identical outputs, rings and requantised checkpoints.
- Padding entries (slot 0) leave the null slot untouched.
- Sequences that join at different times, flush at different steps and reuse
  a released slot match the fp64 oracle of the reference's cycle
  (prototype/bench_gdn_full_contract.py:225-308) per sequence: output rel-L2
  <= 2e-3, requantised codes equal up to < 1e-3 rounding-boundary flips.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import gdn_replayssm_fp8_kernel as gk
import gdn_replayssm_synth as synth
from conftest import rel_l2
from gdn_replayssm_cache import ReplaySSMCache
from gpu_helpers import codes_np, np32
from oracle import gdn_oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("L,nseq", [(8, 8), (32, 8), (64, 8), (64, 17)])
def test_slots_equal_direct_path(device, L, nseq):
    """nseq sequences live in scattered slots of a cache of nseq + 4 slots
    (8: slots 9, 2, 5, 11, 1, 7, 4, 10 of 12); the batch also carries two
    padding entries. 2.5 ring cycles with staggered ring fills (every
    sequence flushes twice): every output, ring row and checkpoint byte
    equals the direct path's on batch-ordered copies. L = 8 runs the decode
    kernel, L = 32 and 64 with 8 sequences its chunked path (10 batch entries
    of 32 value heads); 17 sequences at L = 64 the long-ring kernel (slots and
    direct path both past the decode kernel's 16 sequences)."""
    B, steps = nseq, (5 * L) // 2
    shape = synth.Shape(B)
    gen = synth.generator(61, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 32, gen, device, a_log, dt_bias)
    ck = gk.quantize_checkpoint(state)
    rng = np.random.default_rng(nseq)
    slot_of = [9, 2, 5, 11, 1, 7, 4, 10] if nseq == 8 else [int(x) for x in rng.permutation(np.arange(1, nseq + 4))[:nseq]]
    cache = ReplaySSMCache(nseq + 4, L, device=device)
    for i, sl in enumerate(slot_of):
        cache.payload[sl].copy_(ck.payload[i])
        cache.scale[sl].copy_(ck.scale[i])
        cache.fill[sl] = i % L  # staggered ring phases (the rings start empty: stale rows are never read)
    direct = dict(payload=ck.payload.clone(), scale=ck.scale.clone(),
                  rings=[torch.zeros(B, L, 16, 128, dtype=torch.bfloat16, device=device),
                         torch.zeros(B, L, 32, 128, dtype=torch.bfloat16, device=device),
                         torch.zeros(B, L, 32, dtype=torch.bfloat16, device=device),
                         torch.zeros(B, L, 32, dtype=torch.bfloat16, device=device)])
    fill = np.array([i % L for i in range(B)])
    mixed, a, b = synth.raw_step_inputs(shape, steps, gen, device)
    pad_mixed = torch.randn(2, steps, shape.mixed_width, generator=gen, device=device).to(torch.bfloat16)
    pad_ab = torch.randn(2, steps, 32, generator=gen, device=device).to(torch.bfloat16)
    # batch entry e holds sequence order[e]
    order = [3, 0, 6, 1, 7, 2, 5, 4] if nseq == 8 else [int(x) for x in rng.permutation(nseq)]
    batch_slots = [slot_of[i] for i in order[:4]] + [0] + [slot_of[i] for i in order[4:]] + [0]
    seq_of_entry = order[:4] + [None] + order[4:] + [None]
    null_before = (cache.payload[0].clone(), cache.scale[0].clone(), [r[0].clone() for r in
                                                                     (cache.k_ring, cache.v_ring, cache.g_ring,
                                                                      cache.beta_ring)])
    for step in range(steps):
        rows, pad_rows = [], iter(range(2))
        for e in seq_of_entry:
            if e is None:
                p = next(pad_rows)
                rows.append((pad_mixed[p, step], pad_ab[p, step], pad_ab[p, step]))
            else:
                rows.append((mixed[e, step], a[e, step], b[e, step]))
        m = torch.stack([r[0] for r in rows]).contiguous()
        aa = torch.stack([r[1] for r in rows]).contiguous()
        bb = torch.stack([r[2] for r in rows]).contiguous()
        got = cache.step(batch_slots, m, aa, bb, a_log, dt_bias)
        valid = torch.as_tensor(fill + 1, dtype=torch.int32, device=device)
        q_out = torch.empty(B, 16, 128, dtype=torch.bfloat16, device=device)
        want = gk.gdn_prep_replay_fp8(mixed[:, step].contiguous(), a[:, step].contiguous(), b[:, step].contiguous(),
                                      a_log, dt_bias, valid - 1, direct["payload"], direct["scale"], q_out,
                                      *direct["rings"], valid, valid == L)
        fill = np.where(fill + 1 == L, 0, fill + 1)
        for e, seq in enumerate(seq_of_entry):
            if seq is not None:
                assert torch.equal(got[e], want[seq]), (step, e, seq)
    for i, sl in enumerate(slot_of):
        assert torch.equal(cache.payload[sl].view(torch.uint8), direct["payload"][i].view(torch.uint8))
        assert torch.equal(cache.scale[sl], direct["scale"][i])
        for r_cache, r_direct in zip((cache.k_ring, cache.v_ring, cache.g_ring, cache.beta_ring), direct["rings"]):
            assert torch.equal(r_cache[sl], r_direct[i])
    assert torch.equal(cache.payload[0].view(torch.uint8), null_before[0].view(torch.uint8))
    assert torch.equal(cache.scale[0], null_before[1])
    for r, before in zip((cache.k_ring, cache.v_ring, cache.g_ring, cache.beta_ring), null_before[2]):
        assert torch.equal(r[0], before)


@pytest.mark.parametrize("L,nseq", [(8, 6), (64, 6), (64, 17)])
def test_slots_beyond_4096_equal_direct_path(device, L, nseq):
    """A cache of 5000 slots (a 2.6 GB checkpoint, more than 4 GiB of ring and
    checkpoint together: every sequence's base address needs 64 bits): six
    sequences in slots 4999, 4097, 4096, 2049, 4998 and 17 (17 sequences:
    eleven more, scattered), L + 2 steps with staggered fills (every
    sequence flushes): outputs, ring rows and checkpoint bytes equal the
    direct path's on batch-ordered copies, bit for bit. L = 8: the decode
    kernel; L = 64 (6.4 GiB of cache): its chunked path with 6 sequences,
    the long-ring kernel with 17."""
    B, steps, n_slots = nseq, L + 2, 5000
    shape = synth.Shape(B)
    gen = synth.generator(63, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 16, gen, device, a_log, dt_bias)
    ck = gk.quantize_checkpoint(state)
    slot_of = [4999, 4097, 4096, 2049, 4998, 17, 4500, 3001, 1, 4098, 4995, 2500, 100, 4200, 3999, 4001, 2][:nseq]
    cache = ReplaySSMCache(n_slots, L, device=device)
    for i, sl in enumerate(slot_of):
        cache.payload[sl].copy_(ck.payload[i])
        cache.scale[sl].copy_(ck.scale[i])
        cache.fill[sl] = (3 * i) % L
    direct = dict(payload=ck.payload.clone(), scale=ck.scale.clone(),
                  rings=[torch.zeros(B, L, 16, 128, dtype=torch.bfloat16, device=device),
                         torch.zeros(B, L, 32, 128, dtype=torch.bfloat16, device=device),
                         torch.zeros(B, L, 32, dtype=torch.bfloat16, device=device),
                         torch.zeros(B, L, 32, dtype=torch.bfloat16, device=device)])
    fill = np.array([(3 * i) % L for i in range(B)])
    mixed, a, b = synth.raw_step_inputs(shape, steps, gen, device)
    flushed = 0
    for step in range(steps):
        got = cache.step(slot_of, mixed[:, step].contiguous(), a[:, step].contiguous(), b[:, step].contiguous(),
                         a_log, dt_bias)
        valid = torch.as_tensor(fill + 1, dtype=torch.int32, device=device)
        flushed += int((fill + 1 == L).sum())
        q_out = torch.empty(B, 16, 128, dtype=torch.bfloat16, device=device)
        want = gk.gdn_prep_replay_fp8(mixed[:, step].contiguous(), a[:, step].contiguous(), b[:, step].contiguous(),
                                      a_log, dt_bias, valid - 1, direct["payload"], direct["scale"], q_out,
                                      *direct["rings"], valid, valid == L)
        fill = np.where(fill + 1 == L, 0, fill + 1)
        assert torch.equal(got, want), step
    assert flushed >= B
    for i, sl in enumerate(slot_of):
        assert torch.equal(cache.payload[sl].view(torch.uint8), direct["payload"][i].view(torch.uint8)), sl
        assert torch.equal(cache.scale[sl], direct["scale"][i]), sl
        for r_cache, r_direct in zip((cache.k_ring, cache.v_ring, cache.g_ring, cache.beta_ring), direct["rings"]):
            assert torch.equal(r_cache[sl], r_direct[i]), sl


def test_cache_lifecycle_matches_oracle(device):
    """Three sequences in a 4-slot cache, L=4: A starts at step 0, B at step 2,
    C replaces A in A's slot at step 7 (A released). Each sequence's outputs
    and final checkpoint follow the oracle's cycle started from its own
    checkpoint."""
    L, steps = 4, 12
    shape = synth.Shape(3)
    gen = synth.generator(62, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    states = synth.warm_state(shape, 32, gen, device, a_log, dt_bias)
    mixed, a, b = synth.raw_step_inputs(shape, steps, gen, device)
    cache = ReplaySSMCache(4, L, device=device)
    life = {0: (3, 0, 7), 1: (1, 2, steps), 2: (3, 7, steps)}  # sequence: (slot, first step, end step)
    ck0 = {}
    outs = {s: [] for s in life}
    for step in range(steps):
        for s, (slot, start, end) in life.items():
            if step == end and s == 0:
                cache.release(slot)
            if step == start:
                cache.load_state(slot, states[s])
                ck0[s] = (codes_np(cache.payload[slot:slot + 1]).copy(), cache.scale[slot:slot + 1].cpu().numpy().copy())
        active = [s for s, (slot, start, end) in life.items() if start <= step < end]
        slots = [life[s][0] for s in active]
        idx = torch.as_tensor(active, device=device)
        got = cache.step(slots, mixed[idx, step].contiguous(), a[idx, step].contiguous(), b[idx, step].contiguous(),
                         a_log, dt_bias)
        for e, s in enumerate(active):
            outs[s].append(np32(got[e]))
    for s, (slot, start, end) in life.items():
        codes0, scale0 = ck0[s]
        sl = slice(s, s + 1)
        ref, ref_codes, _ = gdn_oracle.full_contract_decode(
            codes0, scale0, np32(mixed[sl, start:end]), np32(a[sl, start:end]), np32(b[sl, start:end]), np32(a_log),
            np32(dt_bias), L, 16, 128, 32, 128, dtype=np.float64)
        assert rel_l2(np.stack(outs[s]), ref[0]) <= 2e-3, s
        if s != 0:  # A's slot now holds C
            assert np.mean(codes_np(cache.payload[slot:slot + 1]) != ref_codes) < 1e-3, s
