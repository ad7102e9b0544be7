"""The CPU-baseline path (oracle/cpu_torch_path.py, timed by bench.py) computes
the same decode steps as the numpy oracle (CPU only)."""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import cpu_torch_path, gdn_oracle


def test_host_decoder_matches_oracle_cycle():
    rng = np.random.default_rng(0)
    B, H, K, HV, V, L, T = 2, 2, 128, 4, 128, 4, 9
    state = (rng.standard_normal((B, HV, V, K)) * 0.05).astype(np.float32)
    ck = gdn_oracle.quantize_checkpoint(state, "vblock", 32)
    codes_t, scale_t = cpu_torch_path.quantize_vblock32(torch.from_numpy(state))
    # the torch quantiser is the reference quantiser: identical bits
    assert np.array_equal(codes_t.view(torch.uint8).numpy(), ck.payload)
    assert np.array_equal(scale_t.numpy().view(np.uint16), ck.scale.view(np.uint16))
    a_log = rng.uniform(0, math.log(16), HV).astype(np.float32)
    dt_bias = np.zeros(HV, np.float32)
    mixed = gdn_oracle.bf16_round(rng.standard_normal((B, T, 2 * H * K + HV * V)).astype(np.float32))
    a = gdn_oracle.bf16_round(rng.standard_normal((B, T, HV)).astype(np.float32))
    b = gdn_oracle.bf16_round(rng.standard_normal((B, T, HV)).astype(np.float32))
    ref, ref_codes, _ = gdn_oracle.full_contract_decode(ck.payload, ck.scale, mixed, a, b, a_log, dt_bias, L, H, K,
                                                        HV, V, dtype=np.float64)
    dec = cpu_torch_path.HostDecoder(codes_t, scale_t, torch.from_numpy(a_log), torch.from_numpy(dt_bias), H, L)
    outs = []
    for t in range(T):
        outs.append(dec.step(torch.from_numpy(mixed[:, t]).to(torch.bfloat16),
                             torch.from_numpy(a[:, t]).to(torch.bfloat16),
                             torch.from_numpy(b[:, t]).to(torch.bfloat16)).numpy())
    got = np.stack(outs, 1)
    assert gdn_oracle.relative_l2(got, ref) < 1e-5
    assert np.mean(dec.codes.view(torch.uint8).numpy() != ref_codes) < 1e-3
