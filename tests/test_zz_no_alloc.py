"""gdnr_replay_fp8_split_noalloc (marked `gpu`): the split replay with its
T_0 / coefficient buffers in the library's device array, called through the
C-ABI, against gdnr_replay_fp8_split with caller buffers (the same kernels,
so bit for bit), on two calls in a row, the second with a smaller input
(fewer sequences, a shorter ring, other fills). Also: sizes beyond the
array are refused with a clear error."""

from __future__ import annotations

import pytest
import torch

import gdnr_lib
from gpu_helpers import make_replay_case

pytestmark = pytest.mark.gpu


def _split_with_buffers(case, out):
    B, L = case["k"].shape[0], case["k"].shape[1]
    tq = torch.empty(B, 32, 128, dtype=torch.float32, device=out.device)
    coef = torch.zeros(B, 32, L, dtype=torch.float32, device=out.device)
    gdnr_lib.call("gdnr_replay_fp8_split",
                  [case["ckpt"].payload, case["ckpt"].scale, case["q"], case["k"], case["v"], case["g"],
                   case["beta"], case["valid"], tq, coef, out],
                  [128, 128, 1], gdnr_lib.current_stream(out.device))


def _split_noalloc(case, out, grouped=1):
    gdnr_lib.call("gdnr_replay_fp8_split_noalloc",
                  [case["ckpt"].payload, case["ckpt"].scale, case["q"], case["k"], case["v"], case["g"],
                   case["beta"], case["valid"], out],
                  [128, 128, grouped], gdnr_lib.current_stream(out.device))


def test_noalloc_split_equals_split(device):
    for batch, ring_len, seed in ((24, 16, 11), (5, 8, 12)):   # the second call is smaller
        case = make_replay_case(batch, ring_len, device, seed=seed)
        want = torch.empty(batch, 32, 128, dtype=case["q"].dtype, device=device)
        got = torch.full_like(want, float("nan"))
        _split_with_buffers(case, want)
        _split_noalloc(case, got)
        torch.cuda.synchronize(device)
        assert torch.equal(got, want), (batch, ring_len)
        got2 = torch.full_like(want, float("nan"))
        _split_noalloc(case, got2, grouped=0)
        torch.cuda.synchronize(device)
        assert torch.equal(got2, want), (batch, ring_len, "ungrouped")


def test_noalloc_split_refuses_oversize(device):
    case = make_replay_case(1, 4, device, seed=13)
    # 160 sequences x 32 value heads x (128 + 64) x 4 bytes > 3 MiB: refused before any launch
    big = {key: (val.expand(160, *val.shape[1:]) if torch.is_tensor(val) and val.dim() > 0 else val)
           for key, val in case.items() if key in ("q", "valid")}
    ring = {key: torch.zeros(160, 64, *case[key].shape[2:], dtype=case[key].dtype, device=device)
            for key in ("k", "v", "g", "beta")}
    ckpt = torch.zeros(160, 32, 128, 128, dtype=torch.uint8, device=device).view(torch.float8_e4m3fn)
    scale = torch.ones(160, 32, 4, dtype=torch.float16, device=device)
    out = torch.empty(160, 32, 128, dtype=case["q"].dtype, device=device)
    with pytest.raises(gdnr_lib.GdnrError, match="split scratch"):
        gdnr_lib.call("gdnr_replay_fp8_split_noalloc",
                      [ckpt, scale, big["q"].contiguous(), ring["k"], ring["v"], ring["g"], ring["beta"],
                       big["valid"].contiguous(), out],
                      [128, 128, 1], gdnr_lib.current_stream(device))
