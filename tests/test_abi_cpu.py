"""The C-ABI library on the CPU: it loads, exports every symbol include/gdnr.h
declares, and rejects misuse on the host before any HIP call.

Every call here fails validation (or has batch 0), so no kernel is launched
and no GPU is needed; the descriptors carry fake, never-dereferenced device
addresses. The reference wrappers validate nothing
(prototype/gdn_replayssm_fp8_kernel.py:344-405,710-795,1129-1235).
"""

from __future__ import annotations

import ctypes
import re
import subprocess

import pytest
import torch

import gdnr_lib
from conftest import REPO

OK, INVALID, UNSUPPORTED = 0, 1, 2
BF16, F16, F32, FP8, U8, I32, I64, BOOL = range(8)
FAKE = 0x7F0000000000  # 256-byte aligned, never dereferenced


def desc(shape, dtype, data=FAKE, strides=None):
    t = gdnr_lib.GdnrTensor()
    t.data = data or None
    t.dtype = dtype
    t.ndim = len(shape)
    if strides is None:
        strides, acc = [], 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    for d, (s, st) in enumerate(zip(shape, strides)):
        t.shape[d] = s
        t.strides[d] = st
    return t


@pytest.fixture(scope="module")
def lib():
    return gdnr_lib.load_library()


def declared_functions() -> list[str]:
    header = (REPO / "include" / "gdnr.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(gdnr_\w+)\s*\(", header, flags=re.M)))


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert len(names) >= 8, names
    out = subprocess.run(["nm", "-D", "--defined-only", str(gdnr_lib.LIBRARY_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\bT (gdnr_\w+)$", out, flags=re.M))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for name in names:
        assert hasattr(lib, name)
    assert set(gdnr_lib.ENTRY_POINTS) <= set(names)


def test_abi_version(lib):
    assert lib.gdnr_abi_version() == gdnr_lib.ABI_VERSION


class ReplayCase:
    """A valid gdnr_replay_fp8 argument set at B=2, H=2, HV=4, L=4 (bf16);
    tests break one argument at a time."""

    def __init__(self, B=2, H=2, HV=4, K=128, V=128, L=4):
        self.t = {
            "checkpoint": desc([B, HV, V, K], FP8),
            "checkpoint_scale": desc([B, HV, V // 32], F16),
            "q": desc([B, H, K], BF16),
            "k_cache": desc([B, L, H, K], BF16),
            "v_cache": desc([B, L, HV, V], BF16),
            "g_cache": desc([B, L, HV], BF16),
            "beta_cache": desc([B, L, HV], BF16),
            "valid_len": desc([B], I32),
            "flush": desc([B], BOOL),
            "out": desc([B, HV, V], BF16),
        }
        self.block_v = 128

    def call(self, lib):
        ptrs = [ctypes.byref(self.t[k]) for k in ("checkpoint", "checkpoint_scale", "q", "k_cache", "v_cache",
                                                  "g_cache", "beta_cache", "valid_len", "flush", "out")]
        rc = lib.gdnr_replay_fp8(*ptrs, self.block_v, None)
        return rc, lib.gdnr_last_error().decode()


@pytest.mark.parametrize("mutate,code,needle", [
    (lambda c: c.t.__setitem__("checkpoint", desc([2, 4, 128, 64], FP8)), INVALID, "checkpoint"),
    (lambda c: c.t.__setitem__("k_cache", desc([2, 4, 2, 64], BF16)), UNSUPPORTED, "K=64"),
    (lambda c: c.t.__setitem__("checkpoint_scale", desc([2, 4, 4], F32)), INVALID, "checkpoint_scale"),
    (lambda c: c.t.__setitem__("valid_len", desc([2], I64)), INVALID, "valid_len"),
    (lambda c: c.t.__setitem__("flush", desc([3], BOOL)), INVALID, "flush"),
    (lambda c: c.t.__setitem__("q", desc([2, 2, 128], F16)), INVALID, "q"),
    (lambda c: c.t.__setitem__("out", desc([2, 4, 96], BF16)), INVALID, "out"),
    (lambda c: c.t.__setitem__("g_cache", desc([2, 4, 4], F32)), UNSUPPORTED, "g_cache"),
    (lambda c: c.t.__setitem__("checkpoint", desc([2, 4, 128, 128], FP8, data=FAKE + 8)), INVALID, "aligned"),
    (lambda c: c.t.__setitem__("k_cache", desc([2, 4, 2, 128], BF16, strides=[1024, 256, 128, 2])), INVALID,
     "innermost"),
    (lambda c: setattr(c, "block_v", 48), INVALID, "block_v"),
    (lambda c: c.t.__setitem__("checkpoint", desc([2, 4, 128, 128], F32)), INVALID, "checkpoint"),
    (lambda c: c.t.__setitem__("q", desc([2, 2, 128], BF16, data=0)), INVALID, "null data"),
])
def test_replay_rejects_misuse(lib, mutate, code, needle):
    case = ReplayCase()
    mutate(case)
    rc, msg = case.call(lib)
    assert rc == code, msg
    assert needle in msg, msg


def test_ring_longer_than_built_is_unsupported(lib):
    case = ReplayCase(L=65)
    rc, msg = case.call(lib)
    assert rc == UNSUPPORTED and "ring length" in msg


def test_value_heads_must_be_a_multiple_of_key_heads(lib):
    rc, msg = ReplayCase(H=2, HV=3).call(lib)
    assert rc == INVALID and "multiple of key heads" in msg


def test_empty_batch_is_a_no_op(lib):
    case = ReplayCase(B=0)
    rc, msg = case.call(lib)
    assert rc == OK and msg == ""


def test_prep_checks_mixed_qkv_width(lib):
    B, H, HV, K, V, L = 2, 2, 4, 128, 128, 4
    args = [desc([B, 2 * H * K + HV * V - 8], BF16), desc([B, HV], BF16), desc([B, HV], BF16), desc([HV], F32),
            desc([HV], F32), desc([B], I32), desc([B, H, K], BF16), desc([B, L, H, K], BF16),
            desc([B, L, HV, V], BF16), desc([B, L, HV], BF16), desc([B, L, HV], BF16)]
    rc = lib.gdnr_prep_ring(*[ctypes.byref(a) for a in args], 1, None)
    assert rc == INVALID and "mixed_qkv" in lib.gdnr_last_error().decode()
    # wider than 2 H K + HV V: accepted, as by the reference (kernel:500-550
    # reads the first 2 H K + HV V columns of each row); the A_log check below
    # then fails on its own account
    args[0] = desc([B, 2 * H * K + HV * V + 256], BF16)
    args[3] = desc([HV], BF16)                           # A_log must be f32
    rc = lib.gdnr_prep_ring(*[ctypes.byref(a) for a in args], 1, None)
    assert rc == INVALID and "a_log" in lib.gdnr_last_error().decode()


def test_split_rejects_short_coefficient_buffer(lib):
    case = ReplayCase()
    t = case.t
    tq = desc([2, 4, 128], F32)
    coef = desc([2, 4, 3], F32)                          # ring is 4 long
    ptrs = [ctypes.byref(t[k]) for k in ("checkpoint", "checkpoint_scale", "q", "k_cache", "v_cache", "g_cache",
                                         "beta_cache", "valid_len")]
    rc = lib.gdnr_replay_fp8_split(*ptrs, ctypes.byref(tq), ctypes.byref(coef), ctypes.byref(t["out"]), 128, 128, 1,
                                   None)
    assert rc == INVALID and "coefficient_buffer" in lib.gdnr_last_error().decode()


def test_quantize_rejects_wrong_key_dim(lib):
    rc = lib.gdnr_quantize_vblock32(ctypes.byref(desc([1, 2, 32, 64], F32)), ctypes.byref(desc([1, 2, 32, 64], FP8)),
                                    ctypes.byref(desc([1, 2, 1], F16)), None, None)
    assert rc == UNSUPPORTED and "K=64" in lib.gdnr_last_error().decode()


def test_last_error_is_cleared_by_a_good_call(lib):
    ReplayCase(L=65).call(lib)
    assert lib.gdnr_last_error().decode() != ""
    rc, msg = ReplayCase(B=0).call(lib)
    assert rc == OK and msg == ""


def test_python_wrappers_refuse_host_tensors():
    """The drop-in functions never fall back to a CPU path."""
    import gdn_replayssm_fp8_kernel as gk

    B, H, HV, L = 1, 1, 2, 2
    z = lambda *s, dtype=torch.bfloat16: torch.zeros(*s, dtype=dtype)
    with pytest.raises(ValueError, match="GPU"):
        gk.gdn_replay_fp8(z(B, HV, 128, 128, dtype=torch.float8_e4m3fn), z(B, HV, 4, dtype=torch.float16),
                          z(B, H, 128), z(B, L, H, 128), z(B, L, HV, 128), z(B, L, HV), z(B, L, HV),
                          z(B, dtype=torch.int32), z(B, dtype=torch.bool))
    with pytest.raises(ValueError, match="GPU"):
        gk.quantize_checkpoint(torch.zeros(1, 1, 32, 128))


def _rmw_args(B=2, H=2, HV=4, V=128, K=128, state_dt=BF16, act=BF16):
    return {"state": desc([B, HV, V, K], state_dt), "q": desc([B, H, K], act), "k": desc([B, H, K], act),
            "v": desc([B, HV, V], act), "g": desc([B, HV], act), "beta": desc([B, HV], act),
            "out": desc([B, HV, V], act)}


def _rmw_call(lib, args):
    order = ["state", "q", "k", "v", "g", "beta", "out"]
    rc = lib.gdnr_bf16_step(*[ctypes.byref(args[n]) for n in order], None)
    return rc, lib.gdnr_last_error().decode()


@pytest.mark.parametrize("change,code,needle", [
    ({"state": desc([2, 4, 128, 64], BF16)}, UNSUPPORTED, "K=64"),
    ({"state": desc([2, 4, 100, 128], BF16)}, UNSUPPORTED, "V=100"),
    ({"state": desc([2, 4, 128, 128], I32)}, INVALID, "state"),
    ({"state": desc([2, 4, 128, 128], BF16, data=FAKE + 2)}, INVALID, "aligned"),
    ({"q": desc([2, 2, 128], F16)}, INVALID, "q"),
    ({"v": desc([2, 4, 96], BF16)}, INVALID, "v"),
    ({"k": desc([2, 3, 128], BF16)}, INVALID, "key heads"),
    ({"beta": desc([2, 4], BF16, strides=[8, 2])}, INVALID, "innermost"),
])
def test_bf16_step_rejects_misuse(lib, change, code, needle):
    args = _rmw_args()
    args.update(change)
    rc, msg = _rmw_call(lib, args)
    assert rc == code, msg
    assert needle in msg, msg


def test_bf16_step_empty_batch_is_a_no_op(lib):
    rc, msg = _rmw_call(lib, _rmw_args(B=0))
    assert rc == OK and msg == ""


def _slots_args(S=3, B=2, L=4, H=2, HV=4, K=128, V=128, idx_dt=I32):
    return [desc([B, 2 * H * K + HV * V], BF16), desc([B, HV], BF16), desc([B, HV], BF16), desc([HV], F32),
            desc([HV], F32), desc([B], I32), desc([B], idx_dt), desc([S, HV, V, K], FP8),
            desc([S, HV, V // 32], F16), desc([B, H, K], BF16), desc([S, L, H, K], BF16),
            desc([S, L, HV, V], BF16), desc([S, L, HV], BF16), desc([S, L, HV], BF16), desc([B], I32),
            desc([B], BOOL), desc([B, HV, V], BF16)]


def _slots_call(lib, args, block_v=128):
    rc = lib.gdnr_prep_replay_fp8_slots(*[ctypes.byref(t) for t in args], block_v, None)
    return rc, lib.gdnr_last_error().decode()


@pytest.mark.parametrize("kwargs,code,needle", [
    ({"L": 65}, UNSUPPORTED, "ring length 65 outside [1, 64]"),
    ({"idx_dt": I64}, INVALID, "state_indices"),
    ({"S": 0}, INVALID, "null slot"),
])
def test_slots_step_rejects_misuse(lib, kwargs, code, needle):
    rc, msg = _slots_call(lib, _slots_args(**kwargs))
    assert rc == code, msg
    assert needle in msg, msg


def test_slots_step_batch_shape_is_checked(lib):
    args = _slots_args()
    args[16] = desc([3, 4, 128], BF16)  # out with 3 rows for a batch of 2
    rc, msg = _slots_call(lib, args)
    assert rc == INVALID and "out" in msg


def test_slots_step_empty_batch_is_a_no_op(lib):
    rc, msg = _slots_call(lib, _slots_args(B=0))
    assert rc == OK and msg == ""



def _packed_args(S=3, B=2, H=2, HV=4, K=128, V=128, act=BF16, gate=BF16, idx_dt=I32, width=None):
    return {"mixed": desc([B, width or 2 * H * K + HV * V], act), "a": desc([B, HV], gate),
            "b": desc([B, HV], gate), "a_log": desc([HV], F32), "dt_bias": desc([HV], F32),
            "state": desc([S, HV, V, K], BF16), "idx": desc([B], idx_dt), "out": desc([B, 1, HV, V], act)}


def _packed_call(lib, args, scale=128 ** -0.5):
    order = ["mixed", "a", "b", "a_log", "dt_bias", "state", "idx", "out"]
    rc = lib.gdnr_bf16_step_packed(*[ctypes.byref(args[n]) for n in order], scale, None)
    return rc, lib.gdnr_last_error().decode()


@pytest.mark.parametrize("kwargs,change,code,needle", [
    ({"width": 2 * 2 * 128 + 4 * 128 + 64}, {}, INVALID, "2 H K + HV V"),
    ({"H": 3, "width": 2 * 3 * 128 + 4 * 128}, {}, INVALID, "key heads"),
    ({"gate": F16}, {}, INVALID, "a/b"),
    ({"idx_dt": I64}, {}, INVALID, "state_indices"),
    ({"S": 0}, {}, INVALID, "null slot"),
    ({}, {"out": desc([2, 4, 128], BF16)}, INVALID, "out"),
    ({}, {"a_log": desc([4], BF16)}, INVALID, "a_log"),
    ({}, {"state": desc([3, 4, 128, 64], BF16)}, UNSUPPORTED, "K=64"),
])
def test_packed_step_rejects_misuse(lib, kwargs, change, code, needle):
    args = _packed_args(**kwargs)
    args.update(change)
    rc, msg = _packed_call(lib, args)
    assert rc == code, msg
    assert needle in msg, msg


@pytest.mark.parametrize("scale", [float("nan"), float("inf")])
def test_packed_step_rejects_a_non_finite_scale(lib, scale):
    rc, msg = _packed_call(lib, _packed_args(), scale)
    assert rc == INVALID and "scale" in msg, msg


def test_packed_step_empty_batch_is_a_no_op(lib):
    rc, msg = _packed_call(lib, _packed_args(B=0))
    assert rc == OK and msg == ""
