"""The capture record format (gdn_replayssm_capture; writer
prototype/qwen35_capture_raw.py:100-130, reader
prototype/bench_gdn_full_contract.py:83-110) on the CPU: a written record
loads back with torch.load(weights_only=True), one layer's inputs replicate
across the batch unchanged, malformed records are refused, and a file holding
a non-tensor object is refused without executing anything from it."""

from __future__ import annotations

import pickle

import pytest
import torch

import gdn_replayssm_capture as cap

H, HV, K, V, T = 2, 4, 128, 128, 5


def _record(seed=0):
    g = torch.Generator().manual_seed(seed)
    return {
        "mixed_qkv": [torch.randn(1, 2 * H * K + HV * V, generator=g).to(torch.bfloat16) for _ in range(T)],
        "a": [torch.randn(1, HV, generator=g) for _ in range(T)],
        "b": [torch.randn(1, HV, generator=g) for _ in range(T)],
        "production_out": [torch.randn(1, HV * V, generator=g).to(torch.bfloat16) for _ in range(T)],
        "state": 0.02 * torch.randn(1, HV, V, K, generator=g),
        "a_log": torch.rand(HV, generator=g),
        "dt_bias": torch.rand(HV, generator=g) - 4.0,
        "scale": K ** -0.5,
        "use_qk_l2norm_in_kernel": True,
    }


def test_round_trip_and_replication(tmp_path):
    rec = _record()
    path = tmp_path / "capture.pt"
    cap.save_capture(path, {3: rec})
    records = cap.load_capture(path)
    got = cap.captured_inputs(records, batch=3, layer=3, steps=4, device="cpu")
    assert got["mixed_qkv"].shape == (3, 4, 2 * H * K + HV * V) and got["mixed_qkv"].dtype == torch.bfloat16
    assert got["a"].shape == (3, 4, HV) and got["state"].shape == (3, HV, V, K)
    assert got["production_out"].shape == (4, HV * V)
    for bi in range(3):
        assert torch.equal(got["mixed_qkv"][bi], torch.cat(rec["mixed_qkv"][:4]))
        assert torch.equal(got["b"][bi], torch.cat(rec["b"][:4]))
        assert torch.equal(got["state"][bi], rec["state"][0])
    assert got["scale"] == K ** -0.5
    # more steps than captured: the capture's length
    assert cap.captured_inputs(records, 1, 3, 99, "cpu")["a"].shape[1] == T


@pytest.mark.parametrize("break_it,needle", [
    (lambda r: r.pop("dt_bias"), "missing"),
    (lambda r: r["a"].pop(), "list of"),
    (lambda r: r.__setitem__("state", torch.zeros(1, HV + 1, V, K)), "state"),
    (lambda r: r["b"].__setitem__(0, torch.zeros(1, HV + 2)), "b entries"),
    (lambda r: r.__setitem__("use_qk_l2norm_in_kernel", False), "use_qk_l2norm_in_kernel"),
    (lambda r: r.__setitem__("scale", 1.0), "K\\^-1/2"),
    (lambda r: r.__setitem__("mixed_qkv", [torch.zeros(1, 2 * H * K + HV * V + 64) for _ in range(T)]), "mixed_qkv width"),
    (lambda r: r.__setitem__("mixed_qkv", [torch.zeros(1, 2 * 3 * K + HV * V) for _ in range(T)]), "mixed_qkv width"),
    (lambda r: r["mixed_qkv"].__setitem__(2, torch.zeros(1, 2 * H * K + HV * V + 256)), "differ in width"),
    (lambda r: r["production_out"].__setitem__(1, torch.zeros(1, HV * V - 1)), "production_out"),
])
def test_malformed_records_are_refused(tmp_path, break_it, needle):
    rec = _record()
    break_it(rec)
    path = tmp_path / "bad.pt"
    torch.save({0: rec}, path)
    with pytest.raises(cap.CaptureFormatError, match=needle):
        cap.load_capture(path)


class _NotATensor:
    def __reduce__(self):
        return (print, ("this must never run",))


def test_non_tensor_objects_are_not_loaded(tmp_path, capsys):
    path = tmp_path / "evil.pt"
    torch.save({0: {"x": _NotATensor()}}, path)
    with pytest.raises(pickle.UnpicklingError):
        cap.load_capture(path)
    assert "this must never run" not in capsys.readouterr().out
