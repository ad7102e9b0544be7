"""Capture records of the production GDN decode op: the file format the
reference's capture hook writes and its full-contract bench reads, for runs on
real decode inputs when a capture is available (none ships with the reference).

Format (prototype/qwen35_capture_raw.py:100-130, written with torch.save): a
dict {layer index: record}, each record a dict of
  "mixed_qkv"        list over steps of [1, 2*H*K + HV*V] bf16 tensors
  "a", "b"           lists over steps of [1, HV] f32 tensors
  "production_out"   list over steps of [1, HV*V] bf16 tensors (the production op's output)
  "state"            [1, HV, V, K] f32, the recurrent state before the first step (or None)
  "a_log", "dt_bias" [HV] f32
  "scale"            float (the op's output scale)
  "use_qk_l2norm_in_kernel"  bool
The consumer (prototype/bench_gdn_full_contract.py:83-110) replicates one
layer's batch-1 record across the batch. Records are loaded here with
torch.load(weights_only=True), which restores tensors, lists, dicts and
scalars and executes nothing from the file.
"""

from __future__ import annotations

from pathlib import Path

import torch

LIST_KEYS = ("mixed_qkv", "a", "b", "production_out")
REQUIRED_KEYS = LIST_KEYS + ("state", "a_log", "dt_bias", "scale", "use_qk_l2norm_in_kernel")


class CaptureFormatError(ValueError):
    """The file is not a capture in the format above."""


def _check_record(layer, record) -> None:
    if not isinstance(record, dict):
        raise CaptureFormatError(f"layer {layer}: record is {type(record).__name__}, not a dict")
    missing = [k for k in REQUIRED_KEYS if k not in record]
    if missing:
        raise CaptureFormatError(f"layer {layer}: missing keys {missing}")
    steps = len(record["mixed_qkv"])
    for k in LIST_KEYS:
        if not isinstance(record[k], list) or len(record[k]) != steps:
            raise CaptureFormatError(f"layer {layer}: {k} must be a list of {steps} per-step tensors")
        for t in record[k]:
            if not isinstance(t, torch.Tensor) or t.dim() != 2 or t.shape[0] != 1:
                raise CaptureFormatError(f"layer {layer}: {k} entries must be [1, n] tensors")
    hv = record["a_log"].numel()
    for k in ("a", "b"):
        if any(t.shape[1] != hv for t in record[k]):
            raise CaptureFormatError(f"layer {layer}: {k} entries must be [1, {hv}]")
    if record["dt_bias"].numel() != hv:
        raise CaptureFormatError(f"layer {layer}: dt_bias must have {hv} entries")
    state = record["state"]
    if state is not None and (state.dim() != 4 or state.shape[0] != 1 or state.shape[1] != hv):
        raise CaptureFormatError(f"layer {layer}: state must be [1, {hv}, V, K]")
    # the fused step applies an in-kernel q/k L2 norm and the output scale
    # K^-1/2 (kernel:534-562, ref:166-186); a record made otherwise runs other
    # maths than its production_out
    if record["use_qk_l2norm_in_kernel"] is not True:
        raise CaptureFormatError(f"layer {layer}: use_qk_l2norm_in_kernel must be true (the step normalises q/k)")
    if state is not None:
        V, K = state.shape[2], state.shape[3]
        if abs(float(record["scale"]) - K ** -0.5) > 1e-6 * K ** -0.5:
            raise CaptureFormatError(f"layer {layer}: scale {record['scale']} is not K^-1/2 = {K ** -0.5} (K={K})")
        width = record["mixed_qkv"][0].shape[1] if steps else 0
        qk = width - hv * V
        if steps and (qk <= 0 or qk % (2 * K) or hv % (qk // (2 * K))):
            raise CaptureFormatError(f"layer {layer}: mixed_qkv width {width} is not 2 H K + HV V with K={K}, "
                                     f"HV={hv}, V={V} and H dividing HV")
        if any(t.shape[1] != width for t in record["mixed_qkv"]):
            raise CaptureFormatError(f"layer {layer}: mixed_qkv entries differ in width")
        if any(t.shape[1] != hv * V for t in record["production_out"]):
            raise CaptureFormatError(f"layer {layer}: production_out entries must be [1, HV V] = [1, {hv * V}]")


def load_capture(path: str | Path) -> dict:
    """Load and check a capture file; returns {layer: record} on the CPU."""
    records = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(records, dict) or not records:
        raise CaptureFormatError(f"{path}: not a non-empty dict of layer records")
    for layer, record in records.items():
        _check_record(layer, record)
    return records


def save_capture(path: str | Path, records: dict) -> None:
    """Write records in the capture format (checked first)."""
    for layer, record in records.items():
        _check_record(layer, record)
    torch.save(records, path)


def captured_inputs(records: dict, batch: int, layer: int, steps: int, device) -> dict:
    """One layer's first ``steps`` decode inputs, replicated across ``batch``
    sequences (bench_gdn_full_contract.py:83-110): mixed_qkv [B,T,D] bf16,
    a, b [B,T,HV] f32, a_log, dt_bias [HV] f32, state [B,HV,V,K] f32,
    production_out [T, HV*V] bf16, scale, source."""
    record = records[layer]
    if record["state"] is None:
        raise CaptureFormatError(f"layer {layer}: the capture holds no pre-state")
    steps = min(steps, len(record["mixed_qkv"]))
    if steps < 1:
        raise CaptureFormatError(f"layer {layer}: no steps captured")

    def stacked(key, dtype):
        return torch.stack([t[0] for t in record[key][:steps]]).to(device=device, dtype=dtype)

    def per_batch(x):
        return x.unsqueeze(0).expand(batch, *x.shape).contiguous()

    return {
        "mixed_qkv": per_batch(stacked("mixed_qkv", torch.bfloat16)),
        "a": per_batch(stacked("a", torch.float32)),
        "b": per_batch(stacked("b", torch.float32)),
        "a_log": record["a_log"].to(device=device, dtype=torch.float32),
        "dt_bias": record["dt_bias"].to(device=device, dtype=torch.float32),
        "state": per_batch(record["state"][0].to(device=device, dtype=torch.float32)),
        "production_out": stacked("production_out", torch.bfloat16),
        "scale": float(record["scale"]),
        "source": f"capture:layer{layer}",
    }
