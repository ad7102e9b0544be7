"""MI355X (gfx950) ReplaySSM GDN decode path -- drop-in operator API.

Same module name, function names, argument order, defaults and return values
as the reference operator module (prototype/gdn_replayssm_fp8_kernel.py), so
a caller swaps the import and nothing else:

    gdn_replay_fp8        reference :344-405
    gdn_replay_fp8_split  reference :1129-1235
    gdn_prep_ring         reference :710-795
    gdn_bf16_step         reference :408-450 (the bf16 read-modify-write comparator)

plus the checkpoint constructors callers take from the reference's
gdn_replay_fp8_reference.py (QuantizedCheckpoint / quantize_checkpoint /
dequantize_checkpoint, ref:21-134; vblock/32 on the device) and one fused
entry point this build adds, gdn_prep_replay_fp8 (prep + replay/flush in one
launch).

Every function launches hand-written HIP kernels through libgdnreplay.so on
torch's current stream; none synchronises. Triton tuning knobs (num_warps,
num_stages) are accepted and ignored; block_v selects the V-rows a
workgroup streams (results do not depend on it). Unlike the reference,
arguments are validated: misuse raises instead of writing out of bounds.
Differences in accepted dtypes: valid_len/pos are converted to int32 and
flush to bool when given otherwise (one small device op each).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

import gdnr_lib

__all__ = [
    "QuantizedCheckpoint",
    "quantize_checkpoint",
    "dequantize_checkpoint",
    "gdn_replay_fp8",
    "gdn_replay_fp8_split",
    "gdn_prep_ring",
    "gdn_prep_replay_fp8",
    "gdn_bf16_step",
    "gdn_bf16_step_packed",
]

FP8_DTYPE = torch.float8_e4m3fn
VBLOCK = 32


def _require_cuda(**tensors: torch.Tensor | None) -> torch.device:
    device = None
    for name, t in tensors.items():
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"{name} must be a tensor on the GPU")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"{name} is on {t.device}, expected {device}")
    return device


def _as_i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def _as_flag(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype in (torch.bool, torch.uint8) else (t != 0)


# ---------------------------------------------------------------------------
# Checkpoint format (reference ref:21-134)
# ---------------------------------------------------------------------------

@dataclass
class QuantizedCheckpoint:
    """Same fields as the reference container (ref:21-33)."""

    payload: torch.Tensor
    scale: torch.Tensor
    granularity: str
    tile_size: int
    saturation_fraction: float

    @property
    def storage_bytes(self) -> int:
        return self.payload.numel() * self.payload.element_size() + self.scale.numel() * self.scale.element_size()


GRANULARITY_CODES = {"head": 0, "row": 1, "tile": 2, "vblock": 3}


def _format(granularity: str) -> tuple[str, int, bool]:
    is_int8 = granularity.endswith("_int8")
    base = granularity[: -len("_int8")] if is_int8 else granularity
    if base not in GRANULARITY_CODES:
        raise ValueError(f"unsupported granularity: {granularity}")
    return base, GRANULARITY_CODES[base], is_int8


def _scale_shape(base: str, batch: int, heads: int, value_dim: int, key_dim: int, tile_size: int) -> tuple:
    if base == "head":
        return (batch, heads, 1, 1)
    if base == "row":
        return (batch, heads, value_dim, 1)
    if base == "tile":
        return (batch, heads, value_dim // tile_size, key_dim // tile_size)
    return (batch, heads, value_dim // tile_size)


def quantize_checkpoint(state: torch.Tensor, granularity: str = "vblock", tile_size: int = VBLOCK,
                        saturation: bool = True) -> QuantizedCheckpoint:
    """Device quantiser, bit-exact with ref:40-106 for every format: granularity
    "head", "row", "tile" or "vblock" (tile_size for the last two), with
    "_int8" for int8 codes. Per scale group: scale = fp16(amax/qmax) (1 where
    amax is not > 0; qmax 448, or 127 for int8); payload = e4m3fn or
    round-half-even int8 of clamp(state / s), where s is the unrounded
    amax/qmax for tile and vblock and the fp16 scale for head and row. The
    decode path reads "vblock"/32 (its own fast quantiser).

    ``saturation=False`` skips the host read-back of saturation_fraction
    (which synchronises, like the reference's ``.item()``) and reports 0.
    """
    base, code, is_int8 = _format(granularity)
    device = _require_cuda(state=state)
    state32 = state if state.dtype == torch.float32 else state.float()
    if state32.dim() != 4:
        raise ValueError("state must be [B, HV, V, K]")
    batch, heads, value_dim, key_dim = state32.shape
    if base in ("tile", "vblock") and (value_dim % tile_size or (base == "tile" and key_dim % tile_size)):
        raise ValueError(f"{base} granularity requires dimensions divisible by tile_size")
    payload = torch.empty(state32.shape, dtype=torch.int8 if is_int8 else FP8_DTYPE, device=device)
    scale = torch.empty(_scale_shape(base, batch, heads, value_dim, key_dim, tile_size), dtype=torch.float16,
                        device=device)
    saturated = torch.empty(scale.shape, dtype=torch.int32, device=device) if saturation else None
    with torch.cuda.device(device):
        if base == "vblock" and tile_size == VBLOCK and not is_int8:
            gdnr_lib.call("gdnr_quantize_vblock32", [state32, payload, scale, saturated],
                          stream=gdnr_lib.current_stream(device))
        else:
            gdnr_lib.call("gdnr_quantize_checkpoint", [state32, payload, scale, saturated], [code, tile_size],
                          gdnr_lib.current_stream(device))
    fraction = float(saturated.sum().item()) / max(state32.numel(), 1) if saturation else 0.0
    return QuantizedCheckpoint(payload, scale, granularity, tile_size, fraction)


def dequantize_checkpoint(checkpoint: QuantizedCheckpoint) -> torch.Tensor:
    """ref:109-134 for every format: float(payload) * float(scale), the scale
    broadcast over its group."""
    base, code, _ = _format(checkpoint.granularity)
    device = _require_cuda(payload=checkpoint.payload, scale=checkpoint.scale)
    out = torch.empty(checkpoint.payload.shape, dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        if base == "vblock" and checkpoint.tile_size == VBLOCK and checkpoint.payload.dtype != torch.int8:
            gdnr_lib.call("gdnr_dequantize_vblock32", [checkpoint.payload, checkpoint.scale, out],
                          stream=gdnr_lib.current_stream(device))
        else:
            gdnr_lib.call("gdnr_dequantize_checkpoint", [checkpoint.payload, checkpoint.scale, out],
                          [code, checkpoint.tile_size], gdnr_lib.current_stream(device))
    return out


# ---------------------------------------------------------------------------
# Operators
# ---------------------------------------------------------------------------

def _new_out(q: torch.Tensor, v_cache: torch.Tensor) -> torch.Tensor:
    batch, _, value_heads, value_dim = v_cache.shape
    return torch.empty(batch, value_heads, value_dim, dtype=q.dtype, device=q.device)


def gdn_replay_fp8(
    checkpoint: torch.Tensor,
    checkpoint_scale: torch.Tensor,
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    g_cache: torch.Tensor,
    beta_cache: torch.Tensor,
    valid_len: torch.Tensor,
    flush: torch.Tensor,
    block_v: int = 32,
    num_warps: int = 4,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One replay step (reference kernel:344-405). For sequences with
    flush[b] == 0: adjoint replay of ring tokens [0, valid_len[b]) against the
    dequantised checkpoint, o = (S q) K^-1/2. For flush[b] != 0: forward
    rebuild, emit, and requantise checkpoint[b]/checkpoint_scale[b] in place
    (reference quantiser semantics, ref:36-37,83-99). Returns out [B,HV,V]
    (allocated with q's dtype when not given)."""
    del num_warps
    device = _require_cuda(checkpoint=checkpoint, checkpoint_scale=checkpoint_scale, q=q, k_cache=k_cache,
                           v_cache=v_cache, g_cache=g_cache, beta_cache=beta_cache, valid_len=valid_len,
                           flush=flush, out=out)
    output = _new_out(q, v_cache) if out is None else out
    with torch.cuda.device(device):
        gdnr_lib.call("gdnr_replay_fp8",
                      [checkpoint, checkpoint_scale, q, k_cache, v_cache, g_cache, beta_cache,
                       _as_i32(valid_len), _as_flag(flush), output],
                      [block_v], gdnr_lib.current_stream(device))
    return output


def gdn_replay_fp8_split(
    checkpoint: torch.Tensor,
    checkpoint_scale: torch.Tensor,
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    g_cache: torch.Tensor,
    beta_cache: torch.Tensor,
    valid_len: torch.Tensor,
    transformed_query_buffer: torch.Tensor,
    coefficient_buffer: torch.Tensor,
    block_v: int = 32,
    num_warps: int = 4,
    block_kc: int = 128,
    precompute_grouped: bool = True,
    num_stages: int = 2,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Non-flush replay as precompute + apply (reference kernel:1129-1235):
    writes T_0 into transformed_query_buffer [B,HV,K] f32 and c_t into
    coefficient_buffer [B,HV,>=L] f32 (t < valid_len only), then streams the
    checkpoint. Same output as gdn_replay_fp8 with flush = 0."""
    del num_warps, num_stages
    device = _require_cuda(checkpoint=checkpoint, checkpoint_scale=checkpoint_scale, q=q, k_cache=k_cache,
                           v_cache=v_cache, g_cache=g_cache, beta_cache=beta_cache, valid_len=valid_len,
                           transformed_query_buffer=transformed_query_buffer,
                           coefficient_buffer=coefficient_buffer, out=out)
    output = _new_out(q, v_cache) if out is None else out
    with torch.cuda.device(device):
        gdnr_lib.call("gdnr_replay_fp8_split",
                      [checkpoint, checkpoint_scale, q, k_cache, v_cache, g_cache, beta_cache,
                       _as_i32(valid_len), transformed_query_buffer, coefficient_buffer, output],
                      [block_v, block_kc, int(bool(precompute_grouped))], gdnr_lib.current_stream(device))
    return output


def gdn_prep_ring(
    mixed_qkv: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    pos: torch.Tensor,
    q_out: torch.Tensor,
    k_ring: torch.Tensor,
    v_ring: torch.Tensor,
    g_ring: torch.Tensor,
    beta_ring: torch.Tensor,
    num_warps: int = 1,
    fused: bool = True,
) -> None:
    """Full-contract preparation (reference kernel:710-795): q,k <-
    x/sqrt(sum x^2 + 1e-6); q -> q_out; k, v, g = -exp(A_log) softplus_20(a +
    dt_bias), beta = sigmoid(b) -> ring slot pos[b]. A_log and dt_bias are
    read as float32 (converted when given otherwise)."""
    del num_warps
    device = _require_cuda(mixed_qkv=mixed_qkv, a=a, b=b, a_log=a_log, dt_bias=dt_bias, pos=pos, q_out=q_out,
                           k_ring=k_ring, v_ring=v_ring, g_ring=g_ring, beta_ring=beta_ring)
    with torch.cuda.device(device):
        gdnr_lib.call("gdnr_prep_ring",
                      [mixed_qkv, a, b, a_log.float(), dt_bias.float(), _as_i32(pos), q_out, k_ring, v_ring,
                       g_ring, beta_ring],
                      [int(bool(fused))], gdnr_lib.current_stream(device))


def gdn_prep_replay_fp8(
    mixed_qkv: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    pos: torch.Tensor,
    checkpoint: torch.Tensor,
    checkpoint_scale: torch.Tensor,
    q_out: torch.Tensor,
    k_ring: torch.Tensor,
    v_ring: torch.Tensor,
    g_ring: torch.Tensor,
    beta_ring: torch.Tensor,
    valid_len: torch.Tensor,
    flush: torch.Tensor,
    block_v: int = 128,
    out: torch.Tensor | None = None,
    state_indices: torch.Tensor | None = None,
) -> torch.Tensor:
    """The full-contract decode step in one launch: exactly
    gdn_prep_ring(...) followed by gdn_replay_fp8(checkpoint, checkpoint_scale,
    q_out, k_ring, v_ring, g_ring, beta_ring, valid_len, flush, block_v),
    as sequenced by the reference's prototype/bench_gdn_full_contract.py:138-154
    and :246-297, with identical results.

    With state_indices [B] (int32 on the device), the checkpoint, scale and
    rings are a slot-indexed cache [S, ...] (vLLM's layout, slot 0 the null
    slot) and batch entry b uses slot state_indices[b]; the other arguments
    stay per batch entry (gdnr_prep_replay_fp8_slots)."""
    device = _require_cuda(mixed_qkv=mixed_qkv, a=a, b=b, a_log=a_log, dt_bias=dt_bias, pos=pos,
                           checkpoint=checkpoint, checkpoint_scale=checkpoint_scale, q_out=q_out, k_ring=k_ring,
                           v_ring=v_ring, g_ring=g_ring, beta_ring=beta_ring, valid_len=valid_len, flush=flush,
                           out=out, state_indices=state_indices)
    batch = mixed_qkv.shape[0]
    output = (torch.empty(batch, v_ring.shape[2], v_ring.shape[3], dtype=q_out.dtype, device=device)
              if out is None else out)
    with torch.cuda.device(device):
        if state_indices is None:
            gdnr_lib.call("gdnr_prep_replay_fp8",
                          [mixed_qkv, a, b, a_log.float(), dt_bias.float(), _as_i32(pos), checkpoint,
                           checkpoint_scale, q_out, k_ring, v_ring, g_ring, beta_ring, _as_i32(valid_len),
                           _as_flag(flush), output],
                          [block_v], gdnr_lib.current_stream(device))
        else:
            gdnr_lib.call("gdnr_prep_replay_fp8_slots",
                          [mixed_qkv, a, b, a_log.float(), dt_bias.float(), _as_i32(pos), _as_i32(state_indices),
                           checkpoint, checkpoint_scale, q_out, k_ring, v_ring, g_ring, beta_ring,
                           _as_i32(valid_len), _as_flag(flush), output],
                          [block_v], gdnr_lib.current_stream(device))
    return output


def gdn_bf16_step(
    state: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
) -> torch.Tensor:
    """One gated delta-rule token on a state held in full, updated in place
    (reference kernel:408-450, device work :245-341): S <- exp(g) S;
    r = S k; S <- S + beta (v - r) k^T; returns (S q) K^-1/2 as [B,HV,V] in
    q's dtype. state [B,HV,V,K] (bf16, f16 or f32); q, k [B,H,K];
    v [B,HV,V]; g, beta [B,HV] -- views with unit inner stride are taken as
    they are (the reference passes ring slices, bench_gdn_replayssm.py:278-287)."""
    device = _require_cuda(state=state, q=q, k=k, v=v, g=g, beta=beta)
    output = torch.empty(state.shape[0], state.shape[1], state.shape[2], dtype=q.dtype, device=device)
    with torch.cuda.device(device):
        gdnr_lib.call("gdnr_bf16_step", [state, q, k, v, g, beta, output], [], gdnr_lib.current_stream(device))
    return output


def gdn_bf16_step_packed(
    mixed_qkv: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    a_log: torch.Tensor,
    dt_bias: torch.Tensor,
    initial_state: torch.Tensor,
    ssm_state_indices: torch.Tensor,
    out: torch.Tensor | None = None,
    scale: float | None = None,
) -> torch.Tensor:
    """The bf16 read-modify-write comparator in the production operator's
    contract (findings.md:35-45): q/k L2 norm and gating in the kernel,
    initial_state [slots, HV, V, K] updated in place at slot
    ssm_state_indices[b] (slot 0 the null slot), out [B, 1, HV, V] =
    scale (S q); scale defaults to head_k_dim ** -0.5, as vLLM passes it."""
    device = _require_cuda(mixed_qkv=mixed_qkv, a=a, b=b, a_log=a_log, dt_bias=dt_bias,
                           initial_state=initial_state, ssm_state_indices=ssm_state_indices, out=out)
    batch = mixed_qkv.shape[0]
    if out is None:
        out = torch.empty(batch, 1, initial_state.shape[1], initial_state.shape[2], dtype=mixed_qkv.dtype,
                          device=device)
    with torch.cuda.device(device):
        gdnr_lib.call("gdnr_bf16_step_packed", [mixed_qkv, a, b, a_log.float(), dt_bias.float(), initial_state,
                                                _as_i32(ssm_state_indices), out], [],
                      gdnr_lib.current_stream(device),
                      floats=[initial_state.shape[-1] ** -0.5 if scale is None else scale])
    return out

