"""CPU restatement (numpy) of the reference ReplaySSM GDN decode algorithm.

TEST INFRASTRUCTURE ONLY. This module is the checker the HIP path is compared
against. It may be imported by ``tests/``, by ``__graft_entry__.smoke()`` and by
the ``cpu_baseline`` leg of ``bench.py`` -- never by the product package, which
must fail loudly when its HIP library is missing instead of falling back here.

Every function restates the reference's algorithm from its source text; the
citation after each name is the reference file:line it follows
(``ref`` = ``prototype/gdn_replay_fp8_reference.py``,
``kernel`` = ``prototype/gdn_replayssm_fp8_kernel.py``, both under the
reference repository root). How each function is pinned -- golden fixtures,
library casts, closed forms, invariants, brute force -- is stated in its
docstring and exercised by ``tests/test_oracle_*.py``.

Arrays follow the reference layouts:
  state / checkpoint  [B, HV, V, K]     q         [B, H, K]  (or [B, T, H, K])
  k ring              [B, L, H, K]      v ring    [B, L, HV, V]
  g / beta rings      [B, L, HV]        out       [B, HV, V]
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

FP8_MAX = 448.0  # torch.finfo(torch.float8_e4m3fn).max, ref:17-18
INT8_MAX = 127.0  # ref:46
VBLOCK = 32  # rows per checkpoint scale, kernel:401
L2_EPS = 1e-6  # kernel:756
SOFTPLUS_THRESHOLD = 20.0  # kernel:757


# --------------------------------------------------------------------------
# Number formats (pinned against torch's CPU casts and the C restatement in
# oracle/fp8_quant.c; see tests/test_oracle_formats.py)
# --------------------------------------------------------------------------

def _build_e4m3fn_table() -> np.ndarray:
    """Value of every OCP e4m3fn code (S.EEEE.MMM, bias 7, 0x7F/0xFF = NaN)."""
    table = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exponent = (code >> 3) & 0xF
        mantissa = code & 0x7
        if exponent == 0xF and mantissa == 0x7:
            table[code] = np.nan
        elif exponent == 0:
            table[code] = sign * mantissa * 2.0 ** -9
        else:
            table[code] = sign * (1.0 + mantissa / 8.0) * 2.0 ** (exponent - 7)
    return table


E4M3FN_TABLE = _build_e4m3fn_table()


def e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values (exact)."""
    return E4M3FN_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3fn_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn codes, round-to-nearest-even, like torch's
    ``tensor.to(torch.float8_e4m3fn)``: magnitudes above 464 (the midpoint
    between 448 and the NaN encoding), inf and NaN become 0x7F | sign.

    Normal results round the fp32 bit pattern at mantissa bit 20; subnormal
    results (|x| < 2^-6) are ``rint(|x| * 2^9)``.
    """
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint32)
    magnitude = bits & np.uint32(0x7FFFFFFF)
    ax = magnitude.view(np.float32)
    codes = np.zeros(x.shape, dtype=np.uint32)

    normal = ax >= np.float32(2.0 ** -6)
    mant_odd = (magnitude >> 20) & 1
    rounded = ((magnitude + np.uint32(0x7FFFF) + mant_odd) >> 20).astype(np.int64) - (120 << 3)
    codes = np.where(normal, np.clip(rounded, 0, 0x7F).astype(np.uint32), codes)

    sub = ~normal & ~np.isnan(ax)
    sub_codes = np.rint(np.where(sub, ax, 0).astype(np.float64) * 512.0).astype(np.uint32)
    codes = np.where(sub, sub_codes, codes)

    overflow = (ax > np.float32(464.0)) | np.isnan(ax)
    codes = np.where(overflow, np.uint32(0x7F), codes)
    return (codes | sign).astype(np.uint8)


def f16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even float16 (subnormals kept, overflow -> inf) -> float32."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round-to-nearest-even, NaN quietened."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    quiet = ((u >> 16) | 0x40).astype(np.uint16)
    return np.where(nan, quiet, rounded)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest-even bfloat16 -> float32."""
    return (bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values to a storage dtype ('bf16' | 'f16' | 'f32'); float32 out."""
    if dtype == "bf16":
        return bf16_round(np.asarray(x, dtype=np.float32))
    if dtype == "f16":
        return f16_round(x)
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(f"unknown dtype {dtype}")


# --------------------------------------------------------------------------
# Checkpoint formats: ref:21-134
# --------------------------------------------------------------------------

@dataclass
class QuantizedCheckpoint:
    """ref:21-33. ``payload`` holds e4m3fn codes (uint8) or int8 values;
    ``scale`` is float16."""

    payload: np.ndarray
    scale: np.ndarray
    granularity: str
    tile_size: int
    saturation_fraction: float

    @property
    def storage_bytes(self) -> int:  # ref:29-33
        return self.payload.size * self.payload.itemsize + self.scale.size * self.scale.itemsize


def safe_scale(amax: np.ndarray, quant_max: float) -> np.ndarray:
    """ref:36-37: amax/quant_max where amax > 0, else 1 (NaN amax -> 1)."""
    amax = np.asarray(amax, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        positive = amax > 0
    return np.where(positive, amax / np.float32(quant_max), np.float32(1.0)).astype(np.float32)


def _amax(x: np.ndarray, axis) -> np.ndarray:
    """|x| max that propagates NaN like torch.amax."""
    return np.max(np.abs(x), axis=axis, keepdims=True)


def quantize_checkpoint(state: np.ndarray, granularity: str = "vblock", tile_size: int = VBLOCK) -> QuantizedCheckpoint:
    """ref:40-106.

    Note the reference's asymmetry, kept bit for bit: for ``tile`` and
    ``vblock`` the payload is ``source / (amax/qmax)`` with the UNROUNDED fp32
    scale (ref:83-86,94) while the stored scale is its fp16 rounding (ref:87,91);
    ``head`` and ``row`` divide by the fp16-rounded scale (ref:92-93).
    """
    source = np.asarray(state, dtype=np.float32)
    is_int8 = granularity.endswith("_int8")
    base = granularity[: -len("_int8")] if is_int8 else granularity
    quant_max = INT8_MAX if is_int8 else FP8_MAX
    if base == "head":
        scale = safe_scale(_amax(source, (-2, -1)), quant_max)
        expanded = scale
    elif base == "row":
        scale = safe_scale(_amax(source, -1), quant_max)
        expanded = scale
    elif base == "tile":
        value_dim, key_dim = source.shape[-2:]
        if value_dim % tile_size or key_dim % tile_size:
            raise ValueError("tile granularity requires dimensions divisible by tile_size")
        blocks = source.reshape(*source.shape[:-2], value_dim // tile_size, tile_size, key_dim // tile_size, tile_size)
        block_scale = safe_scale(_amax(blocks, (-3, -1)), quant_max)
        expanded = np.broadcast_to(block_scale, blocks.shape).reshape(source.shape)
        scale = block_scale.squeeze(-1).squeeze(-2).astype(np.float16)
    elif base == "vblock":
        value_dim, key_dim = source.shape[-2:]
        if value_dim % tile_size:
            raise ValueError("vblock granularity requires value_dim divisible by tile_size")
        blocks = source.reshape(*source.shape[:-2], value_dim // tile_size, tile_size, key_dim)
        block_scale = safe_scale(_amax(blocks, (-2, -1)), quant_max)
        expanded = np.broadcast_to(block_scale, blocks.shape).reshape(source.shape)
        scale = block_scale.squeeze(-1).squeeze(-1).astype(np.float16)
    else:
        raise ValueError(f"unsupported granularity: {granularity}")

    scale = np.asarray(scale).astype(np.float16)
    if base in ("head", "row"):
        expanded = scale.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        normalized = (source / expanded.astype(np.float32)).astype(np.float32)
        saturation_fraction = float(np.mean(np.abs(normalized) > quant_max))
    if is_int8:
        clipped = np.clip(np.rint(normalized), -quant_max, quant_max)
        payload = np.where(np.isnan(clipped), 0, clipped).astype(np.int8)
    else:
        clipped = np.where(np.isnan(normalized), normalized, np.clip(normalized, -quant_max, quant_max))
        payload = e4m3fn_encode(clipped.astype(np.float32))
    return QuantizedCheckpoint(payload=payload, scale=scale, granularity=granularity,
                               tile_size=tile_size, saturation_fraction=saturation_fraction)


def dequantize_checkpoint(checkpoint: QuantizedCheckpoint) -> np.ndarray:
    """ref:109-134: payload.float() * scale.float(), broadcast per block."""
    base = checkpoint.granularity.removesuffix("_int8")
    if checkpoint.payload.dtype == np.uint8:
        values = e4m3fn_decode(checkpoint.payload)
    else:
        values = checkpoint.payload.astype(np.float32)
    scale = checkpoint.scale.astype(np.float32)
    if base in ("head", "row"):
        expanded = scale
    elif base == "tile":
        value_dim, key_dim = values.shape[-2:]
        ts = checkpoint.tile_size
        blocks_shape = (*values.shape[:-2], value_dim // ts, ts, key_dim // ts, ts)
        expanded = np.broadcast_to(scale[..., :, None, :, None], blocks_shape).reshape(values.shape)
    else:
        value_dim, key_dim = values.shape[-2:]
        ts = checkpoint.tile_size
        blocks_shape = (*values.shape[:-2], value_dim // ts, ts, key_dim)
        expanded = np.broadcast_to(scale[..., :, None, None], blocks_shape).reshape(values.shape)
    return (values * expanded).astype(np.float32)


def dequantize_vblock32(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Shortcut of dequantize_checkpoint for the vblock/32 format."""
    return dequantize_checkpoint(QuantizedCheckpoint(np.asarray(codes, dtype=np.uint8), np.asarray(scale), "vblock", VBLOCK, 0.0))


# --------------------------------------------------------------------------
# Recurrence: ref:137-244
# --------------------------------------------------------------------------

def run_kernel(state, q, k, v, g, beta, dtype=np.float32):
    """ref:137-163. Per-token gated delta rule from ``state``:
    S *= exp(g); r = S k; S += beta (v - r) k^T; o = (S q) K^-1/2, with q/k
    shared by the HV/H value heads of a key head (repeat_interleave).
    q, k [B,T,H,K]; v [B,T,HV,V]; g, beta [B,T,HV]. Returns ([B,T,HV,V], state).
    """
    scratch = np.array(state, dtype=dtype, copy=True)
    value_heads = v.shape[2]
    key_heads = k.shape[2]
    group = value_heads // key_heads
    scale = dtype(q.shape[-1] ** -0.5)
    outputs = []
    for token in range(q.shape[1]):
        q_t = np.repeat(np.asarray(q[:, token], dtype=dtype), group, axis=1)
        k_t = np.repeat(np.asarray(k[:, token], dtype=dtype), group, axis=1)
        v_t = np.asarray(v[:, token], dtype=dtype)
        decay = np.exp(np.asarray(g[:, token], dtype=dtype))[..., None, None]
        beta_t = np.asarray(beta[:, token], dtype=dtype)[..., None]
        scratch = scratch * decay
        retrieved = (scratch * k_t[:, :, None, :]).sum(axis=-1)
        correction = (v_t - retrieved) * beta_t
        scratch = scratch + correction[..., None] * k_t[:, :, None, :]
        output = (scratch * q_t[:, :, None, :]).sum(axis=-1) * scale
        outputs.append(output[:, None])
    return np.concatenate(outputs, axis=1), scratch


def baseline_decode(initial_state, q, k, v, g, beta, dtype=np.float32):
    """ref:166-186: run_kernel one token at a time."""
    state = np.array(initial_state, dtype=dtype, copy=True)
    outputs = []
    for token in range(q.shape[1]):
        sl = slice(token, token + 1)
        output, state = run_kernel(state, q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl], dtype)
        outputs.append(output)
    return np.concatenate(outputs, axis=1), state


def bf16_rmw_step(state, q, k, v, g, beta, state_dtype="bf16", out_dtype="bf16", dtype=np.float32, scale=None):
    """kernel:245-341 (host wrapper kernel:408-450): the full-state
    read-modify-write comparator. One token per sequence, in the kernel's
    order and fp32: S *= exp(g); r = sum_K(S k); c = (v - r) beta;
    S += c k^T; o = sum_K(S q) K^-1/2. S goes back in its storage dtype and
    o in the output dtype, both rounded to nearest even (round_to).
    state [B,HV,V,K]; q, k [B,H,K] (shared by the HV/H value heads of a key
    head); v [B,HV,V]; g, beta [B,HV]; scale (default K^-1/2) multiplies o.
    Returns (out, new_state) as float32
    arrays holding values of those dtypes. Pinned (tests/test_oracle_rmw.py):
    with f32 storage it is run_kernel's one-token step (ref:155-161); from a
    zero state it is S = beta v k^T, o = beta v (k . q) K^-1/2; beta = 0 is
    pure decay; the store rounding is round_to (pinned against torch)."""
    group = v.shape[1] // k.shape[1]
    s = np.asarray(state, dtype=dtype)
    k_t = np.repeat(np.asarray(k, dtype=dtype), group, axis=1)
    q_t = np.repeat(np.asarray(q, dtype=dtype), group, axis=1)
    s = s * np.exp(np.asarray(g, dtype=dtype))[..., None, None]
    retrieved = (s * k_t[:, :, None, :]).sum(axis=-1)
    correction = (np.asarray(v, dtype=dtype) - retrieved) * np.asarray(beta, dtype=dtype)[..., None]
    s = s + correction[..., None] * k_t[:, :, None, :]
    out = (s * q_t[:, :, None, :]).sum(axis=-1) * dtype(k.shape[-1] ** -0.5 if scale is None else scale)
    return round_to(out, out_dtype), round_to(s, state_dtype)


def replay_decode(initial_state, q, k, v, g, beta, window, granularity, tile_size=VBLOCK, dtype=np.float32):
    """ref:189-244. Each token: dequantise the checkpoint, replay the ring
    [ring_start, token] forward from it, emit the last output; when the ring
    holds ``window`` tokens the rebuilt state becomes the new checkpoint
    (requantised when ``granularity`` is not None) and the ring restarts.
    Returns (outputs [B,T,HV,V], final_state, max_saturation, checkpoint_bytes).
    """
    checkpoint = np.array(initial_state, dtype=dtype, copy=True)
    quantized = None
    max_saturation = 0.0
    if granularity is not None:
        quantized = quantize_checkpoint(checkpoint, granularity, tile_size)
    outputs = []
    ring_start = 0
    reconstructed = checkpoint
    for token in range(q.shape[1]):
        if quantized is not None:
            checkpoint = dequantize_checkpoint(quantized).astype(dtype)
        sl = slice(ring_start, token + 1)
        output, reconstructed = run_kernel(checkpoint, q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl], dtype)
        outputs.append(output[:, -1:])
        if token - ring_start + 1 == window:
            checkpoint = reconstructed
            if granularity is not None:
                quantized = quantize_checkpoint(checkpoint, granularity, tile_size)
                max_saturation = max(max_saturation, quantized.saturation_fraction)
            ring_start = token + 1
    final_state = reconstructed
    if quantized is not None and ring_start == q.shape[1]:
        final_state = dequantize_checkpoint(quantized)
    checkpoint_bytes = quantized.storage_bytes if quantized is not None else checkpoint.size * checkpoint.itemsize
    return np.concatenate(outputs, axis=1), final_state, max_saturation, checkpoint_bytes


def error_metrics(actual, expected) -> dict:
    """ref:247-259: max_abs, mean_abs, relative_l2 (denominator >= 1e-12), cosine."""
    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    delta = a - e
    denominator = max(float(np.linalg.norm(e)), 1e-12)
    cos_den = max(float(np.linalg.norm(a)) * float(np.linalg.norm(e)), 1e-8)
    return {
        "max_abs": float(np.max(np.abs(delta))) if delta.size else 0.0,
        "mean_abs": float(np.mean(np.abs(delta))) if delta.size else 0.0,
        "relative_l2": float(np.linalg.norm(delta)) / denominator,
        "cosine": float(np.dot(a, e)) / cos_den,
    }


def relative_l2(actual, expected) -> float:
    return error_metrics(actual, expected)["relative_l2"]


# --------------------------------------------------------------------------
# The fused kernel's semantics: kernel:20-242 (replay), kernel:798-1018 (split)
# --------------------------------------------------------------------------

def _clamp_len(valid_len, ring_len):
    return int(min(max(int(valid_len), 0), ring_len))


def adjoint_replay(state, q, k_cache, v_cache, g_cache, beta_cache, valid_len, dtype=np.float32):
    """kernel:121-176 (non-flush branch). For each sequence b, walk the ring
    backwards over t = valid_len-1 .. 0 carrying the transformed query T:
        c_t = beta_t (k_t . T);  o += c_t v_t;  T <- exp(g_t) (T - c_t k_t)
    then o += S_ckpt T and o *= K^-1/2. Tokens t >= valid_len are inactive.
    state is the dequantised checkpoint [B,HV,V,K]; q [B,H,K].
    Returns (out [B,HV,V], tq [B,HV,K], coef [B,HV,L]) where tq/coef are what
    the split precompute writes (kernel:849-896); coef is 0 for inactive t.
    """
    state = np.asarray(state, dtype=dtype)
    batch, ring_len, heads, key_dim = k_cache.shape
    value_heads, value_dim = v_cache.shape[2], v_cache.shape[3]
    group = value_heads // heads
    out = np.zeros((batch, value_heads, value_dim), dtype=dtype)
    tq = np.zeros((batch, value_heads, key_dim), dtype=dtype)
    coef = np.zeros((batch, value_heads, ring_len), dtype=dtype)
    for b in range(batch):
        n = _clamp_len(valid_len[b], ring_len)
        T = np.repeat(np.asarray(q[b], dtype=dtype), group, axis=0)
        o = np.zeros((value_heads, value_dim), dtype=dtype)
        for t in range(n - 1, -1, -1):
            k_t = np.repeat(np.asarray(k_cache[b, t], dtype=dtype), group, axis=0)
            v_t = np.asarray(v_cache[b, t], dtype=dtype)
            beta_t = np.asarray(beta_cache[b, t], dtype=dtype)
            decay = np.exp(np.asarray(g_cache[b, t], dtype=dtype))
            c = beta_t * (k_t * T).sum(axis=-1)
            coef[b, :, t] = c
            o = o + c[:, None] * v_t
            T = decay[:, None] * (T - c[:, None] * k_t)
        tq[b] = T
        o = o + (state[b] * T[:, None, :]).sum(axis=-1)
        out[b] = o * dtype(key_dim ** -0.5)
    return out, tq, coef


def forward_rebuild(state, q, k_cache, v_cache, g_cache, beta_cache, valid_len, dtype=np.float32):
    """kernel:177-228 (flush branch, before requantisation): forward
    recurrence over the active ring tokens from the dequantised checkpoint,
    then o = (S q) K^-1/2. Returns (out [B,HV,V], rebuilt state [B,HV,V,K])."""
    state = np.array(state, dtype=dtype, copy=True)
    batch, ring_len, heads, key_dim = k_cache.shape
    value_heads = v_cache.shape[2]
    group = value_heads // heads
    out = np.zeros((batch, value_heads, v_cache.shape[3]), dtype=dtype)
    for b in range(batch):
        n = _clamp_len(valid_len[b], ring_len)
        s = state[b]
        for t in range(n):
            k_t = np.repeat(np.asarray(k_cache[b, t], dtype=dtype), group, axis=0)
            v_t = np.asarray(v_cache[b, t], dtype=dtype)
            s = s * np.exp(np.asarray(g_cache[b, t], dtype=dtype))[:, None, None]
            retrieved = (s * k_t[:, None, :]).sum(axis=-1)
            s = s + ((v_t - retrieved) * np.asarray(beta_cache[b, t], dtype=dtype)[:, None])[..., None] * k_t[:, None, :]
        q_b = np.repeat(np.asarray(q[b], dtype=dtype), group, axis=0)
        out[b] = (s * q_b[:, None, :]).sum(axis=-1) * dtype(key_dim ** -0.5)
        state[b] = s
    return out, state


def replay_step(codes, scale, q, k_cache, v_cache, g_cache, beta_cache, valid_len, flush, dtype=np.float32):
    """One gdn_replay_fp8 call (kernel:344-405) on a vblock32 checkpoint, with
    the flush requantising through the REFERENCE quantiser (ref:40-106, not the
    Triton cast of kernel:229-236, whose divide-by-fp16-scale and 1e-12 floor
    differ). Returns (out float [B,HV,V], new codes, new scale).
    """
    dequant = dequantize_vblock32(codes, scale)
    out, _, _ = adjoint_replay(dequant, q, k_cache, v_cache, g_cache, beta_cache, valid_len, dtype)
    new_codes = np.array(codes, dtype=np.uint8, copy=True)
    new_scale = np.array(scale, copy=True)
    flush = np.asarray(flush).astype(bool)
    if flush.any():
        rows = np.nonzero(flush)[0]
        f_out, rebuilt = forward_rebuild(dequant[rows], q[rows], k_cache[rows], v_cache[rows],
                                         g_cache[rows], beta_cache[rows], np.asarray(valid_len)[rows], dtype)
        out[rows] = f_out
        requant = quantize_checkpoint(rebuilt.astype(np.float32), "vblock", VBLOCK)
        new_codes[rows] = requant.payload
        new_scale[rows] = requant.scale.astype(new_scale.dtype)
    return out, new_codes, new_scale


# --------------------------------------------------------------------------
# Full-contract preparation: kernel:453-576
# --------------------------------------------------------------------------

def softplus_thresholded(x):
    """kernel:560: log(1 + exp(x)) for x <= 20, else x -- the formula as the
    reference kernel writes it (not log1p), evaluated here in float64."""
    x = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        return np.where(x <= SOFTPLUS_THRESHOLD, np.log(1.0 + np.exp(np.minimum(x, SOFTPLUS_THRESHOLD))), x)


def prep_values(mixed_qkv, a, b, a_log, dt_bias, heads, key_dim, value_heads, value_dim):
    """kernel:504-562, computed in float64 (unrounded):
    q, k [B,H,K] = x / sqrt(sum x^2 + 1e-6) per key head; v [B,HV,V] copied;
    g = -exp(A_log) softplus_20(a + dt_bias); beta = sigmoid(b) [B,HV].
    mixed_qkv is [B, 2HK + HV V] laid out [q heads | k heads | v heads].
    """
    mixed = np.asarray(mixed_qkv, dtype=np.float64)
    batch = mixed.shape[0]
    hk = heads * key_dim
    q = mixed[:, :hk].reshape(batch, heads, key_dim)
    k = mixed[:, hk:2 * hk].reshape(batch, heads, key_dim)
    v = mixed[:, 2 * hk:2 * hk + value_heads * value_dim].reshape(batch, value_heads, value_dim)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True) + L2_EPS)
    k = k / np.sqrt((k * k).sum(-1, keepdims=True) + L2_EPS)
    x = np.asarray(a, dtype=np.float64) + np.asarray(dt_bias, dtype=np.float64)[None, :]
    g = -np.exp(np.asarray(a_log, dtype=np.float64))[None, :] * softplus_thresholded(x)
    beta = 1.0 / (1.0 + np.exp(-np.asarray(b, dtype=np.float64)))
    return q, k, v, g, beta


def packed_rmw_step(state, slots, mixed_qkv, a, b, a_log, dt_bias, heads, state_dtype="bf16", out_dtype="bf16",
                    scale=None):
    """The comparator in the production operator's contract (findings.md:35-45):
    prep_values (q/k L2 norm, gates; kernel:504-562) then bf16_rmw_step on the
    state of slot slots[i] of state [S,HV,V,K]. Slots outside [0, S) read slot
    0. Entries of slot 0 (the null slot, padding) are computed but not stored:
    the device lets them write the null slot in an unspecified order. The
    gates and normalised q/k enter the step in float32, as the kernel forms
    them. Returns (out [B,1,HV,V], new state [S,HV,V,K]) as float32 arrays
    holding values of the output / storage dtype. Pinned
    (tests/test_oracle_rmw.py): with slots 1..B in order it is bf16_rmw_step of
    the prepared values; permuting the batch permutes the outputs and leaves
    the stored states unchanged; untouched slots keep their bytes."""
    state = np.asarray(state, dtype=np.float32)
    value_heads, value_dim, key_dim = state.shape[1:]
    q, k, v, g, beta = prep_values(mixed_qkv, a, b, a_log, dt_bias, heads, key_dim, value_heads, value_dim)
    idx = np.asarray(slots, dtype=np.int64)
    idx = np.where((idx >= 0) & (idx < state.shape[0]), idx, 0)
    out, new = bf16_rmw_step(state[idx], q.astype(np.float32), k.astype(np.float32), v.astype(np.float32),
                             g.astype(np.float32), beta.astype(np.float32), state_dtype, out_dtype, scale=scale)
    result = state.copy()
    live = idx != 0
    result[idx[live]] = new[live]
    return out[:, None], result


def prep_ring(mixed_qkv, a, b, a_log, dt_bias, pos, q_out, k_ring, v_ring, g_ring, beta_ring, ring_dtype="bf16", q_dtype=None):
    """kernel:710-795 (gdn_prep_ring): write q_out and ring slot pos[b] of every
    ring, rounding to the storage dtype. Arrays are float32 numpy arrays holding
    storage-dtype values; they are modified in place. A pos outside the ring
    appends nothing (the reference would write out of bounds)."""
    heads, key_dim = q_out.shape[1], q_out.shape[2]
    value_heads, value_dim = v_ring.shape[2], v_ring.shape[3]
    q, k, v, g, beta = prep_values(mixed_qkv, a, b, a_log, dt_bias, heads, key_dim, value_heads, value_dim)
    q_out[...] = round_to(q.astype(np.float32), q_dtype or ring_dtype)
    ring_len = k_ring.shape[1]
    for i in range(q_out.shape[0]):
        p = int(pos[i])
        if not 0 <= p < ring_len:
            continue
        k_ring[i, p] = round_to(k[i].astype(np.float32), ring_dtype)
        v_ring[i, p] = round_to(v[i].astype(np.float32), ring_dtype)
        g_ring[i, p] = round_to(g[i].astype(np.float32), ring_dtype)
        beta_ring[i, p] = round_to(beta[i].astype(np.float32), ring_dtype)


# --------------------------------------------------------------------------
# Steady-state cycle: prototype/bench_gdn_full_contract.py:138-154,225-308
# --------------------------------------------------------------------------

def full_contract_decode(codes, scale, mixed_qkv_seq, a_seq, b_seq, a_log, dt_bias, window,
                         heads, key_dim, value_heads, value_dim, ring_dtype="bf16", dtype=np.float32,
                         phase=None):
    """Sequence of full-contract decode steps for a batch: each step appends
    one token (prep), then replays ring slots [0, fill) -- or, when the ring is
    full (fill == window), flushes: rebuild, emit, requantise, restart the ring.

    ``phase[b]`` (default 0) offsets sequence b's ring fill, so a batch can mix
    ring phases (steady state); fill at step s is ((phase + s) % window) + 1.
    mixed_qkv_seq [B,T,D], a_seq/b_seq [B,T,HV]. Returns (outputs [B,T,HV,V],
    codes, scale, saturation per flush list).
    """
    batch, steps = mixed_qkv_seq.shape[:2]
    phase = np.zeros(batch, dtype=np.int64) if phase is None else np.asarray(phase, dtype=np.int64)
    q_out = np.zeros((batch, heads, key_dim), dtype=np.float32)
    k_ring = np.zeros((batch, window, heads, key_dim), dtype=np.float32)
    v_ring = np.zeros((batch, window, value_heads, value_dim), dtype=np.float32)
    g_ring = np.zeros((batch, window, value_heads), dtype=np.float32)
    beta_ring = np.zeros((batch, window, value_heads), dtype=np.float32)
    codes = np.array(codes, dtype=np.uint8, copy=True)
    scale = np.array(scale, copy=True)
    outputs = np.zeros((batch, steps, value_heads, value_dim), dtype=dtype)
    for step in range(steps):
        fill = (phase + step) % window + 1
        pos = fill - 1
        prep_ring(mixed_qkv_seq[:, step], a_seq[:, step], b_seq[:, step], a_log, dt_bias, pos,
                  q_out, k_ring, v_ring, g_ring, beta_ring, ring_dtype)
        flush = fill == window
        out, codes, scale = replay_step(codes, scale, q_out, k_ring, v_ring, g_ring, beta_ring, fill, flush, dtype)
        outputs[:, step] = out
    return outputs, codes, scale


# --------------------------------------------------------------------------
# Byte model: prototype/bench_gdn_replayssm.py:45-87 (logical bytes)
# --------------------------------------------------------------------------

def algorithmic_bytes(batch, heads, value_heads, key_dim, value_dim, fill, flush, act_bytes=2, ring_scalar_bytes=2):
    """Compulsory bytes of one replay (flush=False) or flush (flush=True) call
    with ring fill ``fill``: each tensor element counted once."""
    ckpt = batch * value_heads * value_dim * key_dim
    scales = batch * value_heads * (value_dim // VBLOCK) * 2
    query = batch * heads * key_dim * act_bytes
    ring = batch * (heads * key_dim * act_bytes + value_heads * value_dim * act_bytes + value_heads * 2 * ring_scalar_bytes)
    out = batch * value_heads * value_dim * act_bytes
    if flush:
        return 2 * ckpt + 2 * scales + query + fill * ring + out
    return ckpt + scales + query + fill * ring + out
