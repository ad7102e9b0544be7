"""ctypes bindings of the C quantiser restatement (oracle/fp8_quant.c).

TEST INFRASTRUCTURE ONLY: see oracle/gdn_oracle.py for the import rule.
"""

from __future__ import annotations

import ctypes

import numpy as np

from .build_oracle import LIBRARY, build

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        handle = ctypes.CDLL(str(LIBRARY))
        i64 = ctypes.c_int64
        p = ctypes.c_void_p
        handle.oracle_e4m3fn_encode_array.argtypes = [p, i64, p]
        handle.oracle_f16_bits_array.argtypes = [p, i64, p]
        handle.oracle_quantize_blocks.argtypes = [p, i64, i64, p, p, p]
        handle.oracle_dequantize_blocks.argtypes = [p, p, i64, i64, p]
        _lib = handle
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def e4m3fn_encode(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().oracle_e4m3fn_encode_array(_ptr(x), x.size, _ptr(out))
    return out


def f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f16_bits_array(_ptr(x), x.size, _ptr(out))
    return out


def quantize_vblock32(state):
    """state [..., V, K] float32 -> (codes uint8 [..., V, K], scale float16
    [..., V/32], saturated int32 [..., V/32])."""
    state = np.ascontiguousarray(state, dtype=np.float32)
    value_dim, key_dim = state.shape[-2:]
    if value_dim % 32:
        raise ValueError("V must be a multiple of 32")
    n_blocks = state.size // (32 * key_dim)
    codes = np.empty(state.shape, dtype=np.uint8)
    scale = np.empty(state.shape[:-2] + (value_dim // 32,), dtype=np.uint16)
    sat = np.empty(scale.shape, dtype=np.int32)
    lib().oracle_quantize_blocks(_ptr(state), n_blocks, 32 * key_dim, _ptr(codes), _ptr(scale), _ptr(sat))
    return codes, scale.view(np.float16), sat


def dequantize_vblock32(codes, scale) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    scale_bits = np.ascontiguousarray(np.asarray(scale, dtype=np.float16)).view(np.uint16)
    key_dim = codes.shape[-1]
    out = np.empty(codes.shape, dtype=np.float32)
    lib().oracle_dequantize_blocks(_ptr(codes), _ptr(scale_bits), scale_bits.size, 32 * key_dim, _ptr(out))
    return out
