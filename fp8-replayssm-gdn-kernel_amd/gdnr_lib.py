"""ctypes bindings of libgdnreplay.so (the C ABI declared in include/gdnr.h).

Tensors cross the boundary as ``gdnr_tensor`` descriptors (device pointer,
dtype code, shape, element strides). Every call enqueues on the caller's
current HIP stream and returns without synchronising; a nonzero status is
raised as ``GdnrError`` with the library's own message.

There is no fallback: if the library is not built, the first call raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

PKG_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = Path(os.environ.get("GDNR_LIBRARY", PKG_DIR / "libgdnreplay.so"))

MAX_DIMS = 4
ABI_VERSION = 1

# gdnr_dtype codes
DTYPE_CODES = {
    torch.bfloat16: 0,
    torch.float16: 1,
    torch.float32: 2,
    torch.float8_e4m3fn: 3,
    torch.uint8: 4,
    torch.int32: 5,
    torch.int64: 6,
    torch.bool: 7,
    torch.int8: 8,
}

STATUS_NAMES = {1: "invalid argument", 2: "unsupported", 3: "HIP error"}


class GdnrError(RuntimeError):
    """A nonzero status from libgdnreplay.so."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class GdnrTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * MAX_DIMS),
        ("strides", ctypes.c_int64 * MAX_DIMS),
    ]


# exported entry points: name -> number of gdnr_tensor* arguments, trailing int32 args[, trailing float args]
ENTRY_POINTS = {
    "gdnr_replay_fp8": (10, 1),
    "gdnr_replay_fp8_split": (11, 3),
    "gdnr_replay_fp8_split_noalloc": (9, 3),
    "gdnr_prep_ring": (11, 1),
    "gdnr_prep_replay_fp8": (16, 1),
    "gdnr_prep_replay_fp8_slots": (17, 1),
    "gdnr_quantize_vblock32": (4, 0),
    "gdnr_dequantize_vblock32": (3, 0),
    "gdnr_bf16_step": (7, 0),
    "gdnr_bf16_step_packed": (8, 0, 1),
    "gdnr_quantize_checkpoint": (4, 2),
    "gdnr_dequantize_checkpoint": (3, 2),
    "gdnr_stream_probe": (1, 1),
}

_lib = None


def load_library(path: Path | None = None) -> ctypes.CDLL:
    """Load (once) and type the library. Raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    path = Path(path or LIBRARY_PATH)
    if not path.exists():
        raise RuntimeError(
            f"{path} is not built; run `python {PKG_DIR / 'gdnr_build.py'}` (the HIP path has no fallback)")
    lib = ctypes.CDLL(str(path))
    lib.gdnr_last_error.restype = ctypes.c_char_p
    lib.gdnr_last_error.argtypes = []
    lib.gdnr_abi_version.restype = ctypes.c_int
    lib.gdnr_abi_version.argtypes = []
    lib.gdnr_wait_timeouts.restype = ctypes.c_int
    lib.gdnr_wait_timeouts.argtypes = [ctypes.POINTER(ctypes.c_uint32), ctypes.c_int32]
    lib.gdnr_set_wait_polls.restype = ctypes.c_uint32
    lib.gdnr_set_wait_polls.argtypes = [ctypes.c_uint32]
    lib.gdnr_decode_plan.restype = ctypes.c_int
    lib.gdnr_decode_plan.argtypes = [ctypes.c_int32] * 6 + [ctypes.POINTER(ctypes.c_int32)]
    for name, (n_tensors, n_ints, *n_floats) in ENTRY_POINTS.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = ([ctypes.POINTER(GdnrTensor)] * n_tensors + [ctypes.c_int32] * n_ints
                       + [ctypes.c_float] * sum(n_floats) + [ctypes.c_void_p])
    if lib.gdnr_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {lib.gdnr_abi_version()} != {ABI_VERSION}")
    if path == LIBRARY_PATH:
        _lib = lib
    return lib


def describe(t: torch.Tensor | None) -> GdnrTensor | None:
    """gdnr_tensor descriptor of a torch tensor (None stays None)."""
    if t is None:
        return None
    if t.dim() > MAX_DIMS:
        raise ValueError(f"tensors of rank {t.dim()} are not accepted")
    code = DTYPE_CODES.get(t.dtype)
    if code is None:
        raise TypeError(f"dtype {t.dtype} is not accepted by libgdnreplay")
    desc = GdnrTensor()
    desc.data = t.data_ptr() if t.numel() else None
    desc.dtype = code
    desc.ndim = t.dim()
    for d in range(t.dim()):
        desc.shape[d] = t.shape[d]
        desc.strides[d] = t.stride(d)
    return desc


def call(name: str, tensors, ints=(), stream: int | None = None, floats=()) -> None:
    """Invoke an entry point; tensors must already be on the same CUDA device."""
    lib = load_library()
    fn = getattr(lib, name)
    descs = [describe(t) for t in tensors]
    ptrs = [ctypes.byref(d) if d is not None else None for d in descs]
    status = fn(*ptrs, *[int(i) for i in ints], *[float(x) for x in floats], ctypes.c_void_p(stream))
    if status != 0:
        raise GdnrError(status, lib.gdnr_last_error().decode())


def current_stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def wait_timeouts(reset: bool = False) -> int:
    """Bounded LDS waits of the decode kernels that gave up on the current
    device since the last reset (gdnr_wait_timeouts; synchronises the device).
    Nonzero means some step's output is meaningless; the waves whose waits
    gave up skipped their in-place checkpoint code and scale stores."""
    lib = load_library()
    count = ctypes.c_uint32(0)
    status = lib.gdnr_wait_timeouts(ctypes.byref(count), 1 if reset else 0)
    if status != 0:
        raise GdnrError(status, lib.gdnr_last_error().decode())
    return int(count.value)


DEFAULT_WAIT_POLLS = 1 << 22


def set_wait_polls(polls: int) -> int:
    """Poll budget of the kernels' bounded waits for later launches
    (process-wide; gdnr_set_wait_polls). Returns the previous budget. 0 makes
    every wait give up at once: a test of the give-up path."""
    return int(load_library().gdnr_set_wait_polls(int(polls)))


def decode_plan(batch: int, heads: int, value_heads: int, value_dim: int, ring_len: int,
                act: torch.dtype = torch.bfloat16) -> dict | None:
    """The decode kernel's launch plan for a shape (gdnr_decode_plan), or
    None when the shape takes another kernel."""
    lib = load_library()
    plan = (ctypes.c_int32 * 5)()
    status = lib.gdnr_decode_plan(batch, heads, value_heads, value_dim, ring_len, DTYPE_CODES[act], plan)
    if status == 2:
        return None
    if status != 0:
        raise GdnrError(status, lib.gdnr_last_error().decode())
    return {"rows_per_wave": plan[0], "waves_per_head": plan[1], "heads_per_unit": plan[2], "units": plan[3],
            "lds_bytes": plan[4]}
