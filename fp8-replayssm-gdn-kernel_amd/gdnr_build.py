"""Build libgdnreplay.so (the HIP kernels + the C-ABI layer) for gfx950.

    python gdnr_build.py [-v]

Objects go to _build/ next to this file; the library is written in-tree
(next to this file) so it travels with the source tree to the GPU host.
The C-ABI validation layer (csrc/gdnr_abi.cpp) is plain C++ compiled by g++;
the kernels (csrc/*.hip) by hipcc. Packed-FP32 VALU instructions
are disabled for all device code.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
BUILD_DIR = PKG_DIR / "_build"
LIBRARY = PKG_DIR / "libgdnreplay.so"
ARCH = os.environ.get("GDNR_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]
ACTS = ("bf16", "f16", "f32")  # activation dtypes, one kernel object each (GDNR_ACT = index)
KERNEL_SOURCES = ("gdnr_kernels", "gdnr_step", "gdnr_decode")  # compiled once per activation dtype
SINGLE_SOURCES = ("gdnr_rmw", "gdnr_formats", "gdnr_status", "gdnr_probe")  # compiled once (dtypes are template arguments)
# per-source device flags: the decode kernel's first 13 argument dwords are
# preloaded into SGPRs at wave launch (gfx950 kernarg preload), and its
# wave-uniform branches (workgroup role, replay or flush) are left as scalar
# branches rather than structurised into a chain in which one arm's values
# stay live across the other
SOURCE_FLAGS = {"gdnr_decode": ["-mllvm", "-amdgpu-kernarg-preload-count=13",
                                "-mllvm", "-structurizecfg-skip-uniform-regions=true"]}


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    inc = [f"-I{INCLUDE}", f"-I{CSRC}"]
    kern_objs, jobs = [], []
    for src in KERNEL_SOURCES:
        for i, act in enumerate(ACTS):
            obj = BUILD_DIR / f"{src}_{act}.o"
            kern_objs.append(obj)
            jobs.append([HIPCC, *DEVICE_FLAGS, *SOURCE_FLAGS.get(src, []), *inc, f"-DGDNR_ACT={i}", "-c",
                         str(CSRC / f"{src}.hip"), "-o", str(obj)])
    for src in SINGLE_SOURCES:
        obj = BUILD_DIR / f"{src}.o"
        kern_objs.append(obj)
        jobs.append([HIPCC, *DEVICE_FLAGS, *inc, "-c", str(CSRC / f"{src}.hip"), "-o", str(obj)])
    abi_obj = BUILD_DIR / "gdnr_abi.o"
    jobs.append(["g++", *HOST_FLAGS, *inc, "-c", str(CSRC / "gdnr_abi.cpp"), "-o", str(abi_obj)])
    with ThreadPoolExecutor(max_workers=len(jobs)) as pool:
        for future in [pool.submit(_run, cmd, verbose) for cmd in jobs]:
            future.result()
    tmp = LIBRARY.with_name(LIBRARY.name + ".tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, kern_objs), str(abi_obj), "-o", str(tmp)],
         verbose)
    tmp.replace(LIBRARY)
    return LIBRARY


def device_assembly(act: str = "bf16", src: str = "gdnr_step", out: Path | None = None,
                    verbose: bool = False) -> Path:
    """Write the gfx950 assembly of one source file's kernels for one
    activation dtype (inspection of waits, VGPR counts, instruction mix)."""
    out = out or BUILD_DIR / f"{src}_{act}.s"
    BUILD_DIR.mkdir(exist_ok=True)
    _run([HIPCC, *DEVICE_FLAGS, *SOURCE_FLAGS.get(src, []), f"-I{INCLUDE}", f"-I{CSRC}",
          f"-DGDNR_ACT={ACTS.index(act)}", "--cuda-device-only", "-S", str(CSRC / f"{src}.hip"), "-o", str(out)], verbose)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
