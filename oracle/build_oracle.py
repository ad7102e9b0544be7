"""Build recipe for the oracle's C restatement (test infrastructure only).

Compiles oracle/fp8_quant.c with gcc into oracle/_build/liboracle_fp8.so.
No fast-math and no FP contraction: every float operation in the C oracle
must be one correctly rounded IEEE-754 operation.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
BUILD_DIR = ORACLE_DIR / "_build"
LIBRARY = BUILD_DIR / "liboracle_fp8.so"


def build(verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-Wall", "-Wextra", "-Werror", str(ORACLE_DIR / "fp8_quant.c"), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp.replace(LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
