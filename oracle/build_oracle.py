"""Build the C part of the oracle (test infrastructure only).

Compiles ``oracle/c/vq_bruteforce.c`` with gcc into ``oracle/_build/liboracle.so``.
The reference (wrb1371/tac-vq-kv-cache) is pure Python, so there is no
``oracle/_ref`` build: its path has no C/C++ sources to compile.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "c" / "vq_bruteforce.c"
OUT = HERE / "_build" / "liboracle.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-shared", "-fPIC", "-o", str(OUT), str(SRC), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stderr}")
    return OUT


def load() -> ctypes.CDLL:
    if not OUT.is_file() or OUT.stat().st_mtime < SRC.stat().st_mtime:
        build()
    lib = ctypes.CDLL(str(OUT))
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.bf_rvq_encode.argtypes = [vp, vp, i64, i64, i64, i64, vp, vp, vp]
    lib.bf_rvq_encode.restype = None
    lib.bf_scatter.argtypes = [vp, vp, i64, i64, i64, i64, i64, vp]
    lib.bf_scatter.restype = None
    lib.bf_attention_row.argtypes = [vp, vp, vp, i64, i64, vp]
    lib.bf_attention_row.restype = None
    return lib


if __name__ == "__main__":
    print(build())
