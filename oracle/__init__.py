"""CPU oracle for strata_mlx_amd: a restatement of the reference's block decoders and products.

TEST INFRASTRUCTURE ONLY. Only `tests/`, `__graft_entry__.smoke()` and the CPU-baseline leg of
`bench.py` import this package, and only as the checker. The library never imports it, and its
kernels never fall back to it.

- `blocks.py`: numpy decoders for every type (float64 closed forms, rounded once to float32),
  matvec / SwiGLU / tiles products (strata_mlx/blocks.py, strata_mlx/gguf.py).
- `grids.py`: the IQ3 codebooks in gguf-py's hex encoding, decoded by gguf-py's own rule.
- `unpack.c`: a scalar C restatement of `unpack32`, built by `Makefile` into `_build/liboracle.so`.
"""

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")


def build() -> str:
    """Compile unpack.c (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def c_library() -> ctypes.CDLL:
    """The C restatement; built on first use if it is not there."""
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    p, i64, i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.oracle_dequant.argtypes = [i, p, i64, i64, i64, p, p]
    lib.oracle_dequant.restype = i
    lib.oracle_matvec.argtypes = [i, p, i64, i64, i64, p, i64, p, i64, p, p]
    lib.oracle_matvec.restype = i
    return lib
