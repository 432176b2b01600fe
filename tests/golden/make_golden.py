"""Writes tests/golden/oracle_vectors.npz: small input/output vectors of the oracle, committed so that a change to
the oracle or the kernels shows against fixed numbers.

The reference holds no golden vectors for this path (its oracles are computed at test time, tests/test_blocks.py,
tests/test_gguf.py), so these come from the oracle itself: per block type four seeded random blocks and their
weights; a routed matvec (three experts of 2 x 256, four pairs, float16 activations); a tile layout; SwiGLU values.

Run from the repository root: python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import blocks as O  # noqa: E402

KINDS = ["Q2_0", "IQ4_NL", "IQ4_XS", "IQ3_S", "IQ3_XXS", "Q3_K", "Q4_K", "Q6_K", "Q8_0", "Q4_0", "Q5_0"]
LATER_KINDS = ["Q5_K"]


def main():
    rng = np.random.default_rng(20260101)
    out = {}
    for kind in KINDS:
        per = O.BY_NAME[kind][1]
        n = max(4, 256 // per)  # at least 256 weights
        data = O.random_blocks(kind, n, rng, scale="normal")
        out[f"{kind}/blocks"] = data
        out[f"{kind}/weights"] = O.dequantize(data, kind, (1, n * per)).astype(np.float32)
    data = O.random_blocks("IQ3_S", 3 * 2, rng, scale="normal")
    w = O.dequantize(data, "IQ3_S", (3, 2, 256))
    idx = np.array([2, 0, 2, 1], dtype=np.int64)
    x = (rng.standard_normal((2, 256)) / 4).astype(np.float16)
    out["matvec/blocks"], out["matvec/idx"], out["matvec/x"] = data, idx, x
    out["matvec/out"] = O.expert_matvec(w, idx, x, 2).astype(np.float64)
    ids = rng.integers(0, 5, (7, 3))
    te, token, where = O.tiles_of(ids, 5, 16)
    out["tiles/indices"], out["tiles/tile_expert"], out["tiles/token"], out["tiles/where"] = ids, te, token, where
    g = np.linspace(-12, 12, 97).astype(np.float16)
    u = np.linspace(3, -3, 97).astype(np.float16)
    out["swiglu/g"], out["swiglu/u"] = g, u
    out["swiglu/h16"] = O.swiglu_rounded(g, u, np.float16)
    out["swiglu/h32"] = O.swiglu_rounded(g.astype(np.float32), u.astype(np.float32), np.float32)
    # types added later draw from a stream of their own, so the vectors above stay as they were
    later = np.random.default_rng(20260102)
    for kind in LATER_KINDS:
        data = O.random_blocks(kind, 4, later, scale="normal")
        out[f"{kind}/blocks"] = data
        out[f"{kind}/weights"] = O.dequantize(data, kind, (1, 4 * O.BY_NAME[kind][1])).astype(np.float32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oracle_vectors.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
