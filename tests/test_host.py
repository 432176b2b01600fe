"""Host-side logic of the library that runs without a GPU: packing of the reference's layer parts into the
file's blocks."""

import numpy as np
import torch

from oracle import blocks as O
from strata_mlx_amd.dense import q6k_blocks


def test_q6_k_parts_pack_back_into_the_blocks_they_came_from():
    """dense.q6k_blocks is the inverse of the reference's q6k_parts (strata_mlx/gguf.py:150-165): blocks split
    into (codes, scales, d) as q6k_parts splits them, packed back, give the same bytes; and the packed blocks
    decode to code * scale * d."""
    rng = np.random.default_rng(6)
    rows, cols = 3, 512
    data = O.random_blocks("Q6_K", rows * cols // 256, rng, scale="normal")
    b = data.reshape(-1, 210)
    ql, qh = b[:, :128].reshape(-1, 2, 64), b[:, 128:192].reshape(-1, 2, 32)
    hi = np.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], axis=2)
    lo = np.stack([ql[..., :32] & 15, ql[..., 32:] & 15, ql[..., :32] >> 4, ql[..., 32:] >> 4], axis=2)
    codes = ((lo | (hi << 4)).astype(np.int16) - 32).astype(np.int8).reshape(rows, cols)
    scales = np.ascontiguousarray(b[:, 192:208]).view(np.int8).reshape(rows, -1)
    d = np.ascontiguousarray(b[:, 208:210]).view("<f2").reshape(rows, -1)
    packed = q6k_blocks(torch.from_numpy(codes), torch.from_numpy(scales), torch.from_numpy(d)).numpy()
    assert np.array_equal(packed, data.reshape(-1))
    w = O.dequantize(packed, "Q6_K", (rows, cols))
    want = (codes.astype(np.float64) * np.repeat(scales.astype(np.float64), 16, axis=1)
            * np.repeat(d.astype(np.float64), 256, axis=1))
    assert np.array_equal(w, want.astype(np.float32))
