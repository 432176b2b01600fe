"""The dense one-token matvec of a long Q6_K matrix (an lm_head), whose rows are staged in LDS by 16-byte direct
loads (stream_rows_kernel; from 65536 rows with the non-temporal cache policy): sampled rows are the float64 product of the oracle's weights within the window test's
bound (test_dense.py:49: 4e-3 relative to the largest output), and listed rows (rows.py:30-42) have the full
product's bits, in the order listed, repeats included, NaN for an id past the layer."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows", [8192, 12288, 40037, 65603])
def test_lm_head_rows_are_the_product(gpu, rows):
    rng = np.random.default_rng(rows)
    cols = 4096
    data = O.random_blocks("Q6_K", rows * cols // 256, rng)
    blocks = torch.from_numpy(data).to(gpu)
    row_bytes = cols // 256 * 210
    for seed in (0, 1):
        x = torch.randn((1, cols), generator=torch.Generator().manual_seed(seed)).half().to(gpu)
        full = B.window_matvec(blocks, "Q6_K", rows, cols, x)
        pick = np.unique(np.concatenate([[0, 1, rows - 2, rows - 1], rng.choice(rows, 60, replace=False)]))
        w = O.dequantize(data.reshape(rows, row_bytes)[pick].reshape(-1), "Q6_K", (len(pick), cols))
        want = w.astype(np.float64) @ x.double().cpu().numpy()[0]
        got = full.double().cpu().numpy()[0, pick]
        assert np.abs(got - want).max() <= 4e-3 * np.abs(want).max()
        # every row listed, and a few in another order with a repeat and an id past the layer
        every = B.window_matvec(blocks, "Q6_K", rows, cols, x,
                                row_ids=torch.arange(rows, dtype=torch.int32, device=gpu))
        assert torch.equal(every, full)
        ids = torch.tensor([rows - 1, 5, 5, 0, rows // 2, 17], dtype=torch.int32, device=gpu)
        assert torch.equal(B.window_matvec(blocks, "Q6_K", rows, cols, x, row_ids=ids), full[:, ids.long()])
        past = B.window_matvec(blocks, "Q6_K", rows, cols, x,
                               row_ids=torch.tensor([3, rows], dtype=torch.int32, device=gpu))
        assert torch.equal(past[0, 0], full[0, 3]) and torch.isnan(past[0, 1])
