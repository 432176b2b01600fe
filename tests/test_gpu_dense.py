"""Dense layers on the file's blocks (strata_mlx/dense.py, rows.py restated): ScaledLinear from the reference's
Q6_K parts, BlockLinear with reordered inputs, BlockEmbedding, and the listed rows of an output layer. Products
against the float64 product of the oracle's weights at the reference's tolerances (test_dense.py:49: 2e-5
float32, 4e-3 float16, relative to the largest output)."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import dense as D
from strata_mlx_amd import rows as R

pytestmark = pytest.mark.gpu


def q6k_parts(data, rows):
    b = data.reshape(-1, 210)
    ql, qh = b[:, :128].reshape(-1, 2, 64), b[:, 128:192].reshape(-1, 2, 32)
    hi = np.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], axis=2)
    lo = np.stack([ql[..., :32] & 15, ql[..., 32:] & 15, ql[..., :32] >> 4, ql[..., 32:] >> 4], axis=2)
    codes = ((lo | (hi << 4)).astype(np.int16) - 32).astype(np.int8).reshape(rows, -1)
    return (codes, np.ascontiguousarray(b[:, 192:208]).view(np.int8).reshape(rows, -1),
            np.ascontiguousarray(b[:, 208:210]).view("<f2").reshape(rows, -1))


@pytest.mark.parametrize("tokens", [1, 3, 8, 12])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_scaled_linear_from_parts_multiplies_as_its_weights(gpu, tokens, dtype):
    rng = np.random.default_rng(tokens)
    rows, cols = 40, 1024
    data = O.random_blocks("Q6_K", rows * cols // 256, rng)
    w = O.dequantize(data, "Q6_K", (rows, cols))
    parts = [torch.from_numpy(a).to(gpu) for a in q6k_parts(data, rows)]
    layer = D.ScaledLinear(*parts)
    assert torch.equal(layer.blocks.cpu(), torch.from_numpy(data.reshape(-1)))
    x = torch.randn((tokens, cols), generator=torch.Generator().manual_seed(tokens)).to(dtype)
    got = layer(x.to(gpu)).float().cpu().numpy()
    want = x.double().numpy() @ w.astype(np.float64).T
    tol = 2e-5 if dtype == torch.float32 else 4e-3
    if tokens > D.MAX_TOKENS and dtype == torch.float16:
        tol = 1e-2  # the float16 GEMM of a chunk rounds its sums
    assert np.abs(got - want).max() <= tol * np.abs(want).max()


@pytest.mark.parametrize("kind", ["IQ4_XS", "Q3_K", "Q4_K"])
def test_block_linear_reorders_its_inputs(gpu, kind):
    rng = np.random.default_rng(3)
    rows, cols = 12, 512
    per = O.BY_NAME[kind][1]
    data = O.random_blocks(kind, rows * cols // per, rng)
    w = O.dequantize(data, kind, (rows, cols))
    inputs = rng.permutation(cols)  # where in the file's row each input is
    layer = D.BlockLinear(torch.from_numpy(data).to(gpu), kind, (rows, cols), inputs=inputs)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    got = layer(torch.from_numpy(x).to(gpu)).cpu().numpy()
    x_file = np.zeros_like(x)
    x_file[:, inputs] = x
    want = x_file.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max()


def test_block_embedding_gives_the_rows_of_its_tokens(gpu):
    rng = np.random.default_rng(4)
    vocab, dims = 50, 512
    data = O.random_blocks("IQ4_XS", vocab * dims // 256, rng)
    w = O.dequantize(data, "IQ4_XS", (vocab, dims))
    emb = D.BlockEmbedding(torch.from_numpy(data).to(gpu), "IQ4_XS", (vocab, dims), torch.float32)
    ids = np.array([[3, 49, 3], [0, 17, 22]])
    got = emb(torch.from_numpy(ids).to(gpu)).cpu().numpy()
    assert got.shape == (2, 3, dims)
    assert np.array_equal(got, w[ids])


def test_listed_rows_of_an_output_layer(gpu):
    """rows.py:30-42: the listed rows as a layer of their own give the full layer's outputs bit for bit, in the
    order listed, repeats included; an id past the layer gives NaN."""
    rng = np.random.default_rng(5)
    vocab, dims = 300, 1024
    data = O.random_blocks("Q6_K", vocab * dims // 256, rng)
    head = D.ScaledLinear.from_blocks(torch.from_numpy(data).to(gpu), (vocab, dims))
    x = torch.randn((1, dims), generator=torch.Generator().manual_seed(0)).half().to(gpu)
    full = head(x)
    ids = np.array([7, 299, 3, 150, 8, 7])
    assert torch.equal(R.rows_of(head, ids)(x), full[:, ids])
    past = R.rows_of(head, np.array([2, 300]))(x)
    assert torch.equal(past[0, 0], full[0, 2]) and torch.isnan(past[0, 1])
