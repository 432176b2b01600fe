"""Rows of 24 and 40 run pairs (1536 and 2560 inputs: the down projection, 2560-wide layers) at one token a pass,
the kernel that gives a row 8 lanes: against the float64 product of the oracle's weights (test_blocks.py:65:
2e-3 relative for float16), with an expert named by several pairs (a pass a pair, the token reloaded), every
pair on one token (one pass written to each pair naming the expert), row counts that are not a multiple of 8,
a pair alone against the same pair among others (the same bits), a matrix a pair against the stack
(matvec_separate, blocks.py:331: the same bits), windows of one and three tokens, and listed rows."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B

pytestmark = pytest.mark.gpu

KINDS = ["IQ3_S", "IQ3_XXS", "Q2_0"]


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def stack(kind, rng, experts, rows, cols):
    data = O.random_blocks(kind, experts * rows * cols // O.BY_NAME[kind][1], rng)
    w = O.dequantize(data, kind, (experts * rows, cols)).astype(np.float64).reshape(experts, rows, cols)
    return data, w


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("cols", [1536, 2560])
@pytest.mark.parametrize("rows", [37, 64])
def test_pairs_naming_an_expert_again_are_the_product(gpu, kind, cols, rows):
    rng = np.random.default_rng(cols + rows)
    E = 3
    data, w = stack(kind, rng, E, rows, cols)
    layer = B.BlockSwitchLinear(dev(data, gpu), kind, (E, rows, cols))
    idx = np.array([[2, 0], [0, 2], [1, 1]])  # three tokens, six pairs: expert 0 and 2 twice, 1 twice in a token
    x = (rng.standard_normal((3, 1, 1, cols)) / 8).astype(np.float16)
    got = layer(dev(x, gpu), dev(idx, gpu)).float().cpu().numpy()[:, :, 0]
    want = np.einsum("tkoi,ti->tko", w[idx], x[:, 0, 0].astype(np.float64))
    assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max()
    # each pair alone (one pass) gives the bits it has among the others (a later pass)
    flat = dev(idx.reshape(-1).astype(np.int32), gpu)
    xs = dev(np.repeat(x[:, 0, 0], 2, 0), gpu)
    together = B.expert_matvec(layer, flat, xs, 1)
    for p in range(6):
        alone = B.expert_matvec(layer, flat[p:p + 1], xs[p:p + 1], 1)
        assert torch.equal(alone[0], together[p])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("cols", [1536, 2560])
def test_one_token_on_repeated_experts_writes_every_pair(gpu, kind, cols):
    rng = np.random.default_rng(11)
    E, rows = 4, 45
    data, w = stack(kind, rng, E, rows, cols)
    layer = B.BlockSwitchLinear(dev(data, gpu), kind, (E, rows, cols))
    idx = np.array([3, 0, 3, 1, 0, 3], dtype=np.int32)
    x = (rng.standard_normal((1, cols)) / 8).astype(np.float16)
    got = B.expert_matvec(layer, dev(idx, gpu), dev(x, gpu), len(idx))
    want = w[idx] @ x[0].astype(np.float64)
    assert np.abs(got.float().cpu().numpy() - want).max() <= 2e-3 * np.abs(want).max()
    for p in range(len(idx)):  # pairs naming one expert: the same bits
        assert torch.equal(got[p], got[int(np.flatnonzero(idx == idx[p])[0])])


@pytest.mark.parametrize("kind", KINDS)
def test_a_matrix_a_pair_gives_the_bits_of_the_stack_at_1536(gpu, kind):
    rng = np.random.default_rng(5)
    E, rows, cols = 3, 40, 1536
    data, _ = stack(kind, rng, E, rows, cols)
    blocks = dev(data, gpu)
    layer = B.BlockSwitchLinear(blocks, kind, (E, rows, cols))
    rb = B.row_bytes(kind, cols)
    experts = [blocks[e * rows * rb:(e + 1) * rows * rb].clone() for e in (2, 0, 1, 1)]  # the pairs' matrices
    x = torch.randn((2, cols), generator=torch.Generator().manual_seed(1)).half().to(gpu)
    got = B.matvec_separate(experts, kind, rows, cols, x, 2)
    want = layer(x.reshape(2, 1, 1, cols), dev(np.array([[2, 0], [1, 1]]), gpu)).reshape(4, rows)
    assert torch.equal(got, want)


WINDOW_KINDS = ["IQ3_S", "IQ3_XXS", "Q2_0", "Q3_K", "Q6_K", "Q8_0", "IQ4_XS", "IQ4_NL", "Q4_0", "Q5_0"]


@pytest.mark.parametrize("kind", WINDOW_KINDS)
@pytest.mark.parametrize("cols", [1536, 2560])
@pytest.mark.parametrize("tokens", [1, 3])
def test_a_window_of_odd_rows_is_the_product(gpu, kind, cols, tokens):
    """window_matvec (blocks.py:383-394) on rows of 24 / 40 run pairs: test_dense.py:49's 4e-3 of the largest
    output for float16."""
    rng = np.random.default_rng(cols + tokens)
    rows = 53
    data, w = stack(kind, rng, 1, rows, cols)
    x = torch.randn((tokens, cols), generator=torch.Generator().manual_seed(tokens)).half()
    got = B.window_matvec(dev(data, gpu), kind, rows, cols, x.to(gpu)).float().cpu().numpy()
    want = x.double().numpy() @ w[0].T
    assert got.shape == (tokens, rows)
    assert np.abs(got - want).max() <= 4e-3 * np.abs(want).max()


@pytest.mark.parametrize("kind", ["Q3_K", "Q6_K", "Q8_0", "IQ4_XS"])
@pytest.mark.parametrize("cols", [1536, 2560])
def test_listed_rows_of_odd_rows_have_the_layers_bits(gpu, kind, cols):
    """rows.py:30-42: rows by id give the full layer's outputs bit for bit; an id past the layer gives NaN."""
    rng = np.random.default_rng(3)
    rows = 300
    data, _ = stack(kind, rng, 1, rows, cols)
    blocks = dev(data, gpu)
    x = torch.randn((1, cols), generator=torch.Generator().manual_seed(2)).half().to(gpu)
    full = B.window_matvec(blocks, kind, rows, cols, x)
    ids = torch.tensor([5, 299, 0, 17, 17, 250, 3, 101, 77, 128, 64], dtype=torch.int32, device=gpu)
    got = B.window_matvec(blocks, kind, rows, cols, x, row_ids=ids)
    assert torch.equal(got, full[:, ids.long()])
    bad = B.window_matvec(blocks, kind, rows, cols, x, row_ids=torch.tensor([1, 300], dtype=torch.int32, device=gpu))
    assert torch.isfinite(bad[0, 0]) and torch.isnan(bad[0, 1])
