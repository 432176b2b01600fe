"""Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, IQ4_XS, IQ4_NL, Q4_0 and Q5_0 decoded in registers (the direct kernel's linear kinds) against the float64 product
of the oracle's weights, at the rows the kernel takes at compile time (64 lanes to a 4096-input row, 32 to 1536
and 2048) and at run time (16 to 1024): the dense window (test_dense.py:49: 4e-3 relative to the largest output
for float16), routed pairs with an expert named twice (test_blocks.py:65: 2e-3 relative), gate and up in one
launch (their own bits for gate and up), and an lm_head-wide layer's listed rows (rows.py:30-42: the full
layer's bits, NaN for an id past it)."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B

pytestmark = pytest.mark.gpu

LINEAR = ["Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "IQ4_XS", "IQ4_NL", "Q4_0", "Q5_0"]


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def weights(kind, rng, rows, cols, **kw):
    data = O.random_blocks(kind, rows * cols // O.BY_NAME[kind][1], rng, **kw)
    return data, O.dequantize(data, kind, (rows, cols)).astype(np.float64)


@pytest.mark.parametrize("kind", LINEAR)
@pytest.mark.parametrize("cols", [1024, 1536, 2048, 4096])
@pytest.mark.parametrize("tokens", [1, 3])
def test_a_window_is_the_product(gpu, kind, cols, tokens):
    rng = np.random.default_rng(cols + tokens)
    rows = 72
    data, w = weights(kind, rng, rows, cols)
    x = torch.randn((tokens, cols), generator=torch.Generator().manual_seed(tokens)).half()
    got = B.window_matvec(dev(data, gpu), kind, rows, cols, x.to(gpu)).float().cpu().numpy()
    want = x.double().numpy() @ w.T
    assert got.shape == (tokens, rows)
    assert np.abs(got - want).max() <= 4e-3 * np.abs(want).max()


@pytest.mark.parametrize("kind", LINEAR)
@pytest.mark.parametrize("cols", [1536, 4096])
def test_routed_pairs_are_the_product(gpu, kind, cols):
    rng = np.random.default_rng(cols)
    E, rows = 3, 40
    data, w = weights(kind, rng, E * rows, cols)
    w = w.reshape(E, rows, cols)
    layer = B.BlockSwitchLinear(dev(data, gpu), kind, (E, rows, cols))
    idx = np.array([[2, 0], [1, 1], [0, 2]])  # three tokens, two experts each (one twice)
    x = (rng.standard_normal((3, 1, 1, cols)) / 8).astype(np.float16)
    got = layer(dev(x, gpu), dev(idx, gpu)).float().cpu().numpy()[:, :, 0]
    want = np.einsum("tkoi,ti->tko", w[idx], x[:, 0, 0].astype(np.float64))
    assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max()


@pytest.mark.parametrize("kind", LINEAR)
def test_gate_and_up_in_one_launch_give_their_own_bits(gpu, kind):
    rng = np.random.default_rng(5)
    E, F, H, k = 6, 64, 4096, 4
    gate, up = (B.BlockSwitchLinear(dev(weights(kind, rng, E * F, H, scale="normal")[0], gpu), kind, (E, F, H))
                for _ in range(2))
    idx = dev(rng.choice(E, k, replace=False).astype(np.int32), gpu)
    x = dev((rng.standard_normal((1, H)) / 16).astype(np.float16), gpu)
    g0, u0 = B.gate_up(gate, up, x, idx, k)
    g, u, h = B.gate_up_swiglu(gate, up, x, idx, k)
    assert torch.equal(g, g0) and torch.equal(u, u0)
    want = O.swiglu_rounded(g.cpu().numpy(), u.cpu().numpy(), np.float16)
    hb, wb = h.cpu().numpy().view(np.int16).astype(np.int32), want.view(np.int16).astype(np.int32)
    assert np.abs(hb - wb).max() <= 1 and (hb != wb).mean() <= 0.01  # device expf against numpy's exp


@pytest.mark.parametrize("kind", LINEAR)
def test_listed_rows_of_a_wide_layer_have_its_bits(gpu, kind):
    rng = np.random.default_rng(7)
    rows, cols = 300, 4096
    data, _ = weights(kind, rng, rows, cols)
    blocks = dev(data, gpu)
    x = torch.randn((1, cols), generator=torch.Generator().manual_seed(2)).half().to(gpu)
    full = B.window_matvec(blocks, kind, rows, cols, x)
    ids = torch.tensor([5, 299, 0, 17, 17, 250, 3, 101, 77, 128, 64], dtype=torch.int32, device=gpu)
    got = B.window_matvec(blocks, kind, rows, cols, x, row_ids=ids)
    assert torch.equal(got, full[:, ids.long()])
    bad = B.window_matvec(blocks, kind, rows, cols, x, row_ids=torch.tensor([1, 300], dtype=torch.int32, device=gpu))
    assert torch.isfinite(bad[0, 0]) and torch.isnan(bad[0, 1])
