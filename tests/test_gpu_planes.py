"""Q3_K held as planes on the GPU (strata_mlx/blocks.py:397-512) against the oracle: the planes are the oracle's
rearrangement bit for bit, their dequantization the oracle's Q3_K weights bit for bit, the window's products the
float64 product at the reference's tolerances (test_dense.py:49: 2e-5 float32, 4e-3 float16, relative to the
largest output), a token alone the bits it gets in a window, and BlockLinear over Q3_K holds planes when asked
to (else the file's blocks)."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B
from strata_mlx_amd import dense as D

pytestmark = pytest.mark.gpu


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


@pytest.mark.parametrize("rows,cols", [(7, 256), (64, 2560), (640, 1024)])
def test_planes_and_their_weights_are_the_oracles(gpu, rows, cols):
    rng = np.random.default_rng(rows)
    data = O.random_blocks("Q3_K", rows * cols // 256, rng)
    planes = B.q3k_planes(dev(data, gpu), rows, cols)
    want = O.q3k_planes(data, rows, cols)
    assert np.array_equal(planes["hm"].cpu().numpy().view(np.uint32), want["hm"].reshape(-1))
    assert np.array_equal(planes["qs"].cpu().numpy().view(np.uint32), want["qs"].reshape(-1))
    assert np.array_equal(planes["sc"].cpu().numpy(), want["sc"].reshape(-1))
    assert np.array_equal(planes["dd"].cpu().numpy().view(np.uint16), want["dd"].view(np.uint16))
    w = O.dequantize(data, "Q3_K", (rows, cols))
    got = B.q3k_planes_dequantize(planes, rows, cols, torch.float32).cpu().numpy()
    assert np.array_equal(got, w)
    got16 = B.q3k_planes_dequantize(planes, rows, cols, torch.float16).cpu().numpy()
    assert np.array_equal(got16, w.astype(np.float16))


@pytest.mark.parametrize("tokens", [1, 3, 8, 12])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_the_window_is_the_product(gpu, tokens, dtype):
    rng = np.random.default_rng(tokens)
    rows, cols = 96, 2560
    data = O.random_blocks("Q3_K", rows * cols // 256, rng)
    w = O.dequantize(data, "Q3_K", (rows, cols)).astype(np.float64)
    planes = B.q3k_planes(dev(data, gpu), rows, cols)
    x = torch.randn((tokens, cols), generator=torch.Generator().manual_seed(tokens)).to(dtype)
    got = B.q3k_planes_window(planes, rows, cols, x.to(gpu)).float().cpu().numpy()
    assert got.shape == (tokens, rows)
    want = x.double().numpy() @ w.T
    tol = 2e-5 if dtype == torch.float32 else 4e-3 if dtype == torch.float16 else 2e-2
    assert np.abs(got - want).max() <= tol * np.abs(want).max()
    alone = B.q3k_planes_window(planes, rows, cols, x[-1:].to(gpu))
    assert torch.equal(alone.cpu()[0], B.q3k_planes_window(planes, rows, cols, x.to(gpu)).cpu()[-1])


@pytest.mark.parametrize("planes", [True, False])
def test_block_linear_holds_q3_k_as_planes_or_blocks(gpu, planes, monkeypatch):
    monkeypatch.setattr(D, "PLANES", planes)
    rng = np.random.default_rng(6)
    rows, cols = 40, 1024
    data = O.random_blocks("Q3_K", rows * cols // 256, rng)
    layer = D.BlockLinear(dev(data, gpu), "Q3_K", (rows, cols))
    if not planes:
        assert layer.planes is None and layer.nbytes == rows * cols // 256 * 110
        x = torch.randn((3, cols), generator=torch.Generator().manual_seed(2))
        got = layer(x.half().to(gpu)).float().cpu().numpy()
        want = x.half().double().numpy() @ O.dequantize(data, "Q3_K", (rows, cols)).astype(np.float64).T
        assert np.abs(got - want).max() <= 4e-3 * np.abs(want).max()
        return
    assert layer.planes is not None and layer.nbytes == rows * cols // 256 * B.Q3K_PLANE_BYTES
    x = torch.randn((20, cols), generator=torch.Generator().manual_seed(2))  # more than a window: floats
    got = layer(x.to(gpu)).cpu().numpy()
    want = x.double().numpy() @ O.dequantize(data, "Q3_K", (rows, cols)).astype(np.float64).T
    assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max()
