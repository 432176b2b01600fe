"""The kernels against the committed vectors of tests/golden/ (the oracle's output at a fixed seed): dequant bit
for bit for every type, the routed matvec within the float16 tolerance, the tile layout bit for bit."""

import os

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_vectors.npz")
KINDS = ["Q2_0", "IQ4_NL", "IQ4_XS", "IQ3_S", "IQ3_XXS", "Q3_K", "Q4_K", "Q6_K", "Q8_0", "Q4_0", "Q5_0", "Q5_K"]


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_gives_the_committed_weights(gpu, gold, kind):
    data = gold[f"{kind}/blocks"]
    per, size = O.BY_NAME[kind][1], O.BY_NAME[kind][2]
    n = data.size // size
    got = B.dequantize(torch.from_numpy(data.reshape(-1)).to(gpu), kind, (1, n * per)).cpu().numpy()
    assert np.array_equal(got, gold[f"{kind}/weights"])


def test_routed_matvec_gives_the_committed_products(gpu, gold):
    lin = B.BlockSwitchLinear(torch.from_numpy(gold["matvec/blocks"].reshape(-1)).to(gpu), "IQ3_S", (3, 2, 256))
    idx = torch.from_numpy(gold["matvec/idx"]).to(gpu)
    x = torch.from_numpy(gold["matvec/x"]).to(gpu)
    got = B.expert_matvec(lin, idx, x, 2).double().cpu().numpy()
    want = gold["matvec/out"]
    assert np.linalg.norm(got - want) <= 1e-3 * np.linalg.norm(want)


def test_tiles_give_the_committed_layout(gpu, gold):
    te, token, where = B.tiles_of(torch.from_numpy(gold["tiles/indices"]).to(gpu), 5)
    assert np.array_equal(te.cpu().numpy().astype(np.uint32), gold["tiles/tile_expert"])
    assert np.array_equal(token.cpu().numpy().astype(np.uint32), gold["tiles/token"])
    assert np.array_equal(where.cpu().numpy().astype(np.uint32), gold["tiles/where"])
