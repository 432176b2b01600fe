"""Prompt chunks through tiles on the GPU: the tile layout is the oracle's, bit for bit; the MFMA products are the
float64 products of the oracle's weights rounded as the reference rounds them (tests/test_blocks.py:97-206 of the
reference)."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B

pytestmark = pytest.mark.gpu

KINDS = ["Q2_0", "IQ4_NL", "IQ4_XS", "IQ3_S", "IQ3_XXS", "Q3_K", "Q4_K", "Q6_K", "Q8_0", "Q4_0", "Q5_0", "Q5_K"]


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def stack(kind, rng, experts, rows, cols, lo=0.001, hi=0.01):
    per = O.BY_NAME[kind][1]
    data = O.random_blocks(kind, experts * rows * cols // per, rng, lo=lo, hi=hi)
    return data, O.dequantize(data, kind, (experts, rows, cols))


@pytest.mark.parametrize("tokens, k, experts", [(211, 3, 7), (5, 2, 40), (64, 10, 512), (1, 1, 3), (512, 8, 256),
                                                (2048, 8, 256)])
def test_the_gpu_tile_layout_is_the_oracles(gpu, tokens, k, experts):
    rng = np.random.default_rng(tokens)
    idx = rng.integers(0, experts, (1, tokens, k))
    idx[0, :tokens // 3] = 1
    if tokens >= 33 and experts > 4:
        idx[0, -33:, 0] = np.repeat([3, 4], [16, 17])
    te, token, where = (t.cpu().numpy() for t in B.tiles_of(dev(idx, gpu), experts))
    want = O.tiles_of(idx, experts)
    np.testing.assert_array_equal(te.astype(np.uint32), want[0])
    np.testing.assert_array_equal(token.astype(np.uint32), want[1])
    np.testing.assert_array_equal(where.astype(np.uint32), want[2])


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_the_tile_product_is_the_product_with_the_weights(gpu, kind, dtype):
    rng = np.random.default_rng(0)
    shape = (4, 128, 512)
    data, w = stack(kind, rng, *shape)
    # weights as the MFMA takes them: exact for float32 activations and for the codebook types' whole blocks
    # (float16 integer codes, the run scale on the float32 sums); rounded to float16 otherwise
    exact = dtype == torch.float32 or (kind in ("IQ3_S", "IQ3_XXS", "Q2_0") and shape[2] % 256 == 0)
    w = w.astype(np.float32 if exact else np.float16).astype(np.float64)
    tiles = np.array([3, 0, 0, 2, 3])
    a = torch.from_numpy(rng.standard_normal((16 * len(tiles), shape[2])).astype(np.float32)).to(dtype)
    got = B.tile_matmul(dev(data, gpu), kind, shape, a.to(gpu), dev(tiles.astype(np.int32), gpu)).cpu().numpy()
    af = a.double().numpy()  # bfloat16 rows reach the MFMA scaled into float16 exactly
    want = np.einsum("poi,pi->po", w[np.repeat(tiles, 16)], af)
    assert got.shape == want.shape and got.dtype == np.float32
    assert np.abs(got - want).max() <= 2e-6 * np.abs(want).max()


@pytest.mark.parametrize("kind", ["IQ3_XXS", "IQ3_S", "Q2_0"])
@pytest.mark.parametrize("cols", [512, 256])
def test_runs_of_an_experts_tiles_of_any_length(gpu, kind, cols):
    """The prompt kernels cut each run of one expert's consecutive tiles into chunks from the run's first tile:
    runs of 1 to 7 tiles, of 70 and of 300 (past the 256 tiles a look back covers at once), the same expert again
    after others, and tiles of no expert between them; every tile's product against the oracle's weights. Rows of 256
    columns (98 or 110 bytes, not whole dwords) take the kernels that load the fields straight into registers."""
    rng = np.random.default_rng(11)
    shape = (4, 64, cols)
    data, w = stack(kind, rng, *shape)
    w = w.astype(np.float32).astype(np.float64)  # exact for these types at whole blocks (see above)
    runs = [(2, 1), (0, 2), (1, 3), (4, 1), (3, 4), (2, 5), (0, 7), (1, 70), (0, 1), (4, 2), (3, 2), (0, 6), (2, 300),
            (3, 1)]
    tiles = np.concatenate([np.full(n, e) for e, n in runs])  # expert 4: no expert, left out
    a = torch.from_numpy(rng.standard_normal((16 * len(tiles), shape[2])).astype(np.float16))
    got = B.tile_matmul(dev(data, gpu), kind, shape, a.to(gpu), dev(tiles.astype(np.int32), gpu)).cpu().numpy()
    af = a.double().numpy()
    for t, e in enumerate(tiles):
        if e < shape[0]:
            want = af[16 * t:16 * t + 16] @ w[e].T
            assert np.abs(got[16 * t:16 * t + 16] - want).max() <= 2e-6 * np.abs(want).max(), (t, e)


def test_a_tile_of_no_expert_is_left_out(gpu):
    rng = np.random.default_rng(3)
    data, w = stack("Q2_0", rng, 4, 128, 192)
    tiles = np.array([1, 4, 2, 9])
    a = rng.standard_normal((64, 192)).astype(np.float16)
    out = torch.full((64, 128), 7.0, device=gpu)
    got = B.tile_matmul(dev(data, gpu), "Q2_0", (4, 128, 192), dev(a, gpu), dev(tiles.astype(np.int32), gpu),
                        out=out).cpu().numpy()
    for t in (0, 2):
        want = a[16 * t:16 * t + 16].astype(np.float64) @ w[tiles[t]].astype(np.float16).astype(np.float64).T
        assert np.abs(got[16 * t:16 * t + 16] - want).max() <= 2e-6 * np.abs(want).max()
    assert (got[16:32] == 7.0).all() and (got[48:64] == 7.0).all()


@pytest.mark.parametrize("kinds", [("Q2_0", "Q2_0"), ("IQ3_S", "IQ4_NL"), ("IQ3_XXS", "Q2_0")])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_a_prompt_through_tiles_is_the_prompt_a_pair_at_a_time(gpu, kinds, dtype):
    rng = np.random.default_rng(1)
    experts, hidden, inner, k = 7, 256, 64, 3
    mats = {}
    for name, kind, (rows, cols) in (("gate", kinds[0], (inner, hidden)), ("up", kinds[0], (inner, hidden)),
                                     ("down", kinds[1], (hidden, inner * 4))):
        data, w = stack(kind, rng, experts, rows, cols)
        mats[name] = (B.BlockSwitchLinear(dev(data, gpu), kind, w.shape), w.astype(np.float64))
    rows = 211
    x = rng.standard_normal((1, rows, hidden)).astype(np.float32)
    idx = rng.integers(0, experts - 1, (1, rows, k))
    idx[0, :40] = 2
    xs, ix = torch.from_numpy(x).to(dtype).to(gpu), dev(idx, gpu)
    t, token, where = B.tiles_of(ix, experts)
    a = xs.reshape(-1, hidden)[token.long()]
    xf = xs.double().cpu().numpy()[0]
    tol = 2e-3 if dtype == torch.float16 else 2e-5
    for name in ("gate", "up"):
        lin, w = mats[name]
        got = B.tile_matmul(lin.blocks, lin.kind, (experts, inner, hidden), a, t)[where.long()].reshape(1, rows, k, inner)
        want = np.einsum("tkoi,ti->tko", w[idx[0]], xf)
        assert np.abs(got.double().cpu().numpy()[0] - want).max() <= tol * np.abs(want).max()


def test_a_prompts_three_products_go_through_tiles(gpu):
    """switch_glu sends a chunk's pairs through the tiles, and what comes out is what a pair at a time gives."""
    rng = np.random.default_rng(1)
    experts, hidden, inner, k = 7, 128, 64, 3
    mats = {n: stack("Q2_0", rng, experts, r, c) for n, (r, c) in (("gate", (inner, hidden)), ("up", (inner, hidden)),
                                                                    ("down", (hidden, inner)))}
    lin = {n: B.BlockSwitchLinear(dev(d, gpu), "Q2_0", w.shape) for n, (d, w) in mats.items()}
    x = torch.from_numpy(rng.standard_normal((1, 211, hidden)).astype(np.float16)).to(gpu)
    idx = rng.integers(0, experts - 1, (1, 211, k))
    idx[0, :40] = 2
    glu = B.BlockSwitchGLU(lin["gate"], lin["up"], lin["down"])
    old = B.TILES_FROM
    try:
        B.TILES_FROM = 1 << 62
        a_pair = glu(x, dev(idx, gpu)).double().cpu().numpy()
        B.TILES_FROM = 100
        in_tiles = glu(x, dev(idx, gpu)).double().cpu().numpy()
    finally:
        B.TILES_FROM = old
    assert in_tiles.shape == a_pair.shape == (1, 211, k, hidden)
    xs = x.double().cpu().numpy()[0]
    g, u = (np.einsum("tkoi,ti->tko", mats[n][1][idx[0]].astype(np.float64), xs) for n in ("gate", "up"))
    want = np.einsum("tkoi,tki->tko", mats["down"][1][idx[0]].astype(np.float64), g / (1 + np.exp(-g)) * u)
    scale = np.abs(want).max()
    assert np.abs(a_pair[0] - want).max() <= 5e-3 * scale
    assert np.abs(in_tiles[0] - want).max() <= 5e-3 * scale


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prompt_chunk_at_model_shape(gpu, dtype):
    """512 tokens, top-8 of 32 experts of 1536 x 4096 IQ3_XXS: gate, up and down against the oracle at 1e-3
    relative L2 (float32 sums)."""
    rng = np.random.default_rng(4)
    E, H, F, k, T = 32, 4096, 1536, 8, 512
    mats = {}
    for name, (r, c) in (("gate", (F, H)), ("up", (F, H)), ("down", (H, F))):
        data = O.random_blocks("IQ3_XXS", E * r * c // 256, rng, scale="normal")
        mats[name] = (B.BlockSwitchLinear(dev(data, gpu), "IQ3_XXS", (E, r, c)), data)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])[None]
    x = torch.from_numpy(rng.standard_normal((1, T, H)).astype(np.float32)).to(dtype).to(gpu)
    t, token, where = B.tiles_of(dev(idx, gpu), E)
    a = x.reshape(-1, H)[token.long()]
    lin, data = mats["gate"]
    got = B.tile_matmul(lin.blocks, "IQ3_XXS", (E, F, H), a, t)[where.long()].cpu().numpy()
    w = O.dequantize(data, "IQ3_XXS", (E, F, H))
    want = O.expert_matvec(w, idx.reshape(-1), x.float().cpu().numpy().reshape(T, H), k)
    assert np.linalg.norm(got - want) <= 1e-3 * np.linalg.norm(want)
