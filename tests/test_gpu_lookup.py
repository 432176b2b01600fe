"""The Q2_0 table of sums on the GPU (strata_mlx/blocks.py:697-928) against oracle/lookup.py: the tables bit for
bit (the table of silu(g) * u within one float16 step on at most one entry in a hundred: expf and numpy's exp may
round a sigmoid differently); the products bit for bit against the oracle's float32 steps (its fused multiply-add
is emulated in float64, which may round an extreme case differently: one float16 step on one output in a thousand
at most); gate and up in one launch give the bits of two (test_blocks.py:233-249), down building its own table
gives the bits of the separate table (test_blocks.py:215-229); and a layer through switch_glu is the float64
product within 2e-3 relative L2 (the table's sums are float16)."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from oracle import lookup as LK
from strata_mlx_amd import blocks as B

pytestmark = pytest.mark.gpu

EXPERTS = 6


def dev(a, gpu):
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def stack(rng, rows, cols, gpu):
    data = O.random_blocks("Q2_0", EXPERTS * rows * cols // 64, rng)
    return data, B.BlockSwitchLinear(dev(data, gpu), "Q2_0", (EXPERTS, rows, cols))


def close_bits(got, want, frac):
    g, w = got.view(np.int16).astype(np.int32), want.view(np.int16).astype(np.int32)
    assert np.abs(g - w).max() <= 1 and (g != w).mean() <= frac


@pytest.mark.parametrize("cols", [64, 640, 2560, 4096])
def test_tables_are_the_oracles(gpu, cols):
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((3, cols)).astype(np.float16)
    got = B.lookup_table(dev(x, gpu)).cpu().numpy()
    assert got.shape == (3, cols // 2, 16) and np.array_equal(got, LK.lookup_table(x))
    g, u = rng.standard_normal((2, 3, cols)).astype(np.float16)
    got = B.lookup_table_glu(dev(g, gpu), dev(u, gpu)).cpu().numpy()
    close_bits(got, LK.lookup_table_glu(g, u), 0.01)


@pytest.mark.parametrize("rows,cols,pairs,share", [(64, 2560, 8, 2), (40, 640, 30, 1), (96, 128, 10, 1),
                                                   (40, 2048, 12, 4), (1536, 4096, 8, 8)])
def test_products_are_the_oracles(gpu, rows, cols, pairs, share):
    rng = np.random.default_rng(rows + cols)
    data, lin = stack(rng, rows, cols, gpu)
    idx = rng.integers(0, EXPERTS, pairs)
    x = rng.standard_normal((pairs // share, cols)).astype(np.float16)
    table = B.lookup_table(dev(x, gpu))
    got = B.lookup_matvec(lin, dev(idx, gpu), table, share).cpu().numpy()
    want = LK.lookup_matvec(data, (EXPERTS, rows, cols), idx, LK.lookup_table(x), share,
                            B._lookup_per_row(cols, pairs))
    close_bits(got, want, 0.001)


@pytest.mark.parametrize("tokens", [1, 4, 8])
@pytest.mark.parametrize("rows,cols", [(64, 2560), (40, 640)])
def test_gate_and_up_in_one_launch_give_the_bits_of_two(gpu, tokens, rows, cols):
    rng = np.random.default_rng(tokens + rows)
    (_, gate), (_, up), k = stack(rng, rows, cols, gpu), stack(rng, rows, cols, gpu), 2
    idx = dev(rng.integers(0, EXPERTS, tokens * k), gpu)
    table = B.lookup_table(dev(rng.standard_normal((tokens, cols)).astype(np.float16), gpu))
    g, u = B.lookup_gate_up(gate, up, idx, table, k)
    assert torch.equal(g, B.lookup_matvec(gate, idx, table, k)) and torch.equal(u, B.lookup_matvec(up, idx, table, k))


@pytest.mark.parametrize("pairs", [1, 10, 30])
@pytest.mark.parametrize("rows,cols", [(256, 640), (96, 128), (40, 2048)])
def test_the_table_built_in_down_gives_the_bits_of_its_own_launch(gpu, pairs, rows, cols):
    rng = np.random.default_rng(pairs + rows)
    _, down = stack(rng, rows, cols, gpu)
    idx = dev(rng.integers(0, EXPERTS, pairs), gpu)
    gate = dev(rng.standard_normal((pairs, cols)).astype(np.float16), gpu)
    up = dev(rng.standard_normal((pairs, cols)).astype(np.float16), gpu)
    got = B.lookup_down_glu(down, idx, gate, up)
    assert got is not None and got.dtype == torch.float16
    assert torch.equal(got, B.lookup_matvec(down, idx, B.lookup_table_glu(gate, up), 1))


@pytest.fixture
def lookup_dispatch():
    old = B.LOOKUP_GLU
    B.LOOKUP_GLU = True  # switch_glu takes the table of sums for Q2_0 over float16, as the reference's does
    yield
    B.LOOKUP_GLU = old


def test_a_layer_through_switch_glu_is_the_product(gpu, lookup_dispatch):
    """Config 3's shape: 5 tokens x top-8 over Q2_0 gate/up 1536 x 4096, down 4096 x 1536, through the table path
    (float16 sums: 2e-3 relative L2)."""
    rng = np.random.default_rng(3)
    E, H, F, k, tokens = 16, 4096, 1536, 8, 5
    mats = {n: O.random_blocks("Q2_0", E * r * c // 64, rng, scale="normal")
            for n, (r, c) in (("gate", (F, H)), ("up", (F, H)), ("down", (H, F)))}
    shapes = {"gate": (E, F, H), "up": (E, F, H), "down": (E, H, F)}
    lin = {n: B.BlockSwitchLinear(dev(d, gpu), "Q2_0", shapes[n]) for n, d in mats.items()}
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(tokens)])
    x = (rng.standard_normal((tokens, H)) / 64).astype(np.float16)
    got = B.switch_glu(dev(x, gpu), dev(idx, gpu), lin["up"], lin["gate"], lin["down"]).float().cpu().numpy()
    assert got.shape == (tokens, k, H)
    w = {n: O.dequantize(d, "Q2_0", shapes[n]) for n, d in mats.items()}
    flat = idx.reshape(-1)
    g64 = O.expert_matvec(w["gate"], flat, x, k)
    u64 = O.expert_matvec(w["up"], flat, x, k)
    h = g64 / (1 + np.exp(-g64)) * u64
    want = O.expert_matvec(w["down"], flat, h, 1)
    assert np.linalg.norm(got.reshape(-1, H) - want) <= 2e-3 * np.linalg.norm(want)


def test_a_pair_naming_no_expert_gives_nan(gpu):
    rng = np.random.default_rng(4)
    _, lin = stack(rng, 32, 256, gpu)
    table = B.lookup_table(dev(rng.standard_normal((2, 256)).astype(np.float16), gpu))
    out = B.lookup_matvec(lin, dev(np.array([1, EXPERTS + 3]), gpu), table, 1).cpu().numpy()
    assert np.isfinite(out[0]).all() and np.isnan(out[1]).all()
