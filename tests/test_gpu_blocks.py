"""The kernels on the file's blocks give the oracle's weights and products (tests/test_blocks.py, test_dense.py of
the reference, restated against the CPU oracle).

Dequant is bit-exact; products are within the reference's own tolerances against the float64 product of the
oracle's weights: 1e-5 * max|w| * sqrt(cols) for float32 activations (test_blocks.py:35), 2e-3 relative for
float16 (test_blocks.py:65), 2e-5 / 4e-3 for the dense window (test_dense.py:49).
"""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B

pytestmark = pytest.mark.gpu

KINDS = ["Q2_0", "IQ4_NL", "IQ4_XS", "IQ3_S", "IQ3_XXS", "Q3_K", "Q4_K", "Q6_K", "Q8_0", "Q4_0", "Q5_0", "Q5_K"]
EXPERTS, OUT = 3, 2  # 6 rows of 2560: three experts of two rows (test_blocks.py:10)


def tensor(kind, seed, rows=6, cols=2560, **kw):
    per = O.BY_NAME[kind][1]
    rng = np.random.default_rng(seed)
    data = O.random_blocks(kind, rows * cols // per, rng, **kw)
    return data, O.dequantize(data, kind, (rows, cols))


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_unpacked_blocks_are_the_oracle_weights_bit_for_bit(gpu, kind, dtype):
    data, want = tensor(kind, 0)
    got = B.dequantize(dev(data, gpu), kind, want.shape, dtype).cpu().numpy()
    want = want.astype(np.float16) if dtype == torch.float16 else want
    assert got.dtype == want.dtype and got.shape == want.shape
    np.testing.assert_array_equal(got.view(np.uint16 if dtype == torch.float16 else np.uint32),
                                  want.view(np.uint16 if dtype == torch.float16 else np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_of_a_stack_with_extreme_scales(gpu, kind):
    """Scales at fp16's extremes (subnormal, near 65504, negative): still the closed form, bit for bit."""
    per, size = O.BY_NAME[kind][1:]
    rng = np.random.default_rng(11)
    n = 3 * 2 * 512 // per
    data = rng.integers(0, 256, (n, size), dtype=np.uint8)
    special = np.array([0x0001, 0x03FF, 0x0400, 0x7BFF, 0x8001, 0xFBFF, 0x3C00, 0x0000], dtype="<u2")
    for at in O.SCALE_BYTES[kind]:
        data[:, at:at + 2] = special[rng.integers(0, len(special), n)].view(np.uint8).reshape(n, 2)
    data = data.reshape(-1)
    want = O.dequantize(data, kind, (3, 2, 512))
    got = B.dequantize(dev(data, gpu), kind, (3, 2, 512)).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_products_on_blocks_are_products_on_the_weights(gpu, kind):
    data, w = tensor(kind, 1)
    w = w.reshape(EXPERTS, OUT, -1)
    layer = B.BlockSwitchLinear(dev(data, gpu), kind, w.shape)
    rng = np.random.default_rng(2)
    idx = np.array([[2, 0], [1, 1], [0, 2], [2, 2], [0, 1]])  # five tokens, two experts each (one twice)
    scale = np.abs(w).max() * np.sqrt(w.shape[-1])

    x = rng.standard_normal((5, 1, 1, w.shape[-1])).astype(np.float32)  # a row to each token: gate and up
    got = layer(dev(x, gpu), dev(idx, gpu)).cpu().numpy()
    assert got.shape == (5, 2, 1, OUT)
    want = np.einsum("tkoi,ti->tko", w[idx].astype(np.float64), x[:, 0, 0].astype(np.float64))
    assert np.abs(got[:, :, 0] - want).max() <= 1e-5 * scale

    x = rng.standard_normal((5, 2, 1, w.shape[-1])).astype(np.float32)  # a row to each pair: down
    got = layer(dev(x, gpu), dev(idx, gpu)).cpu().numpy()
    want = np.einsum("tkoi,tki->tko", w[idx].astype(np.float64), x[:, :, 0].astype(np.float64))
    assert np.abs(got[:, :, 0] - want).max() <= 1e-5 * scale


@pytest.mark.parametrize("kind", ["IQ3_XXS", "IQ3_S", "Q2_0"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_half_precision_activations_come_back_in_their_type(gpu, kind, dtype):
    data, w = tensor(kind, 5)
    w = w.reshape(EXPERTS, OUT, -1)
    layer = B.BlockSwitchLinear(dev(data, gpu), kind, w.shape)
    x = torch.randn((2, 1, 1, 2560), generator=torch.Generator().manual_seed(0)).to(dtype).to(gpu)
    idx = dev(np.array([[0, 1], [2, 0]]), gpu)
    out = layer(x, idx)
    assert out.dtype == dtype and out.shape == (2, 2, 1, OUT)
    want = layer(x.float(), idx)
    tol = 2e-3 if dtype == torch.float16 else 8e-3
    assert (out.float() - want).abs().max().item() <= tol * want.abs().max().item()


@pytest.mark.parametrize("kind", ["IQ3_S", "Q2_0", "IQ3_XXS", "IQ4_NL"])
@pytest.mark.parametrize("tokens", [1, 4, 5])
def test_routed_decode_at_model_shape(gpu, kind, tokens):
    """Gate/up (1536 x 4096) and down with SwiGLU (4096 x 1536), 16 experts, top-8: against the oracle at
    1e-3 relative L2 (float16 activations, float32 sums)."""
    rng = np.random.default_rng(tokens)
    E, H, F, k = 16, 4096, 1536, 8
    per = O.BY_NAME[kind][1]
    mats = {}
    for name, (rows, cols) in (("gate", (F, H)), ("up", (F, H)), ("down", (H, F))):
        data = O.random_blocks(kind, E * rows * cols // per, rng, scale="normal")
        mats[name] = (data, (E, rows, cols))
    lin = {n: B.BlockSwitchLinear(dev(d, gpu), kind, s) for n, (d, s) in mats.items()}
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(tokens)])
    # activations at 1/64 keep gate, up and down inside float16's range with these scales (|w| ~ 1)
    x = (rng.standard_normal((tokens, H)) / 64).astype(np.float16)
    xs = dev(x, gpu)
    g, u = B.gate_up(lin["gate"], lin["up"], xs, dev(idx, gpu), k)
    y = B.matvec_glu(lin["down"], dev(idx.reshape(-1), gpu), g, u)
    used = np.unique(idx)
    w = {n: np.zeros((E,) + s[1:], np.float32) for n, (d, s) in mats.items()}
    for n, (d, s) in mats.items():
        rb = B.row_bytes(kind, s[2])
        for e in used:
            w[n][e] = O.dequantize(d[e * s[1] * rb:(e + 1) * s[1] * rb], kind, s[1:])
    flat = idx.reshape(-1)
    g64 = O.expert_matvec(w["gate"], flat, x, k)
    u64 = O.expert_matvec(w["up"], flat, x, k)
    for got, want in ((g, g64), (u, u64)):
        got = got.float().cpu().numpy()
        assert np.linalg.norm(got - want) <= 1e-3 * np.linalg.norm(want)
    h = O.swiglu_rounded(g.cpu().numpy(), u.cpu().numpy(), np.float16)  # down's own input, from the kernel's g, u
    y64 = O.expert_matvec(w["down"], flat, h, 1)
    got = y.float().cpu().numpy()
    assert np.linalg.norm(got - y64) <= 1e-3 * np.linalg.norm(y64)


def test_a_pair_naming_no_expert_gives_nan_and_reads_nothing(gpu):
    data, w = tensor("IQ3_S", 3)
    layer = B.BlockSwitchLinear(dev(data, gpu), "IQ3_S", (EXPERTS, OUT, 2560))
    x = torch.ones((2, 1, 1, 2560), device=gpu)
    out = layer(x, dev(np.array([[0, 7], [1, 2]]), gpu)).cpu().numpy()
    assert np.isnan(out[0, 1]).all() and np.isfinite(out[0, 0]).all() and np.isfinite(out[1]).all()


@pytest.mark.parametrize("kind", ["IQ3_S", "IQ4_NL", "Q2_0"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_down_taking_swiglu_itself_is_swiglu_then_down(gpu, kind, dtype):
    """matvec_glu == matvec of the SwiGLU as mlx-lm rounds it (test_blocks.py:252-275): bit-equal when the
    SwiGLU agrees, which it does unless expf and the oracle's exp round a sigmoid differently."""
    rng = np.random.default_rng(7)
    per = O.BY_NAME[kind][1]
    data = O.random_blocks(kind, 6 * 512 * 256 // per, rng)
    down = B.BlockSwitchLinear(dev(data, gpu), kind, (6, 512, 256))
    pairs = 12
    idx = dev(rng.integers(0, 6, pairs), gpu)
    gate = dev(rng.standard_normal((pairs, 256)).astype(np.float32), gpu).to(dtype)
    up = dev(rng.standard_normal((pairs, 256)).astype(np.float32), gpu).to(dtype)
    got = B.matvec_glu(down, idx, gate, up)
    h = O.swiglu_rounded(gate.float().cpu().numpy(), up.float().cpu().numpy(),
                         np.float16 if dtype == torch.float16 else np.float32)
    want = down(dev(h, gpu).reshape(pairs, 1, 256), idx.reshape(pairs, 1).squeeze(-1).reshape(pairs))
    want = want.reshape(pairs, 512)
    diff = (got.float() - want.float()).abs().max().item()
    assert diff <= (1e-3 if dtype == torch.float16 else 1e-5) * want.float().abs().max().item()


@pytest.mark.parametrize("kind", ["IQ3_S", "Q4_K"])
def test_separate_buffers_give_the_bits_of_the_stack(gpu, kind):
    data, w = tensor(kind, 4)
    stack = dev(data, gpu)
    layer = B.BlockSwitchLinear(stack, kind, (EXPERTS, OUT, 2560))
    rb = B.row_bytes(kind, 2560)
    experts = [stack[e * OUT * rb:(e + 1) * OUT * rb].clone() for e in (2, 0, 1, 1)]
    x = torch.randn((2, 2560), generator=torch.Generator().manual_seed(1)).half().to(gpu)
    got = B.matvec_separate(experts, kind, OUT, 2560, x, 2)
    want = layer(x.reshape(2, 1, 1, 2560), dev(np.array([[2, 0], [1, 1]]), gpu)).reshape(4, OUT)
    assert torch.equal(got, want)


@pytest.mark.parametrize("kind", ["Q6_K", "Q8_0", "Q4_K", "Q3_K", "IQ4_XS"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 5, 7, 8, 12])
def test_a_window_multiplies_as_the_weights_do(gpu, kind, dtype, tokens):
    data, w = tensor(kind, tokens, rows=12, cols=1024)
    x = torch.randn((tokens, 1024), generator=torch.Generator().manual_seed(tokens)).to(dtype)
    got = B.window_matvec(dev(data, gpu), kind, 12, 1024, x.to(gpu)).float().cpu().numpy()
    want = x.double().numpy() @ w.astype(np.float64).T
    assert got.shape == (tokens, 12)
    assert np.abs(got - want).max() <= (2e-5 if dtype == torch.float32 else 4e-3) * np.abs(want).max()


@pytest.mark.parametrize("kind", ["Q6_K", "IQ4_XS", "Q3_K"])
def test_a_token_gets_the_same_bits_alone_as_in_a_window(gpu, kind):
    data, _ = tensor(kind, 3, rows=40, cols=2048)
    blocks = dev(data, gpu)
    x = torch.randn((9, 2048), generator=torch.Generator().manual_seed(3)).half().to(gpu)
    together = B.window_matvec(blocks, kind, 40, 2048, x)
    for i in range(9):
        assert torch.equal(B.window_matvec(blocks, kind, 40, 2048, x[i:i + 1]), together[i:i + 1])


def test_listed_rows_have_the_layers_own_bits(gpu):
    """The lm_head row list of strata_mlx/rows.py:30-42: rows by id give the full layer's outputs, bit for bit;
    an id past the layer gives NaN."""
    data, _ = tensor("Q6_K", 9, rows=400, cols=256)
    blocks = dev(data, gpu)
    x = torch.randn((1, 256), generator=torch.Generator().manual_seed(2)).half().to(gpu)
    full = B.window_matvec(blocks, "Q6_K", 400, 256, x, out_dtype=torch.float32)
    ids = torch.tensor([5, 399, 0, 17, 17, 250, 3, 101, 77], dtype=torch.int32, device=gpu)
    got = B.window_matvec(blocks, "Q6_K", 400, 256, x, row_ids=ids, out_dtype=torch.float32)
    assert torch.equal(got, full[:, ids.long()])
    bad = B.window_matvec(blocks, "Q6_K", 400, 256, x, row_ids=torch.tensor([1, 400], dtype=torch.int32, device=gpu))
    assert torch.isfinite(bad[0, 0]) and torch.isnan(bad[0, 1])


def _h_matches_swiglu(h, g, u):
    """h against the oracle's SwiGLU of the same g, u: equal, or one float16 step apart where the device expf and
    the oracle's exp round a sigmoid differently (at most 1 in 100 elements)."""
    want = O.swiglu_rounded(g, u, np.float16)
    hb, wb = h.view(np.int16).astype(np.int32), want.view(np.int16).astype(np.int32)
    off = hb != wb
    assert np.abs(hb - wb).max() <= 1
    assert off.mean() <= 0.01


@pytest.mark.parametrize("kind,dtype", [("IQ3_S", torch.float16), ("IQ3_XXS", torch.float16), ("Q2_0", torch.float16),
                                        ("Q4_K", torch.float16), ("IQ3_S", torch.float32)])
def test_gate_up_with_swiglu_gives_gate_up_and_their_swiglu(gpu, kind, dtype):
    """The paired launch (float16 IQ3_S / IQ3_XXS / Q2_0) and the two-launch form (other types and dtypes) give
    gate_up's own bits for gate and up, and the SwiGLU of those bits."""
    rng = np.random.default_rng(11)
    per = O.BY_NAME[kind][1]
    E, F, H, tokens, k = 8, 96, 1024, 3, 4
    stacks = [O.random_blocks(kind, E * F * H // per, rng, scale="normal") for _ in range(2)]
    gate, up = (B.BlockSwitchLinear(dev(d, gpu), kind, (E, F, H)) for d in stacks)
    idx = dev(np.stack([rng.choice(E, k, replace=False) for _ in range(tokens)]).reshape(-1), gpu)
    x = dev((rng.standard_normal((tokens, H)) / 16).astype(np.float32), gpu).to(dtype)
    g0, u0 = B.gate_up(gate, up, x, idx, k)
    g, u, h = B.gate_up_swiglu(gate, up, x, idx, k)
    assert torch.equal(g, g0) and torch.equal(u, u0)
    if dtype == torch.float16:
        _h_matches_swiglu(h.cpu().numpy(), g.cpu().numpy(), u.cpu().numpy())
    else:
        want = O.swiglu_rounded(g.cpu().numpy(), u.cpu().numpy(), np.float32)
        np.testing.assert_allclose(h.cpu().numpy(), want, rtol=1e-6, atol=1e-30)


@pytest.mark.parametrize("kind", ["IQ3_S", "IQ3_XXS", "Q2_0"])
@pytest.mark.parametrize("rows,cols", [(37, 512), (64, 2048), (5, 4096)])
def test_many_pairs_on_few_experts_match_each_pair_alone(gpu, kind, rows, cols):
    """200 pairs (25 tokens x top-8) over 16 experts: an expert's rows are read once and multiplied by every pair
    naming it. Each pair gets the bits it gets alone, and the products are the oracle's within 1e-3 relative L2.
    Rows that do not fill a work unit (37, 5) and rows shorter than a wave (512, 2048 inputs) included."""
    rng = np.random.default_rng(rows)
    per = O.BY_NAME[kind][1]
    E, tokens, k = 16, 25, 8
    data = O.random_blocks(kind, E * rows * cols // per, rng, scale="normal")
    lin = B.BlockSwitchLinear(dev(data, gpu), kind, (E, rows, cols))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(tokens)])
    x = (rng.standard_normal((tokens, cols)) / 32).astype(np.float16)
    xs, flat = dev(x, gpu), dev(idx.reshape(-1), gpu)
    together = B.expert_matvec(lin, flat, xs, k)
    per_token = B.expert_matvec(lin, flat, torch.repeat_interleave(xs, k, 0), 1)
    assert torch.equal(together, per_token)
    for p in (0, 7, 64, 130, 199):
        alone = B.expert_matvec(lin, flat[p:p + 1], xs[p // k:p // k + 1], 1)
        assert torch.equal(alone[0], together[p])
    w = O.dequantize(data, kind, (E, rows, cols))
    want = O.expert_matvec(w, idx.reshape(-1), x, k)
    got = together.float().cpu().numpy()
    assert np.linalg.norm(got - want) <= 1e-3 * np.linalg.norm(want)


@pytest.mark.parametrize("kind", ["IQ3_S", "IQ3_XXS", "Q2_0"])
@pytest.mark.parametrize("tokens", [1, 2, 3, 5, 12])
def test_a_float16_window_on_codebook_types(gpu, kind, tokens):
    data, w = tensor(kind, tokens, rows=40, cols=1024)
    x = (torch.randn((tokens, 1024), generator=torch.Generator().manual_seed(tokens)) / 8).half()
    got = B.window_matvec(dev(data, gpu), kind, 40, 1024, x.to(gpu)).float().cpu().numpy()
    want = x.double().numpy() @ w.astype(np.float64).T
    assert np.abs(got - want).max() <= 4e-3 * np.abs(want).max()
    one = B.window_matvec(dev(data, gpu), kind, 40, 1024, x[:1].to(gpu)).float().cpu().numpy()
    assert np.array_equal(one[0], got[0])
