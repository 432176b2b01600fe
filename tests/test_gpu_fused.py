"""The router, its choice of experts and the combine on the GPU (strata_mlx/fused.py:334-497) against the oracle:
the router's float32 sums within 1e-5 of the float64 product (tests/test_fused.py of the reference compares with
MLX's own product at its tolerance); the experts chosen exactly, ties included, and their weights within 1e-6; the
combine bit for bit (the sigmoid's exp may move one element in a hundred by one float16 step)."""

import numpy as np
import pytest
import torch

from oracle import fused as OF
from strata_mlx_amd import fused as FU

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tokens", [1, 3, 8, 11])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_router_sums_are_the_product(gpu, tokens, dtype):
    rng = np.random.default_rng(tokens)
    w = (rng.standard_normal((256, 4096)) / 64).astype(np.float16)
    x = rng.standard_normal((tokens, 4096)).astype(np.float32)
    router = FU.WindowLinear(torch.from_numpy(w).to(gpu))
    got = router(torch.from_numpy(x).to(dtype).to(gpu)).cpu().numpy()
    xin = torch.from_numpy(x).to(dtype).float().numpy()
    want = OF.router_matvec(w, xin)
    assert got.dtype == np.float32 and got.shape == (tokens, 256)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("n,k", [(256, 8), (512, 10), (64, 1), (2048, 64), (100, 7)])
def test_top_k_chooses_as_a_stable_sort_and_weights_by_softmax(gpu, n, k):
    rng = np.random.default_rng(n + k)
    rows = 37
    logits = rng.integers(-5, 6, (rows, n)).astype(np.float32)  # ties everywhere
    logits[::3] = rng.standard_normal((len(logits[::3]), n)).astype(np.float32)
    idx, wts = FU.top_k(torch.from_numpy(logits).to(gpu), k, weights=True)
    want = OF.top_k(logits, k)
    assert np.array_equal(idx.cpu().numpy(), want)
    np.testing.assert_allclose(wts.cpu().numpy(), OF.softmax_k(logits, want), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("rows,k,d", [(1, 8, 4096), (4, 8, 4096), (2, 4, 1024), (5, 6, 768), (16, 10, 512),
                                      (3, 20, 256)])
def test_combine_has_the_references_bits(gpu, rows, k, d):
    rng = np.random.default_rng(rows * k)
    y = (rng.standard_normal((rows, k, d)) * 4).astype(np.float16)
    w = rng.dirichlet(np.ones(k), rows).astype(np.float32)
    g = rng.standard_normal(rows).astype(np.float16)
    s = rng.standard_normal((rows, d)).astype(np.float16)
    dev = lambda a: torch.from_numpy(a).to(gpu)
    got = FU.moe_combine(dev(y), dev(w), dev(g).reshape(rows, 1), dev(s)).cpu().numpy()
    want = OF.moe_combine(y, w, g, s)
    gb, wb = got.view(np.int16).astype(np.int32), want.view(np.int16).astype(np.int32)
    assert np.abs(gb - wb).max() <= 1 and (gb != wb).mean() <= 0.01


def test_combine_declines_what_the_reference_declines(gpu):
    y = torch.zeros((17, 8, 256), dtype=torch.float16, device=gpu)  # more tokens than COMBINE_UPTO
    w = torch.zeros((17, 8), device=gpu)
    assert FU.moe_combine(y, w, torch.zeros((17, 1), dtype=torch.float16, device=gpu),
                          torch.zeros((17, 256), dtype=torch.float16, device=gpu)) is None


def test_route_gives_experts_and_weights_of_the_router(gpu):
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((256, 1024)) / 32).astype(np.float16)
    x = rng.standard_normal((4, 1024)).astype(np.float16)
    idx, wts = FU.route(FU.WindowLinear(torch.from_numpy(w).to(gpu)), torch.from_numpy(x).to(gpu), 8)
    logits = OF.router_matvec(w, x.astype(np.float32)).astype(np.float32)
    want = OF.top_k(logits, 8)
    # a near-tie between float32 sums may order two experts differently; the chosen set is the oracle's
    assert all(set(a) == set(b) for a, b in zip(idx.cpu().numpy(), want))
    assert np.allclose(wts.sum(dim=-1).cpu().numpy(), 1.0, atol=1e-6)


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return np.linalg.norm(got - want) / np.linalg.norm(want)


# The whole MoE block (strata_mlx/fused.py:484-497): router, top-k, IQ3_S routed experts (SwitchGLU), a Q4_K shared
# expert and its sigmoid gate, the combine; at one token with the shared expert in the routed launches, at two
# apart, at 20 past the router's and the combine's kernels (torch's product, the reference's fallback sum in
# float32). Against the oracle's chain on the library's own choice of experts (checked above): float64 products of
# the oracle's weights, h as mlx-lm's SwiGLU rounds it, y and s rounded to float16, the reference's combine, within
# 2e-3 relative L2 (an h on the other side of a rounding boundary moves a few elements by a float16 step).
@pytest.mark.parametrize("tokens", [1, 2, 20])
def test_moe_block_against_the_oracle(gpu, tokens):
    from oracle import blocks as O
    from strata_mlx_amd import blocks as B
    from strata_mlx_amd import dense as D
    from strata_mlx_amd import synth
    H, F, E, K = 4096, 1536, 10, 8
    g = torch.Generator(device=gpu).manual_seed(41 + tokens)
    shapes = ((F, H), (F, H), (H, F))
    stacks = [synth.random_stack("IQ3_S", E * r * c, gpu, g) for r, c in shapes]
    switch = B.BlockSwitchGLU(*(B.BlockSwitchLinear(st, "IQ3_S", (E, r, c)) for st, (r, c) in zip(stacks, shapes)))
    shared = [D.BlockLinear(synth.random_stack("Q4_K", r * c, gpu, g), "Q4_K", (r, c)) for r, c in shapes]
    rng = np.random.default_rng(tokens)
    rw = (rng.standard_normal((E, H)) / 64).astype(np.float16)
    gw = (rng.standard_normal((1, H)) / 64).astype(np.float16)
    router = FU.WindowLinear(torch.from_numpy(rw).to(gpu))
    moe = FU.RoutedMoE(router, switch, *shared, FU.WindowLinear(torch.from_numpy(gw).to(gpu)), K)
    x = (rng.standard_normal((tokens, H)) / 64).astype(np.float16)
    xs = torch.from_numpy(x).to(gpu)
    out = moe(xs)
    assert out.shape == (tokens, H) and out.dtype == (torch.float16 if tokens <= FU.COMBINE_UPTO else torch.float32)
    assert moe.last_path == ("choice in the launch" if tokens == 1 else "apart")
    idx_t, w_t = FU.route(router, xs, K)
    idx, w = idx_t.cpu().numpy(), w_t.cpu().numpy()
    got = out.float().cpu().numpy()

    xd = x.astype(np.float64)
    raw = [st.cpu().numpy().reshape(E, -1) for st in stacks]
    y = np.zeros((tokens, K, H), np.float16)
    for e in np.unique(idx):
        gate, up, down = (O.dequantize(raw[i][e], "IQ3_S", shapes[i]).astype(np.float64) for i in range(3))
        for t, j in zip(*np.nonzero(idx == e)):
            h = O.swiglu_rounded(gate @ xd[t], up @ xd[t], np.float16).astype(np.float64)
            y[t, j] = (down @ h).astype(np.float16)
    sgw, suw, sdw = (O.dequantize(lay.blocks.cpu().numpy(), "Q4_K", (lay.output_dims, lay.input_dims))
                     .astype(np.float64) for lay in shared)
    sh = O.swiglu_rounded(xd @ sgw.T, xd @ suw.T, np.float16).astype(np.float64)
    s = (sh @ sdw.T).astype(np.float16)
    gl = (xd @ gw.astype(np.float64).T).reshape(tokens).astype(np.float16)
    want = OF.moe_combine(y, w, gl, s)
    assert rel_l2(got, want) <= 2e-3


# The router's product and the choice in one launch (strata_router_route) against the two launches it replaces:
# the same experts, the same weights' bits, the rows past the experts (a shared expert's gate) the router's float32
# sums rounded once to float16; calls in a row and graph replays (the launch's count returns to zero each time).
@pytest.mark.parametrize("tokens,experts,extra,k", [(1, 256, 1, 8), (3, 256, 0, 8), (8, 100, 3, 7), (5, 64, 1, 64),
                                                    (2, 2048, 2, 10)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_router_and_choice_in_one_launch(gpu, tokens, experts, extra, k, dtype):
    rng = np.random.default_rng(tokens * 31 + experts + extra)
    wt = (rng.standard_normal((experts + extra, 4096)) / 64).astype(np.float16)
    stacked = FU.WindowLinear(torch.from_numpy(wt).to(gpu))
    router = FU.WindowLinear(torch.from_numpy(wt[:experts]).to(gpu))
    xs = [torch.from_numpy(rng.standard_normal((tokens, 4096)).astype(np.float32)).to(dtype).to(gpu) for _ in range(3)]

    def check(got, x):
        idx, w, ex = got
        want_idx, want_w = FU.route(router, x, k)
        assert torch.equal(idx, want_idx)
        assert torch.equal(w.view(torch.int32), want_w.view(torch.int32))
        if extra:
            want_ex = stacked(x)[:, experts:].to(torch.float16)
            assert torch.equal(ex.view(torch.int16), want_ex.view(torch.int16))
        else:
            assert ex is None

    for x in xs:  # calls in a row
        check(FU.route_gated(stacked, x, experts, k), x)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        FU.route_gated(stacked, xs[0], experts, k)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    x_in = xs[0].clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = FU.route_gated(stacked, x_in, experts, k)
    for r in range(3):
        x_in.copy_(xs[r])
        graph.replay()
        torch.cuda.synchronize()
        check(got, xs[r])
        FU.route_gated(stacked, xs[(r + 1) % 3], experts, k)  # eager work between the replays
        torch.cuda.synchronize()
    assert FU.route_gated(stacked, torch.cat([xs[0]] * 9)[:9], experts, k) is None  # 9 tokens: the calls apart


# The routed gate/up launch that makes the choice of experts itself from the router's logits
# (strata_moe_gate_up_swiglu_shared) against the calls it replaces, top_k on the logits then the gate/up launch with
# the shared expert: the same experts, the weights', h's and the shared expert's h's bits, the rows past the experts
# rounded once to float16. Logits with ties, -inf, and NaN (never chosen; a row of NaN chooses no expert, as top_k,
# and h is then NaN); calls in a row; a shape the form does not take (ten pairs) declines.
@pytest.mark.parametrize("kind,experts,extra,k", [("IQ3_S", 256, 1, 8), ("IQ3_S", 10, 1, 8), ("IQ3_S", 64, 0, 6),
                                                  ("Q2_0", 256, 1, 8), ("IQ3_S", 256, 1, 10)])
def test_gate_up_with_the_choice_in_the_launch(gpu, kind, experts, extra, k):
    from strata_mlx_amd import blocks as B
    from strata_mlx_amd import dense as D
    from strata_mlx_amd import synth
    F, H = 1536, 4096
    g = torch.Generator(device=gpu).manual_seed(experts * 7 + k)
    gate, up = (B.BlockSwitchLinear(synth.random_stack(kind, experts * F * H, gpu, g), kind, (experts, F, H))
                for _ in range(2))
    sg, su = (D.BlockLinear(synth.random_stack("Q4_K", F * H, gpu, g), "Q4_K", (F, H)) for _ in range(2))
    rng = np.random.default_rng(experts + k)
    n = experts + extra
    cases = [rng.standard_normal(n).astype(np.float32) for _ in range(2)]
    tied = np.round(rng.standard_normal(n), 1).astype(np.float32)  # many ties
    odd = rng.standard_normal(n).astype(np.float32)
    odd[::3] = np.nan
    odd[1::7] = -np.inf
    cases += [tied, odd, np.full(n, np.nan, np.float32)]
    x = torch.from_numpy((rng.standard_normal((1, H)) / 64).astype(np.float16)).to(gpu)

    def same(a, b):  # the same bits, or NaN at both
        bits = a.view(torch.int16 if a.dtype == torch.float16 else torch.int32)
        want = b.view(bits.dtype)
        return bool(((bits == want) | (torch.isnan(a) & torch.isnan(b))).all())

    for lg in cases:
        logits = torch.from_numpy(lg).reshape(1, n).to(gpu)
        got = B.moe_gate_up_swiglu_shared(gate, up, x, logits, experts, k, sg, su)
        if k > 8:
            assert got is None
            return
        h, idx, w, sh, ex = got
        want_idx, want_w = FU.top_k(logits[:, :experts].contiguous(), k, weights=True)
        assert torch.equal(idx, want_idx.reshape(k))
        assert same(w, want_w.reshape(k))
        _, _, want_h, want_sh = B.gate_up_swiglu_shared(gate, up, x, want_idx.reshape(k), sg, su)
        assert same(h, want_h) and torch.equal(sh.view(torch.int16), want_sh.view(torch.int16))
        if extra:
            assert same(ex, logits[:, experts:].to(torch.float16))
        else:
            assert ex is None
        if np.isnan(lg[:experts]).all():
            assert torch.isnan(h).all() and not torch.isnan(sh).any()
