"""The benchmark workloads at their own shapes, against the oracle: the kernel instances the benchmark times are
the ones checked here.

  decode    IQ3_S experts, 256 of 1536 x 4096 (gate, up) and 4096 x 1536 (down), top-8 of Zipf(1.1) routing,
            float16, one and four tokens, through BlockSwitchGLU (strata_mlx/blocks.py:958-996)
  speculate the same layer in Q2_0, five rows (1 + 4 draft tokens)
  dense     Q4_K 4096 x 4096 with float32 activations (the reference's CPU-path workload), and the mixed model's
            dense layers: Q6_K / Q8_0 attention projections, the Q4_K shared expert, lm_head 151936 x 4096 Q6_K
  prompt    512 tokens, IQ3_XXS, 256 experts top-8 Zipf, bfloat16, through the tiles (blocks.py:634-694)
  prefill   2048 tokens of the mixed model: IQ3_S experts through the tiles and the dense layers

Values: the blocks are the benchmark's (uniform bytes, fp16 scales |N(0,1)| * 0.01) and bfloat16 activations are
N(0,1). IQ3_S float16 activations are N(0,1) / 64: at N(0,1) the float16 SwiGLU of these random IQ3_S blocks
(|w| ~ 1.4, so |g| ~ 90 and |h| up to ~1e5) leaves float16's range, which the shapes and kernels do not depend on.

Tolerance: 1e-3 relative L2 against float64 products of the oracle's weights (float32 sums on the GPU), as the
reference's tests compare its kernels with float products (tests/test_blocks.py:35, 65, 107). Where every pair of
a 256-expert layer would make the numpy oracle slow, a sample is checked: whole experts (every pair naming them,
the heaviest expert included) or a sample of output rows.
"""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B
from strata_mlx_amd import dense as D
from strata_mlx_amd import synth

pytestmark = pytest.mark.gpu

E, H, F, K = 256, 4096, 1536, 8
REL = 1e-3


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return np.linalg.norm(got - want) / np.linalg.norm(want)


def as_dtype(v, dtype):
    """float64 values rounded once to a torch dtype, as float64: what an exact product gives in that type (the
    reference returns its products in the activations' type)."""
    return torch.from_numpy(np.asarray(v, np.float64)).to(dtype).double().numpy()


class Stack:
    """A stack of random blocks made on the GPU (synth.random_stack), with the oracle's weights of any expert or
    rows on demand (the bytes copied back and decoded by oracle/blocks.py)."""

    def __init__(self, kind, experts, rows, cols, seed, device):
        g = torch.Generator(device=device).manual_seed(seed)
        self.kind, self.shape = kind, (experts, rows, cols)
        self.blocks = synth.random_stack(kind, experts * rows * cols, device, g)
        self.rb = B.row_bytes(kind, cols)
        self.lin = B.BlockSwitchLinear(self.blocks, kind, self.shape)
        self._cache = {}

    def rows_bytes(self, e, rows):
        rows = np.asarray(rows, np.int64)
        at = torch.as_tensor((e * self.shape[1] + rows), device=self.blocks.device)
        raw = self.blocks.reshape(-1, self.rb).index_select(0, at)
        return raw.cpu().numpy().reshape(-1)

    def weights(self, e, rows=None):
        """Expert e's weights (rows x cols, float32), all rows or the listed ones."""
        if rows is None:
            if e not in self._cache:
                self._cache[e] = O.dequantize(self.rows_bytes(e, np.arange(self.shape[1])), self.kind,
                                              self.shape[1:])
            return self._cache[e]
        return O.dequantize(self.rows_bytes(e, rows), self.kind, (len(rows), self.shape[2]))


@pytest.fixture(scope="module")
def iq3s_layer(gpu):
    return {n: Stack("IQ3_S", E, r, c, 100 + i, gpu) for i, (n, (r, c)) in
            enumerate((("gate", (F, H)), ("up", (F, H)), ("down", (H, F))))}


def routing(tokens, seed):
    idx, w = synth.zipf_routing(tokens, E, K, np.random.default_rng(seed))
    return idx


def glu_oracle(layer, x, idx, dtype):
    """g, u (float64) and the rounded SwiGLU h for every pair of idx (tokens, k); x (tokens, H)."""
    flat = idx.reshape(-1)
    xs = np.asarray(x, np.float64)
    g = np.empty((len(flat), F))
    u = np.empty((len(flat), F))
    for e in np.unique(flat):
        at = np.nonzero(flat == e)[0]
        rows = xs[at // idx.shape[1]]
        g[at] = rows @ layer["gate"].weights(e).astype(np.float64).T
        u[at] = rows @ layer["up"].weights(e).astype(np.float64).T
    return g, u


def down_oracle(layer, h, flat):
    y = np.empty((len(flat), H))
    for e in np.unique(flat):
        at = np.nonzero(flat == e)[0]
        y[at] = np.asarray(h[at], np.float64) @ layer["down"].weights(e).astype(np.float64).T
    return y


@pytest.mark.parametrize("tokens", [1, 4])
def test_routed_decode_as_benchmarked(gpu, iq3s_layer, tokens):
    """The decode layer the benchmark times: gate+up+SwiGLU in one launch (the paired kernel, 64-lane rows of
    4096 inputs) and down (rows of 1536 inputs); g, u and y at 1e-3 relative L2, h within one float16 step of the
    SwiGLU of the kernel's own g and u, and BlockSwitchGLU's output equal to those launches'."""
    L = iq3s_layer
    idx = routing(tokens, tokens)
    rng = np.random.default_rng(7 + tokens)
    x = (rng.standard_normal((tokens, H)) / 64).astype(np.float16)
    xs, ix = torch.from_numpy(x).to(gpu), torch.from_numpy(idx).to(gpu)
    flat = idx.reshape(-1)
    g, u, h = B.gate_up_swiglu(L["gate"].lin, L["up"].lin, xs, ix.reshape(-1), K)
    y = B.expert_matvec(L["down"].lin, ix.reshape(-1), h)
    glu = B.BlockSwitchGLU(L["gate"].lin, L["up"].lin, L["down"].lin)(xs, ix)
    torch.cuda.synchronize()
    assert torch.equal(glu.reshape(-1, H), y)  # switch_glu takes these very launches

    g64, u64 = glu_oracle(L, x, idx, np.float16)
    gk, uk, hk = (t.cpu().numpy() for t in (g, u, h))
    assert rel_l2(gk, g64) <= REL and rel_l2(uk, u64) <= REL
    want_h = O.swiglu_rounded(gk, uk, np.float16)
    steps = np.abs(hk.astype(np.float64) - want_h.astype(np.float64)) / np.maximum(
        np.spacing(np.abs(want_h.astype(np.float16))).astype(np.float64), 2.0 ** -24)
    assert steps.max() <= 1.0
    y64 = down_oracle(L, hk, flat)
    assert rel_l2(y.float().cpu().numpy(), y64) <= REL


def test_speculative_verify_in_q2_0(gpu):
    """Config 3: the Q2_0 layer, five rows (1 + 4 draft tokens) through top-8 of 256 Zipf experts. BlockSwitchGLU
    takes gate_up_swiglu / expert_matvec (exact products, float32 sums), held to 1e-3; with LOOKUP_GLU it takes the
    table of sums (the reference's path for Q2_0 over float16), whose sums are rounded to float16 as the reference
    rounds them, within 4e-3."""
    L = {n: Stack("Q2_0", E, r, c, 200 + i, gpu) for i, (n, (r, c)) in
         enumerate((("gate", (F, H)), ("up", (F, H)), ("down", (H, F))))}
    idx = routing(5, 5)
    x = np.random.default_rng(5).standard_normal((5, H)).astype(np.float16)
    xs, ix = torch.from_numpy(x).to(gpu), torch.from_numpy(idx).to(gpu)
    flat = idx.reshape(-1)
    g, u, h = B.gate_up_swiglu(L["gate"].lin, L["up"].lin, xs, ix.reshape(-1), K)
    y = B.expert_matvec(L["down"].lin, ix.reshape(-1), h)
    glu = B.BlockSwitchGLU(L["gate"].lin, L["up"].lin, L["down"].lin)
    assert torch.equal(glu(xs, ix).reshape(-1, H), y)  # switch_glu takes these very launches
    old, B.LOOKUP_GLU = B.LOOKUP_GLU, True
    try:
        table = glu(xs, ix)
    finally:
        B.LOOKUP_GLU = old
    g64, u64 = glu_oracle(L, x, idx, np.float16)
    assert rel_l2(g.float().cpu().numpy(), g64) <= REL and rel_l2(u.float().cpu().numpy(), u64) <= REL
    y64 = down_oracle(L, h.cpu().numpy(), flat)
    assert rel_l2(y.float().cpu().numpy(), y64) <= REL
    # the table path: float16 table sums (blocks.py:718-781); against the chain of exact products
    h64 = O.swiglu_rounded(g64, u64, np.float16)
    assert rel_l2(table.float().cpu().numpy().reshape(-1, H), down_oracle(L, h64, flat)) <= 4e-3


def test_q4_k_matvec_with_float32_activations(gpu):
    """Config 1: one Q4_K matrix of 4096 x 4096, float32 x, batch 1 (the reference converts Q4_K to its affine form,
    gguf.py:207-217, and multiplies in float32): within test_blocks.py:35's bound and 1e-3 relative L2."""
    s = Stack("Q4_K", 1, 4096, 4096, 300, gpu)
    x = np.random.default_rng(1).standard_normal((1, 4096)).astype(np.float32)
    xs = torch.from_numpy(x).to(gpu)
    w = s.weights(0).astype(np.float64)
    want = x.astype(np.float64) @ w.T
    for got in (B.window_matvec(s.blocks, "Q4_K", 4096, 4096, xs), D.BlockLinear(s.blocks, "Q4_K", (4096, 4096))(xs)):
        got = got.cpu().numpy()
        assert got.dtype == np.float32
        assert np.abs(got - want).max() <= 1e-5 * np.abs(w).max() * np.sqrt(4096)
        assert rel_l2(got, want) <= REL


@pytest.mark.parametrize("kind, rows", [("Q6_K", 4096), ("Q8_0", 4096), ("Q4_K", 1536), ("Q6_K", 151936),
                                        ("Q8_0", 20001)])
def test_dense_decode_layers_of_the_mixed_model(gpu, kind, rows):
    """Config 5's decode: q, k, v (Q6_K), o (Q8_0), the shared expert (Q4_K 1536 x 4096) and lm_head (151936 x 4096
    Q6_K) at one float16 token, checked on a sample of rows (lm_head) or all of them; a Q8_0 matrix past 16384 rows
    (an odd row count) takes the direct kernel as lm_head does."""
    s = Stack(kind, 1, rows, 4096, 400 + rows % 97, gpu)
    x = np.random.default_rng(2).standard_normal((1, 4096)).astype(np.float16)
    layer = D.BlockLinear(s.blocks, kind, (rows, 4096))
    got = layer(torch.from_numpy(x).to(gpu)).float().cpu().numpy()[0]
    pick = np.arange(rows) if rows <= 4096 else np.sort(np.random.default_rng(3).choice(rows, 2048, replace=False))
    want = s.weights(0, pick).astype(np.float64) @ x[0].astype(np.float64)
    assert rel_l2(got[pick], want) <= REL


def test_fused_qkv_as_benchmarked(gpu):
    """The decode benchmark's q/k/v: three Q6_K 4096 x 4096 layers fused into one 12288-row matrix (dense.FusedLinear,
    one launch: the one-matrix form at three units a wave), one float16 token, against the oracle on 1024 rows of
    each of q, k and v (the first and last rows included)."""
    parts = [Stack("Q6_K", 1, 4096, 4096, 650 + i, gpu) for i in range(3)]
    fused = D.FusedLinear([D.BlockLinear(p.blocks, "Q6_K", (4096, 4096)) for p in parts])
    x = np.random.default_rng(12).standard_normal((1, 4096)).astype(np.float16)
    xs = torch.from_numpy(x).to(gpu)
    outs = fused(xs)
    whole = B.window_matvec(fused.blocks, "Q6_K", 3 * 4096, 4096, xs)  # the benchmark's call
    torch.cuda.synchronize()
    assert torch.equal(torch.cat(outs, dim=-1), whole)
    pick = np.sort(np.random.default_rng(13).choice(4096, 1024, replace=False))
    pick[0], pick[-1] = 0, 4095
    for part, got in zip(parts, outs):
        want = part.weights(0, pick).astype(np.float64) @ x[0].astype(np.float64)
        assert rel_l2(got.float().cpu().numpy()[0][pick], want) <= REL


def prompt_check(gpu, layer, kind, tokens, dtype, seed, x_scale=1.0):
    """A prompt chunk through switch_glu's tiles, every pair of a sample of experts (the heaviest, a middling one,
    the lightest used, and those of a few random pairs) against the oracle's chain g, u -> SwiGLU rounded to the
    activations' type -> down."""
    idx = routing(tokens, seed)
    rng = np.random.default_rng(seed)
    x32 = (rng.standard_normal((tokens, H)) * x_scale).astype(np.float32)
    xs = torch.from_numpy(x32).to(dtype).to(gpu)
    ix = torch.from_numpy(idx).to(gpu)
    assert idx.size >= B.TILES_FROM
    y = B.BlockSwitchGLU(layer["gate"].lin, layer["up"].lin, layer["down"].lin)(xs, ix)
    torch.cuda.synchronize()
    y = y.float().cpu().numpy().reshape(-1, H)
    flat = idx.reshape(-1)
    counts = np.bincount(flat, minlength=E)
    used = np.nonzero(counts)[0]
    by = used[np.argsort(counts[used], kind="stable")]
    sample = set([by[-1], by[len(by) // 2], by[0]]) | set(flat[rng.choice(len(flat), 3, replace=False)].tolist())
    pairs = np.nonzero(np.isin(flat, list(sample)))[0]
    xr = xs.float().cpu().numpy().astype(np.float64)  # the activations as the kernels get them
    sub = idx.reshape(-1)[pairs]
    g = np.empty((len(pairs), F))
    u = np.empty((len(pairs), F))
    for e in np.unique(sub):
        at = np.nonzero(sub == e)[0]
        rows = xr[pairs[at] // K]
        g[at] = rows @ layer["gate"].weights(e).astype(np.float64).T
        u[at] = rows @ layer["up"].weights(e).astype(np.float64).T
    npdt = np.float16 if dtype == torch.float16 else np.float32
    silu = g / (1.0 + np.exp(-g)) * u
    h = silu.astype(np.float32)
    h = torch.from_numpy(h).to(dtype).float().numpy() if dtype == torch.bfloat16 else h.astype(npdt)
    want = as_dtype(down_oracle(layer, h, sub), dtype)
    assert counts[by[-1]] > 16 * 8  # the heaviest expert fills several chunks of tiles
    assert rel_l2(y[pairs], want) <= REL, sorted(sample)


def test_prompt_chunk_as_benchmarked(gpu):
    """Config 4: 512 tokens, IQ3_XXS, 256 experts top-8 of Zipf routing, bfloat16 activations."""
    layer = {n: Stack("IQ3_XXS", E, r, c, 500 + i, gpu) for i, (n, (r, c)) in
             enumerate((("gate", (F, H)), ("up", (F, H)), ("down", (H, F))))}
    prompt_check(gpu, layer, "IQ3_XXS", 512, torch.bfloat16, 4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prompt_chunk_in_q2_0(gpu, dtype):
    """Config 4's shape in Q2_0 (the prompt-chunk target is stated for IQ3_S and Q2_0 blocks): 512 tokens, 256
    experts top-8 of Zipf routing, gate/up 1536 x 4096 and down 4096 x 1536, through switch_glu's tiles (the fused
    gate/up SwiGLU and scatter-down kernels on Q2_0's rows staged in LDS), bfloat16 and float16."""
    layer = {n: Stack("Q2_0", E, r, c, 520 + i, gpu) for i, (n, (r, c)) in
             enumerate((("gate", (F, H)), ("up", (F, H)), ("down", (H, F))))}
    prompt_check(gpu, layer, "Q2_0", 512, dtype, 14)


@pytest.mark.parametrize("kind", ["IQ3_S", "IQ3_XXS", "Q2_0"])
def test_prompt_rows_of_three_steps(gpu, kind):
    """Rows of 768 inputs (three steps of 256: an odd step count, whose last step starts two bytes into a dword in the
    staged form) through switch_glu's tiles: gate/up 512 x 768, down 768 x 512, 16 experts, 256 tokens top-8,
    float16, against the oracle's chain."""
    experts, rows, cols, tokens, k = 16, 512, 768, 256, 8
    layer = {n: Stack(kind, experts, r, c, 900 + i, gpu) for i, (n, (r, c)) in
             enumerate((("gate", (rows, cols)), ("up", (rows, cols)), ("down", (cols, rows))))}
    rng = np.random.default_rng(15)
    idx = np.stack([rng.choice(experts, k, replace=False) for _ in range(tokens)])
    x = (rng.standard_normal((tokens, cols)) / 16).astype(np.float16)
    xs, ix = torch.from_numpy(x).to(gpu), torch.from_numpy(idx).to(gpu)
    assert idx.size >= B.TILES_FROM
    y = B.BlockSwitchGLU(layer["gate"].lin, layer["up"].lin, layer["down"].lin)(xs, ix)
    y = y.float().cpu().numpy().reshape(-1, cols)
    flat = idx.reshape(-1)
    xr = x.astype(np.float64)
    want = np.empty((len(flat), cols))
    for e in np.unique(flat):
        at = np.nonzero(flat == e)[0]
        g = xr[at // k] @ layer["gate"].weights(e).astype(np.float64).T
        u = xr[at // k] @ layer["up"].weights(e).astype(np.float64).T
        h = (g / (1.0 + np.exp(-g)) * u).astype(np.float32).astype(np.float16)  # float32 SwiGLU rounded once
        want[at] = h.astype(np.float64) @ layer["down"].weights(e).astype(np.float64).T
    assert rel_l2(y, as_dtype(want, torch.float16)) <= REL


def test_prefill_routed_experts(gpu, iq3s_layer):
    """Config 5's prefill: 2048 tokens through the IQ3_S experts' tiles, bfloat16 and float16."""
    prompt_check(gpu, iq3s_layer, "IQ3_S", 2048, torch.bfloat16, 8)
    prompt_check(gpu, iq3s_layer, "IQ3_S", 2048, torch.float16, 9, x_scale=1 / 64)


@pytest.mark.parametrize("kind, rows, cols", [("Q6_K", 4096, 4096), ("Q8_0", 4096, 4096), ("Q4_K", 1536, 4096),
                                              ("Q4_K", 4096, 1536)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_dense_layers(gpu, kind, rows, cols, dtype):
    """Config 5's prefill: 2048 tokens through the dense layers (attention projections, the shared expert), on a
    sample of 256 output rows."""
    s = Stack(kind, 1, rows, cols, 600 + rows % 89 + cols % 7, gpu)
    x = np.random.default_rng(6).standard_normal((2048, cols)).astype(np.float32)
    xs = torch.from_numpy(x).to(dtype).to(gpu)
    got = D.BlockLinear(s.blocks, kind, (rows, cols))(xs).float().cpu().numpy()
    pick = np.sort(np.random.default_rng(7).choice(rows, 256, replace=False))
    want = xs.float().cpu().numpy().astype(np.float64) @ s.weights(0, pick).astype(np.float64).T
    assert rel_l2(got[:, pick], as_dtype(want, dtype)) <= REL


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_dense_layer_in_a_graph(gpu, dtype):
    """The prompt-chunk product (the layer dequantized, then the library product) captured in a HIP graph, as the
    benchmark runs it: every replay, with eager work between them, gives the eager call's bits."""
    s = Stack("Q6_K", 1, 1024, 4096, 611, gpu)
    layer = D.BlockLinear(s.blocks, "Q6_K", (1024, 4096))
    x = torch.from_numpy(np.random.default_rng(8).standard_normal((512, 4096)).astype(np.float32)).to(dtype).to(gpu)
    want = layer(x)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        layer(x)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got = layer(x)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"replay {r}"
        layer(x * 2)  # eager work between the replays
        torch.cuda.synchronize()


def test_matvec_separate_against_the_oracle(gpu):
    """matvec_separate (blocks.py:331-346): every pair brings its expert's blocks as a tensor of its own; 1536 x 4096
    IQ3_S experts, one token shared by eight pairs and a row for each pair, against the oracle."""
    s = Stack("IQ3_S", 8, F, H, 700, gpu)
    mats = [s.blocks[e * F * s.rb:(e + 1) * F * s.rb].clone() for e in range(8)]
    order = [3, 0, 7, 7, 1, 5, 2, 6]
    rng = np.random.default_rng(8)
    x1 = rng.standard_normal((1, H)).astype(np.float16)
    got = B.matvec_separate([mats[e] for e in order], "IQ3_S", F, H, torch.from_numpy(x1).to(gpu), 8)
    want = np.stack([s.weights(e).astype(np.float64) @ x1[0].astype(np.float64) for e in order])
    assert rel_l2(got.float().cpu().numpy(), want) <= REL
    x8 = rng.standard_normal((8, H)).astype(np.float16)
    got = B.matvec_separate([mats[e] for e in order], "IQ3_S", F, H, torch.from_numpy(x8).to(gpu), 1)
    want = np.stack([s.weights(e).astype(np.float64) @ x8[i].astype(np.float64) for i, e in enumerate(order)])
    assert rel_l2(got.float().cpu().numpy(), want) <= REL


def test_bfloat16_prompt_outside_float16s_range(gpu):
    """bfloat16 activations far outside float16's range (rows reaching 1e9 and rows of 1e-12) through the tiles:
    rows scaled into float16 by a power of two each, so every product is the oracle's (blocks.py:684-694)."""
    layer = {n: Stack("IQ3_XXS", 16, r, c, 800 + i, gpu) for i, (n, (r, c)) in
             enumerate((("gate", (256, 512)), ("up", (256, 512)), ("down", (512, 256))))}
    rng = np.random.default_rng(9)
    tokens, k = 256, 8
    idx = np.stack([rng.choice(16, k, replace=False) for _ in range(tokens)])
    x = rng.standard_normal((tokens, 512))
    x[::3] *= 1e9
    x[1::3] *= 1e-12
    x[5, :7] = 0.0
    xs = torch.from_numpy(x.astype(np.float32)).to(torch.bfloat16).to(gpu)
    y = B.BlockSwitchGLU(layer["gate"].lin, layer["up"].lin, layer["down"].lin)(xs, torch.from_numpy(idx).to(gpu))
    y = y.float().cpu().numpy().reshape(-1, 512)
    xr = xs.float().cpu().numpy().astype(np.float64)
    flat = idx.reshape(-1)
    h = np.empty((len(flat), 256))
    for e in np.unique(flat):
        at = np.nonzero(flat == e)[0]
        g = xr[at // k] @ layer["gate"].weights(e).astype(np.float64).T
        u = xr[at // k] @ layer["up"].weights(e).astype(np.float64).T
        h[at] = (g / (1.0 + np.exp(-np.clip(g, -700, 700))) * u)
    h = as_dtype(h, torch.bfloat16)
    want = np.empty((len(flat), 512))
    for e in np.unique(flat):
        at = np.nonzero(flat == e)[0]
        want[at] = h[at] @ layer["down"].weights(e).astype(np.float64).T
    want = as_dtype(want, torch.bfloat16)
    assert np.isfinite(y).all()
    for rows in (slice(0, None, 3), slice(1, None, 3), slice(2, None, 3)):  # each scale of rows on its own
        sel = np.arange(len(flat)).reshape(tokens, k)[rows].reshape(-1)
        assert rel_l2(y[sel], want[sel]) <= REL


@pytest.mark.parametrize("kind", ["IQ3_S", "IQ3_XXS", "Q2_0"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prompt_full_chunks_and_tails(gpu, kind, dtype):
    """A long prompt over few experts, eight tiles an expert or more: each expert's run of tiles split into full
    chunks of 16 (the wide form, an expert's rows decoded once a step for all 16 tiles) and a tail of 0 to 15 tiles
    (the chunked form), through switch_glu's tiles: gate/up 512 x 768 (three steps), down 768 x 512, 16 experts
    picked with weights 1 .. 16 (runs of about 4 to 30 tiles), 1024 tokens top-4, against the oracle's chain."""
    experts, rows, cols, tokens, k = 16, 512, 768, 1024, 4
    layer = {n: Stack(kind, experts, r, c, 940 + i, gpu) for i, (n, (r, c)) in
             enumerate((("gate", (rows, cols)), ("up", (rows, cols)), ("down", (cols, rows))))}
    rng = np.random.default_rng(17)
    weights = np.arange(1, experts + 1, dtype=np.float64)
    idx = np.stack([rng.choice(experts, k, replace=False, p=weights / weights.sum()) for _ in range(tokens)])
    tiles = -(-np.bincount(idx.reshape(-1), minlength=experts) // 16)
    assert tiles.sum() >= 8 * experts and (tiles >= 16).sum() >= 4 and len(set(tiles % 16)) >= 6
    x = (rng.standard_normal((tokens, cols)) / 16).astype(np.float32)
    xs, ix = torch.from_numpy(x).to(dtype).to(gpu), torch.from_numpy(idx.astype(np.int32)).to(gpu)
    y = B.BlockSwitchGLU(layer["gate"].lin, layer["up"].lin, layer["down"].lin)(xs, ix)
    y = y.float().cpu().numpy().reshape(-1, cols)
    flat = idx.reshape(-1)
    xr = xs.float().cpu().numpy().astype(np.float64)
    want = np.empty((len(flat), cols))
    for e in np.unique(flat):
        at = np.nonzero(flat == e)[0]
        g = xr[at // k] @ layer["gate"].weights(e).astype(np.float64).T
        u = xr[at // k] @ layer["up"].weights(e).astype(np.float64).T
        h = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
        h = torch.from_numpy(h).to(dtype).float().numpy().astype(np.float64)  # the SwiGLU rounded to the type
        want[at] = h @ layer["down"].weights(e).astype(np.float64).T
    assert rel_l2(y, as_dtype(want, dtype)) <= REL


@pytest.mark.parametrize("kind", ["IQ3_S", "Q2_0"])
def test_prompt_split_with_an_expert_in_two_runs(gpu, kind):
    """The C ABI's tiles in any order (strata_prompt_gate_up_swiglu, strata_prompt_down: every slot of a tile naming
    an expert, whatever the tiles around it), with the full-chunk split on (eight tiles an expert or more): expert 0
    in two runs (20 tiles, then 17 after another expert's 3), expert 2 in a run of exactly 16, short runs, and
    tiles naming no expert, whose rows of h stay as they were. h and y against the oracle's chain at 1e-3."""
    from strata_mlx_amd import _lib
    experts, rows, cols, n_tok = 4, 512, 768, 64
    runs = [(0, 20), (1, 3), (0, 17), (2, 16), (3, 2), (experts, 2)]
    te = np.concatenate([np.full(n, e, np.uint32) for e, n in runs])
    n_tiles = len(te)
    assert n_tiles >= 8 * experts
    layer = {n: Stack(kind, experts, r, c, 960 + i, gpu) for i, (n, (r, c)) in
             enumerate((("gate", (rows, cols)), ("up", (rows, cols)), ("down", (cols, rows))))}
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((n_tok, cols)) / 16).astype(np.float16)
    slots = n_tiles * 16
    token = rng.integers(0, n_tok, slots).astype(np.uint32)
    e_slot = np.repeat(te, 16)
    filled = e_slot < experts
    pairs = int(filled.sum())
    slot_pair = np.full(slots, 0xFFFFFFFF, np.uint32)
    slot_pair[filled] = rng.permutation(pairs).astype(np.uint32)
    idx = np.empty(pairs, np.uint32)
    idx[slot_pair[filled]] = e_slot[filled]
    d = lambda a: torch.from_numpy(a).to(gpu)
    xs, tok, tes, sp, ix = d(x), d(token.view(np.int32)), d(te.view(np.int32)), d(slot_pair.view(np.int32)), d(
        idx.view(np.int32))
    h = torch.full((slots, rows), 7.0, dtype=torch.float16, device=gpu)
    y = torch.empty((pairs, cols), dtype=torch.float16, device=gpu)
    lib, kid = _lib.library(), _lib.kind_id(kind)
    _lib.check(lib.strata_prompt_gate_up_swiglu(kid, layer["gate"].lin.blocks.data_ptr(), layer["up"].lin.blocks.data_ptr(),
                                                experts, rows, cols, xs.data_ptr(), None, tok.data_ptr(), tes.data_ptr(),
                                                n_tiles, 16, h.data_ptr(), _lib.dtype_id(torch.float16), _lib.stream()),
               "gate/up")
    _lib.check(lib.strata_prompt_down(kid, layer["down"].lin.blocks.data_ptr(), experts, cols, rows, h.data_ptr(), None,
                                      tes.data_ptr(), n_tiles, 16, sp.data_ptr(), ix.data_ptr(), pairs, y.data_ptr(),
                                      _lib.dtype_id(torch.float16), _lib.stream()), "down")
    torch.cuda.synchronize()
    hg, yg = h.float().cpu().numpy(), y.float().cpu().numpy()
    assert (hg[~filled] == 7.0).all()
    xr = x.astype(np.float64)
    h_want = np.zeros((slots, rows))
    y_want = np.zeros((pairs, cols))
    for e in range(experts):
        at = np.nonzero(e_slot == e)[0]
        g = xr[token[at]] @ layer["gate"].weights(e).astype(np.float64).T
        u = xr[token[at]] @ layer["up"].weights(e).astype(np.float64).T
        he = (g / (1.0 + np.exp(-g)) * u).astype(np.float32).astype(np.float16)
        h_want[at] = he
        y_want[slot_pair[at]] = he.astype(np.float64) @ layer["down"].weights(e).astype(np.float64).T
    assert rel_l2(hg[filled], h_want[filled]) <= REL
    assert rel_l2(yg, as_dtype(y_want, torch.float16)) <= REL
