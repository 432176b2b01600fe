"""The persistent decode kernels (routed_glu_kernel: gate/up/SwiGLU on rows of 4096 inputs; routed_down_kernel: a
routed matrix on rows of 1536 or 2560 inputs), IQ3_S and Q2_0, at the unit counts that pick each of their forms
(one to sixteen units a wave, more units than one round of resident waves holds) and at one to eight tokens.
Against the oracle: g and u at 1e-3 relative L2 against float64 products of the oracle's weights, h within one
float16 step of the SwiGLU of the kernel's own g and u (strata_mlx/blocks.py:222-236), NaN rows for a pair naming
no expert, and a pair repeating an expert equal to the first pair naming it."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B
from strata_mlx_amd import synth

pytestmark = pytest.mark.gpu

H, REL = 4096, 1e-3


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return np.linalg.norm(got - want) / np.linalg.norm(want)


@pytest.fixture(scope="module")
def stacks(gpu):
    experts, rows = 12, 1536
    g = torch.Generator(device=gpu).manual_seed(31)
    out = {}
    for name in ("gate", "up"):
        blocks = synth.random_stack("IQ3_S", experts * rows * H, gpu, g)
        out[name] = (blocks, B.row_bytes("IQ3_S", H))
    return out, experts, rows


# (pairs, rows): units = pairs * rows; 4096 waves are resident at once on 256 CUs
@pytest.mark.parametrize("pairs,rows", [(1, 64), (3, 1536), (8, 1536), (10, 1536), (24, 1536), (5, 200), (64, 1536)])
def test_one_token_gate_up(gpu, stacks, pairs, rows):
    (gate_b, rb), (up_b, _) = stacks[0]["gate"], stacks[0]["up"]
    experts, all_rows = stacks[1], stacks[2]
    # the first `rows` rows of each expert: a stack of `experts` matrices of `rows` rows
    gate_s = gate_b.reshape(experts, all_rows, rb)[:, :rows].contiguous()
    up_s = up_b.reshape(experts, all_rows, rb)[:, :rows].contiguous()
    gate = B.BlockSwitchLinear(gate_s, "IQ3_S", (experts, rows, H))
    up = B.BlockSwitchLinear(up_s, "IQ3_S", (experts, rows, H))
    rng = np.random.default_rng(pairs * 1000 + rows)
    idx = rng.integers(0, experts, pairs).astype(np.int32)
    if pairs >= 3:
        idx[1] = experts + 5  # names no expert
        idx[2] = idx[0]       # repeats the first pair's expert
    x = (rng.standard_normal((1, H)) / 64).astype(np.float16)
    xs, ix = torch.from_numpy(x).to(gpu), torch.from_numpy(idx).to(gpu)
    g, u, h = B.gate_up_swiglu(gate, up, xs, ix, pairs)
    torch.cuda.synchronize()
    gk, uk, hk = (t.cpu().numpy() for t in (g, u, h))
    ok = idx < experts
    assert np.isnan(gk[~ok]).all() and np.isnan(uk[~ok]).all() and np.isnan(hk[~ok]).all()
    if pairs >= 3:
        assert np.array_equal(hk[2], hk[0]) and np.array_equal(gk[2], gk[0])
    gw = gate_s.cpu().numpy().reshape(experts, -1)
    uw = up_s.cpu().numpy().reshape(experts, -1)
    xd = x.astype(np.float64)[0]
    for p in np.nonzero(ok)[0]:
        e = idx[p]
        wg = O.dequantize(gw[e], "IQ3_S", (rows, H)).astype(np.float64)
        wu = O.dequantize(uw[e], "IQ3_S", (rows, H)).astype(np.float64)
        assert rel_l2(gk[p], wg @ xd) <= REL and rel_l2(uk[p], wu @ xd) <= REL
    want_h = O.swiglu_rounded(gk[ok], uk[ok], np.float16)
    steps = np.abs(hk[ok].astype(np.float64) - want_h.astype(np.float64)) / np.maximum(
        np.spacing(np.abs(want_h.astype(np.float16))).astype(np.float64), 2.0 ** -24)
    # the sigmoid's exp is float32 expf on the GPU and float64 in the oracle: where the float16 sigmoid lands on
    # the other side of a rounding boundary, g * sig and its product with u each move by up to one more step
    assert steps.max() <= 2.0 and np.mean(steps > 1.0) <= 1e-3


# (pairs, share, rows, cols): the routed one-matrix kernel (routed_down_kernel) at both row widths it takes, one and
# two units a wave (more units than 4096 waves), several rounds of workgroups (40 pairs of 4096 rows: five; 300 pairs
# of 128 rows), a pair's last workgroup partly idle (1000, 3000 and 100 rows), rows not a multiple of eight, tokens
# shared by several pairs
@pytest.mark.parametrize("pairs,share,rows,cols", [(8, 1, 4096, 1536), (12, 1, 4096, 1536), (6, 3, 1000, 1536),
                                                    (4, 1, 2048, 2560), (9, 9, 3000, 2560), (40, 1, 4096, 1536),
                                                    (32, 4, 4096, 1536), (64, 8, 2048, 2560), (300, 3, 128, 1536),
                                                    (20, 1, 100, 1536)])
@pytest.mark.parametrize("kind", ["IQ3_S", "Q2_0"])
def test_routed_down(gpu, kind, pairs, share, rows, cols):
    experts = 6
    g = torch.Generator(device=gpu).manual_seed(rows + cols)
    blocks = synth.random_stack(kind, experts * rows * cols, gpu, g)
    lin = B.BlockSwitchLinear(blocks, kind, (experts, rows, cols))
    rng = np.random.default_rng(pairs * 7 + rows)
    idx = rng.integers(0, experts, pairs).astype(np.int32)
    idx[1] = experts  # names no expert
    x = (rng.standard_normal((pairs // share, cols)) / 8).astype(np.float16)
    y = B.expert_matvec(lin, torch.from_numpy(idx).to(gpu), torch.from_numpy(x).to(gpu), share)
    torch.cuda.synchronize()
    yk = y.float().cpu().numpy()
    assert np.isnan(yk[1]).all()
    raw = blocks.cpu().numpy().reshape(experts, -1)
    ws = {}
    for p in range(pairs):
        if p == 1:
            continue
        if idx[p] not in ws:
            ws[idx[p]] = O.dequantize(raw[idx[p]], kind, (rows, cols)).astype(np.float64)
        assert rel_l2(yk[p], ws[idx[p]] @ x[p // share].astype(np.float64)) <= REL


# (kind, tokens, k, rows): gate/up/SwiGLU at several tokens (the tokens in LDS, units row by row over the pairs)
# and Q2_0 at one token; experts repeat across tokens as routing makes them repeat
# (80 pairs: more than a wave has lanes)
@pytest.mark.parametrize("kind,tokens,k,rows", [("IQ3_S", 4, 8, 1536), ("IQ3_S", 2, 8, 640), ("IQ3_S", 8, 8, 512),
                                                ("Q2_0", 5, 8, 1536), ("Q2_0", 1, 8, 1536), ("Q2_0", 3, 4, 900),
                                                ("IQ3_S", 8, 10, 256), ("Q2_0", 8, 10, 200)])
def test_gate_up_tokens(gpu, kind, tokens, k, rows):
    experts = 10
    g = torch.Generator(device=gpu).manual_seed(tokens * 100 + rows)
    gate_b = synth.random_stack(kind, experts * rows * H, gpu, g)
    up_b = synth.random_stack(kind, experts * rows * H, gpu, g)
    gate = B.BlockSwitchLinear(gate_b, kind, (experts, rows, H))
    up = B.BlockSwitchLinear(up_b, kind, (experts, rows, H))
    rng = np.random.default_rng(tokens * 7 + rows)
    idx = np.stack([rng.choice(experts, k, replace=False) for _ in range(tokens)]).astype(np.int32)
    idx[0, 1] = experts + 3  # names no expert
    idx[-1, -1] = idx[-1, 0]  # the last token names an expert twice
    x = (rng.standard_normal((tokens, H)) / 64).astype(np.float16)
    gk, uk, hk = (t.cpu().numpy() for t in B.gate_up_swiglu(gate, up, torch.from_numpy(x).to(gpu),
                                                             torch.from_numpy(idx.reshape(-1)).to(gpu), k))
    flat = idx.reshape(-1)
    ok = flat < experts
    assert np.isnan(hk[~ok]).all() and np.isnan(gk[~ok]).all()
    gw = gate_b.cpu().numpy().reshape(experts, -1)
    uw = up_b.cpu().numpy().reshape(experts, -1)
    for e in np.unique(flat[ok]):
        at = np.nonzero(flat == e)[0]
        xs = x[at // k].astype(np.float64)
        wg = O.dequantize(gw[e], kind, (rows, H)).astype(np.float64)
        wu = O.dequantize(uw[e], kind, (rows, H)).astype(np.float64)
        assert rel_l2(gk[at], xs @ wg.T) <= REL and rel_l2(uk[at], xs @ wu.T) <= REL
    want_h = O.swiglu_rounded(gk[ok], uk[ok], np.float16)
    steps = np.abs(hk[ok].astype(np.float64) - want_h.astype(np.float64)) / np.maximum(
        np.spacing(np.abs(want_h.astype(np.float16))).astype(np.float64), 2.0 ** -24)
    # the sigmoid's exp is float32 expf on the GPU and float64 in the oracle: where the float16 sigmoid lands on
    # the other side of a rounding boundary, g * sig and its product with u each move by up to one more step
    assert steps.max() <= 2.0 and np.mean(steps > 1.0) <= 1e-3


# one token through the dense launches: the linear types at an odd row count and at 4096 rows, and q, k and v
# fused into one launch (FusedLinear), whose outputs are the separate layers' bits
@pytest.mark.parametrize("kind", ["Q4_K", "Q6_K", "Q8_0"])
@pytest.mark.parametrize("rows", [1537, 4096])
def test_dense_one_token(gpu, kind, rows):
    from strata_mlx_amd import dense as D
    g = torch.Generator(device=gpu).manual_seed(rows)
    blocks = synth.random_stack(kind, rows * H, gpu, g)
    x = (np.random.default_rng(rows).standard_normal((1, H)) / 8).astype(np.float16)
    y = B.window_matvec(blocks, kind, rows, H, torch.from_numpy(x).to(gpu)).float().cpu().numpy()
    w = O.dequantize(blocks.cpu().numpy(), kind, (rows, H)).astype(np.float64)
    assert rel_l2(y[0], w @ x[0].astype(np.float64)) <= REL
    lin = D.BlockLinear(blocks, kind, (rows, H))
    assert torch.equal(lin(torch.from_numpy(x).to(gpu)).float().cpu(), torch.from_numpy(y))


@pytest.mark.parametrize("kind", ["Q6_K", "Q4_K"])
def test_fused_layers(gpu, kind):
    from strata_mlx_amd import dense as D
    g = torch.Generator(device=gpu).manual_seed(9)
    sizes = (4096, 1024, 1024) if kind == "Q6_K" else (1536, 1536)
    layers = [D.BlockLinear(synth.random_stack(kind, r * H, gpu, g), kind, (r, H)) for r in sizes]
    x = (torch.randn((1, H), generator=g, device=gpu) / 8).half()
    fused = D.FusedLinear(layers)(x)
    for f, lay in zip(fused, layers):
        assert torch.equal(f, lay(x))
    if kind == "Q4_K":  # the shared expert's gate and up with the SwiGLU in one launch
        gk, uk, hk = (t.float().cpu().numpy() for t in D.gate_up_swiglu(layers[0], layers[1], x))
        xd = x.float().cpu().numpy().astype(np.float64)[0]
        for got, lay in ((gk, layers[0]), (uk, layers[1])):
            w = O.dequantize(lay.blocks.cpu().numpy(), kind, (lay.output_dims, H)).astype(np.float64)
            assert rel_l2(got[0], w @ xd) <= REL
        assert torch.equal(torch.from_numpy(gk).half(), fused[0].cpu()) and torch.equal(torch.from_numpy(uk).half(),
                                                                                       fused[1].cpu())
        want = O.swiglu_rounded(gk, uk, np.float16).astype(np.float64)
        steps = np.abs(hk - want) / np.maximum(np.spacing(np.abs(want.astype(np.float16))).astype(np.float64),
                                               2.0 ** -24)
        assert steps.max() <= 2.0


def test_q4_k_lm_head_one_matrix_form(gpu):
    """Q4_K rows of 4096 inputs from 32768 rows take the one-matrix form (rows 2i and 2i + 1 a unit): 40000 rows (an
    odd unit count) against the oracle on a sample of rows."""
    rows, kind = 40001, "Q4_K"
    g = torch.Generator(device=gpu).manual_seed(3)
    blocks = synth.random_stack(kind, rows * H, gpu, g)
    x = (np.random.default_rng(3).standard_normal((1, H)) / 8).astype(np.float16)
    y = B.window_matvec(blocks, kind, rows, H, torch.from_numpy(x).to(gpu)).float().cpu().numpy()[0]
    rb = B.row_bytes(kind, H)
    at = np.sort(np.random.default_rng(4).choice(rows, 600, replace=False))
    at[-1] = rows - 1
    raw = blocks.reshape(rows, rb)[torch.from_numpy(at).to(gpu)].cpu().numpy()
    w = O.dequantize(raw.reshape(-1), kind, (len(at), H)).astype(np.float64)
    assert rel_l2(y[at], w @ x[0].astype(np.float64)) <= REL


@pytest.mark.parametrize("scale", [1e-30, 1.0, 1e6, 1e30])
def test_q4_k_float32_token_any_range(gpu, scale):
    """A float32 token against Q4_K rows of 4096 inputs takes the persistent form, which scales the token by a power
    of two into float16 and splits it into two float16 parts: exact products to about 2^-22 of the largest input,
    whatever the token's range (beyond float16's, and below its normal numbers)."""
    rows, kind = 1000, "Q4_K"
    g = torch.Generator(device=gpu).manual_seed(5)
    blocks = synth.random_stack(kind, rows * H, gpu, g)
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((1, H)) * scale).astype(np.float32)
    x[0, :64] *= 1e-4  # a stretch of much smaller values
    y = B.window_matvec(blocks, kind, rows, H, torch.from_numpy(x).to(gpu)).cpu().numpy()[0]
    assert y.dtype == np.float32
    w = O.dequantize(blocks.cpu().numpy(), kind, (rows, H)).astype(np.float64)
    want = w @ x[0].astype(np.float64)
    assert rel_l2(y, want) <= 1e-5
    assert np.abs(y - want).max() <= 1e-5 * np.abs(w).max() * np.abs(x).max() * np.sqrt(H)


# the shared expert's gate and up (Q4_K) in the routed gate/up launch at one token: the routed outputs are the
# plain launch's bits, the shared h the SwiGLU of the oracle's float64 products (strata_mlx/fused.py:492-493);
# cases the launch does not take (several tokens, more shared rows than the launch has waves) return None
@pytest.mark.parametrize("kind,pairs,rows,s_rows", [("IQ3_S", 8, 1536, 1536), ("Q2_0", 8, 1536, 1000),
                                                    ("IQ3_S", 3, 200, 517), ("IQ3_S", 1, 64, 200)])
def test_gate_up_with_shared_expert(gpu, kind, pairs, rows, s_rows):
    from strata_mlx_amd import dense as D
    experts = 10
    g = torch.Generator(device=gpu).manual_seed(pairs * 10 + s_rows)
    gate = B.BlockSwitchLinear(synth.random_stack(kind, experts * rows * H, gpu, g), kind, (experts, rows, H))
    up = B.BlockSwitchLinear(synth.random_stack(kind, experts * rows * H, gpu, g), kind, (experts, rows, H))
    sg, su = (D.BlockLinear(synth.random_stack("Q4_K", s_rows * H, gpu, g), "Q4_K", (s_rows, H)) for _ in range(2))
    rng = np.random.default_rng(rows + s_rows)
    idx = rng.choice(experts, pairs, replace=False).astype(np.int32)
    if pairs >= 3:
        idx[1] = experts + 2  # names no expert
    x = (rng.standard_normal((1, H)) / 64).astype(np.float16)
    xs, ix = torch.from_numpy(x).to(gpu), torch.from_numpy(idx).to(gpu)
    got = B.gate_up_swiglu_shared(gate, up, xs, ix, sg, su, with_shared_gu=True)
    x2 = torch.from_numpy(np.repeat(x, 2, axis=0)).to(gpu)
    assert B.gate_up_swiglu_shared(gate, up, x2, torch.cat([ix, ix]), sg, su) is None  # two tokens
    if s_rows > pairs * rows:  # fewer waves than shared rows
        assert got is None
        return
    gs, us, hs, sh, sgk, suk = got
    torch.cuda.synchronize()
    for a, b in zip((gs, us, hs), B.gate_up_swiglu(gate, up, xs, ix, pairs)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    xd = x.astype(np.float64)[0]
    gd, ud = (O.dequantize(lay.blocks.cpu().numpy(), "Q4_K", (s_rows, H)).astype(np.float64) @ xd for lay in (sg, su))
    # the shared expert's own g and u from that launch at 1e-3 of the float64 products; h within two float16 steps
    # of the SwiGLU of the launch's own g and u (strata_mlx/blocks.py:222-236), and at 2e-3 of the float64 chain
    gk, uk = sgk.float().cpu().numpy()[0], suk.float().cpu().numpy()[0]
    assert rel_l2(gk, gd) <= REL and rel_l2(uk, ud) <= REL
    own = O.swiglu_rounded(sgk.cpu().numpy()[0], suk.cpu().numpy()[0], np.float16).astype(np.float64)
    steps = np.abs(sh.cpu().numpy()[0].astype(np.float64) - own) / np.maximum(
        np.spacing(np.abs(own.astype(np.float16))).astype(np.float64), 2.0 ** -24)
    assert steps.max() <= 2.0
    want = O.swiglu_rounded(gd, ud, np.float16)
    assert rel_l2(sh.float().cpu().numpy()[0], want) <= 2e-3
    _, _, hd = D.gate_up_swiglu(sg, su, xs)
    assert rel_l2(sh.float().cpu().numpy()[0], hd.float().cpu().numpy()[0]) <= 2e-3


# the shared expert's down (Q4_K rows of 1536 inputs) in the routed down launch at one token: the routed outputs
# are the plain launch's bits (NaN for the pair naming no expert), the shared rows at 1e-3 of the oracle's float64
# product (strata_mlx/fused.py:492-493); cases the launch does not take (inputs of 2560, more shared rows than two
# units a workgroup cover) return None
@pytest.mark.parametrize("kind,pairs,rows,cols,s_rows", [("IQ3_S", 8, 4096, 1536, 4096), ("Q2_0", 8, 4096, 1536, 4096),
                                                         ("IQ3_S", 3, 200, 1536, 90), ("Q2_0", 1, 4096, 1536, 500),
                                                         ("IQ3_S", 3, 200, 1536, 100), ("IQ3_S", 4, 512, 2560, 64)])
def test_down_with_shared_expert(gpu, kind, pairs, rows, cols, s_rows):
    from strata_mlx_amd import dense as D
    experts = 10
    g = torch.Generator(device=gpu).manual_seed(pairs * 10 + s_rows)
    lin = B.BlockSwitchLinear(synth.random_stack(kind, experts * rows * cols, gpu, g), kind, (experts, rows, cols))
    sd = D.BlockLinear(synth.random_stack("Q4_K", s_rows * cols, gpu, g), "Q4_K", (s_rows, cols))
    rng = np.random.default_rng(rows + s_rows)
    idx = rng.choice(experts, pairs, replace=False).astype(np.int32)
    if pairs >= 3:
        idx[1] = experts + 2  # names no expert
    x = (rng.standard_normal((pairs, cols)) / 8).astype(np.float16)
    sx = (rng.standard_normal((1, cols)) / 8).astype(np.float16)
    xs, ix, sxs = torch.from_numpy(x).to(gpu), torch.from_numpy(idx).to(gpu), torch.from_numpy(sx).to(gpu)
    got = B.expert_matvec_shared(lin, ix, sd)(xs, sxs)
    groups = pairs * -(-rows // 128)  # sixteen units of eight rows a workgroup
    if cols != 1536 or -(-s_rows // 8) > 2 * groups:
        assert got is None
        return
    y, sy = got
    torch.cuda.synchronize()
    plain = B.expert_matvec(lin, ix, xs)
    assert torch.equal(y.view(torch.int16), plain.view(torch.int16))
    if pairs >= 3:
        assert torch.isnan(y[1]).all()
    want = O.dequantize(sd.blocks.cpu().numpy(), "Q4_K", (s_rows, cols)).astype(np.float64) @ sx[0].astype(np.float64)
    assert rel_l2(sy.float().cpu().numpy()[0], want) <= REL
    # calls with another shared token, then the first again: nothing carried from one call to the next
    call = B.expert_matvec_shared(lin, ix, sd)
    y2, sy2 = call(xs, -sxs)
    y3, sy3 = call(xs, sxs)
    torch.cuda.synchronize()
    assert torch.equal(y2.view(torch.int16), plain.view(torch.int16))
    assert rel_l2(sy2.float().cpu().numpy()[0], -want) <= REL
    assert torch.equal(y3.view(torch.int16), plain.view(torch.int16))
    assert torch.equal(sy3.view(torch.int16), sy.view(torch.int16))
