"""The routed experts of one decode token in one launch (strata_expert_layer: gate, up, the SwiGLU and down, the
pair's workgroups handing h over through tagged words in memory). Its outputs are held to the bits of the two
launches it replaces (gate_up_swiglu, then expert_matvec on down), which the oracle pins in test_gpu_routed.py and
test_gpu_configs.py: at every pair count the launch takes (1 to 16: one to six gate/up units a wave), both row
widths of down (1536 and 2560 inputs), IQ3_S and Q2_0, a pair naming no expert (NaN rows) and repeated experts; in
a graph replayed several times with eager work between the replays (the launch tags change on every replay with
the same arguments); and no wait ever gives up (the workspace's status word stays 0). The per-pair path of
strata_mlx/blocks.py:958-986 at one token."""

import numpy as np
import pytest
import torch

from oracle import blocks as O
from strata_mlx_amd import blocks as B
from strata_mlx_amd import synth

pytestmark = pytest.mark.gpu

H = 4096


def layer(kind, experts, ffn, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    mats = [synth.random_stack(kind, experts * r * c, device, g) for r, c in ((ffn, H), (ffn, H), (H, ffn))]
    return (B.BlockSwitchLinear(mats[0], kind, (experts, ffn, H)), B.BlockSwitchLinear(mats[1], kind, (experts, ffn, H)),
            B.BlockSwitchLinear(mats[2], kind, (experts, H, ffn)))


@pytest.fixture(scope="module")
def layers(gpu):
    return {("IQ3_S", 1536): layer("IQ3_S", 24, 1536, 1, gpu), ("Q2_0", 1536): layer("Q2_0", 24, 1536, 2, gpu),
            ("IQ3_S", 2560): layer("IQ3_S", 6, 2560, 3, gpu), ("Q2_0", 2560): layer("Q2_0", 6, 2560, 4, gpu)}


def two_launches(gate, up, down, x, idx):
    _, _, h = B.gate_up_swiglu(gate, up, x, idx, idx.numel())
    return B.expert_matvec(down, idx, h), h


def token(seed, scale, device):
    rng = np.random.default_rng(seed)
    return torch.from_numpy((rng.standard_normal((1, H)) * scale).astype(np.float16)).to(device)


@pytest.mark.parametrize("kind,ffn", [("IQ3_S", 1536), ("Q2_0", 1536), ("IQ3_S", 2560), ("Q2_0", 2560)])
@pytest.mark.parametrize("pairs", [1, 2, 3, 5, 8, 12, 16])
def test_layer_is_the_two_launches(gpu, layers, kind, ffn, pairs):
    gate, up, down = layers[(kind, ffn)]
    experts = gate.num_experts
    rng = np.random.default_rng(pairs * 31 + ffn)
    idx = rng.integers(0, experts, pairs).astype(np.int32)
    if pairs >= 3:
        idx[1] = experts + 3  # names no expert
        idx[2] = idx[0]       # repeats the first pair's expert
    ix = torch.from_numpy(idx).to(gpu)
    x = token(pairs, 1 / 64, gpu)
    got = B.expert_layer(gate, up, down, x, ix, with_h=True)
    if ffn == 2560 and pairs > 8:  # more than one down unit a wave on rows of 2560 inputs: not taken
        assert got is None
        return
    y, h = got
    want_y, want_h = two_launches(gate, up, down, x, ix)
    torch.cuda.synchronize()
    assert B.layer_status(gpu) == 0
    ok = torch.from_numpy(idx < experts).to(gpu)
    assert torch.isnan(y[~ok]).all() and torch.isnan(h[~ok]).all()
    assert torch.equal(y[ok], want_y[ok]) and torch.equal(h[ok], want_h[ok])
    if pairs >= 3:
        assert torch.equal(y[2], y[0])


def test_layer_against_the_oracle(gpu, layers):
    """h at 1e-3 relative L2 against the oracle's SwiGLU of float64 products of its weights, and y against float64
    products of down's weights and the launch's own h."""
    gate, up, down = layers[("IQ3_S", 1536)]
    idx = np.array([3, 17, 5, 22, 0, 9, 11, 4], np.int32)
    x = token(11, 1 / 64, gpu)
    y, h = B.expert_layer(gate, up, down, x, torch.from_numpy(idx).to(gpu), with_h=True)
    torch.cuda.synchronize()
    xd = x.double().cpu().numpy()[0]
    yk, hk = y.double().cpu().numpy(), h.cpu().numpy()
    for lin in (gate, up, down):
        lin.host = lin.blocks.cpu().numpy().reshape(lin.num_experts, -1)
    for p, e in enumerate(idx):
        wg = O.dequantize(gate.host[e], "IQ3_S", (1536, H)).astype(np.float64)
        wu = O.dequantize(up.host[e], "IQ3_S", (1536, H)).astype(np.float64)
        wd = O.dequantize(down.host[e], "IQ3_S", (H, 1536)).astype(np.float64)
        g, u = wg @ xd, wu @ xd
        want_h = O.swiglu_rounded(g.astype(np.float16), u.astype(np.float16), np.float16).astype(np.float64)
        assert np.linalg.norm(hk[p] - want_h) / np.linalg.norm(want_h) <= 1e-3
        want_y = wd @ hk[p].astype(np.float64)
        assert np.linalg.norm(yk[p] - want_y) / np.linalg.norm(want_y) <= 1e-3


def test_layer_in_a_graph(gpu, layers):
    """Eight layer calls captured once (two stacks, fresh routing each) and replayed three times, with eager calls of
    the same launch on the same stream between the replays: every replay gives the eager bits."""
    stream = torch.cuda.Stream()
    cases = []
    for n, key in enumerate([("IQ3_S", 1536), ("Q2_0", 1536)] * 4):
        gate, up, down = layers[key]
        rng = np.random.default_rng(100 + n)
        idx = torch.from_numpy(rng.choice(gate.num_experts, 8, replace=False).astype(np.int32)).to(gpu)
        cases.append((gate, up, down, token(200 + n, 1 / 64, gpu), idx))
    with torch.cuda.stream(stream):
        eager = [B.expert_layer(*c) for c in cases]
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            outs = [B.expert_layer(*c) for c in cases]
        for rep in range(3):
            graph.replay()
            again = [B.expert_layer(*c) for c in cases[::-1]]
            torch.cuda.synchronize()
            for o, e in zip(outs, eager):
                assert torch.equal(o, e), f"replay {rep}"
            for a, e in zip(again, eager[::-1]):
                assert torch.equal(a, e)
    torch.cuda.synchronize()
    assert B.layer_status(gpu) == 0


def test_switch_glu_and_the_layer_agree(gpu, layers):
    """BlockSwitchGLU at one token (gate/up/SwiGLU, then down: two launches) and the one launch give the same bits."""
    gate, up, down = layers[("IQ3_S", 1536)]
    idx = torch.tensor([[1, 4, 9, 16, 23, 2, 7, 12]], device=gpu)
    x = token(5, 1 / 64, gpu)
    out = B.BlockSwitchGLU(gate, up, down)(x, idx)
    want = B.expert_layer(gate, up, down, x, idx.reshape(-1))
    torch.cuda.synchronize()
    assert out.shape == (1, 8, H) and torch.equal(out.reshape(8, H), want)


def test_layer_declines_what_it_does_not_take(gpu, layers):
    gate, up, down = layers[("IQ3_S", 1536)]
    x = token(1, 1 / 64, gpu)
    idx = torch.arange(8, device=gpu, dtype=torch.int32)
    assert B.expert_layer(gate, up, down, x.float(), idx) is None  # float32 token
    assert B.expert_layer(gate, up, down, torch.cat([x, x]), idx) is None  # two tokens
    assert B.expert_layer(gate, up, down, x, torch.arange(17, device=gpu) % 24) is None  # 17 pairs
