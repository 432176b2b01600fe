"""strata_route_tiles_noalloc, the routing entry point that allocates nothing (its workspace is the library's own
device array), gives strata_route_tiles' outputs bit for bit, through the C ABI, on two calls in a row, the second
one smaller (the array keeps the first call's contents)."""

import numpy as np
import pytest
import torch

from strata_mlx_amd import _lib, synth

pytestmark = pytest.mark.gpu

TILE = 16


def outputs(lib, pairs, experts, dev):
    n_tiles = lib.strata_route_tiles_max(pairs, experts, TILE)
    junk = lambda n: torch.full((max(1, n),), 0x5A5A5A5A, dtype=torch.int32, device=dev)  # every word must be written
    return n_tiles, junk(n_tiles), junk(n_tiles * TILE), junk(pairs), junk(n_tiles * TILE)


def route(lib, idx, k, experts, noalloc):
    dev = idx.device
    pairs = idx.numel()
    n_tiles, tile_expert, token, where, slot_pair = outputs(lib, pairs, experts, dev)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.strata_route_tiles_noalloc(idx.data_ptr(), pairs, k, experts, TILE, tile_expert.data_ptr(),
                                            token.data_ptr(), where.data_ptr(), slot_pair.data_ptr(), stream)
    else:
        ws = torch.empty(max(1, lib.strata_route_tiles_workspace(pairs, experts)), dtype=torch.uint8, device=dev)
        rc = lib.strata_route_tiles(idx.data_ptr(), pairs, k, experts, TILE, tile_expert.data_ptr(), token.data_ptr(),
                                    where.data_ptr(), slot_pair.data_ptr(), ws.data_ptr(), stream)
    assert rc == _lib.OK
    torch.cuda.synchronize()
    return [t[:n].cpu().numpy() for t, n in ((tile_expert, n_tiles), (token, n_tiles * TILE), (where, pairs),
                                             (slot_pair, n_tiles * TILE))]


def test_the_routing_that_allocates_nothing_gives_the_same_tiles(gpu):
    lib = _lib.library()
    rng = np.random.default_rng(12)
    cases = [(4096, 8, 256, synth.zipf_routing(512, 256, 8, rng)[0]),  # a 512-token prompt chunk
             (65536, 8, 1024, rng.integers(0, 1024, (8192, 8))),        # the largest the array takes
             (330, 2, 40, rng.integers(0, 44, (165, 2)))]               # smaller, some pairs naming no expert
    for pairs, k, experts, idx in cases:
        ix = torch.from_numpy(np.ascontiguousarray(idx).reshape(-1).astype(np.int32)).to(gpu)
        want = route(lib, ix, k, experts, noalloc=False)
        got = route(lib, ix, k, experts, noalloc=True)
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b)
    # past the array's size: refused before anything runs
    ix = torch.zeros(65537, dtype=torch.int32, device=gpu)
    n_tiles, te, tok, wh, sp = outputs(lib, 65537, 8, gpu)
    assert lib.strata_route_tiles_noalloc(ix.data_ptr(), 65537, 1, 8, TILE, te.data_ptr(), tok.data_ptr(),
                                          wh.data_ptr(), sp.data_ptr(), 0) == _lib.ERR_SHAPE


def test_the_routing_that_allocates_nothing_replays_in_a_graph(gpu):
    """Captured in a HIP graph (torch's global capture mode) and replayed three times, with eager calls between the
    replays, the call that allocates nothing gives the allocating call's tiles on every replay."""
    lib = _lib.library()
    rng = np.random.default_rng(13)
    idx = torch.from_numpy(synth.zipf_routing(512, 256, 8, rng)[0].reshape(-1).astype(np.int32)).to(gpu)
    pairs, experts, k = idx.numel(), 256, 8
    want = route(lib, idx, k, experts, noalloc=False)
    n_tiles, te, tok, wh, sp = outputs(lib, pairs, experts, gpu)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            rc = lib.strata_route_tiles_noalloc(idx.data_ptr(), pairs, k, experts, TILE, te.data_ptr(), tok.data_ptr(),
                                                wh.data_ptr(), sp.data_ptr(), stream.cuda_stream)
    assert rc == _lib.OK
    other = torch.from_numpy(rng.integers(0, 40, 330).astype(np.int32)).to(gpu)
    for rep in range(3):
        for t in (te, tok, wh, sp):
            t.fill_(0x5A5A5A5A)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [t[:n].cpu().numpy() for t, n in ((te, n_tiles), (tok, n_tiles * TILE), (wh, pairs), (sp, n_tiles * TILE))]
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b, err_msg=f"replay {rep}")
        route(lib, other, 2, 40, noalloc=True)  # eager work on the same array between the replays


FIRST_CALL_IN_A_CAPTURE = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from strata_mlx_amd import _lib
lib = _lib.library()
dev = torch.device("cuda:0")
rng = np.random.default_rng(3)
idx = torch.from_numpy(rng.integers(0, 64, 2048).astype(np.int32)).to(dev)
pairs, experts, k, tile = 2048, 64, 8, 16
n_tiles = lib.strata_route_tiles_max(pairs, experts, tile)
outs = [torch.zeros(max(1, n), dtype=torch.int32, device=dev) for n in (n_tiles, n_tiles * tile, pairs, n_tiles * tile)]
ref = [torch.zeros_like(t) for t in outs]
ws = torch.empty(lib.strata_route_tiles_workspace(pairs, experts), dtype=torch.uint8, device=dev)
assert lib.strata_route_tiles(idx.data_ptr(), pairs, k, experts, tile, *[t.data_ptr() for t in ref], ws.data_ptr(),
                              torch.cuda.current_stream().cuda_stream) == 0
torch.cuda.synchronize()
stream = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(stream):
    with torch.cuda.graph(graph, stream=stream):  # the process's first call that allocates nothing
        rc = lib.strata_route_tiles_noalloc(idx.data_ptr(), pairs, k, experts, tile, *[t.data_ptr() for t in outs],
                                            stream.cuda_stream)
assert rc == 0, rc
for rep in range(2):
    graph.replay()
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(outs, ref)), rep
print("first call in a capture: ok")
"""


def test_the_first_call_that_allocates_nothing_can_be_in_a_capture(gpu):
    """A fresh process whose first call of the entry point (the one that looks the array's address up) is inside a
    graph capture: the capture succeeds and its replays give the allocating call's tiles."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    run = subprocess.run([sys.executable, "-c", FIRST_CALL_IN_A_CAPTURE, root], capture_output=True, text=True,
                         timeout=300)
    assert run.returncode == 0 and "first call in a capture: ok" in run.stdout, run.stdout + run.stderr
