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
