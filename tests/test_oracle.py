"""The CPU oracle is pinned before anything is checked against it.

- The IQ3 codebooks: two transcriptions in different encodings (gguf-py's hex in oracle/grids.py, ggml's uint32
  words in the library's tables.h) agree entry by entry, and each grid has ggml's structure.
- Two restatements of every decoder (vectorised numpy, oracle/blocks.py; scalar C following unpack32,
  oracle/unpack.c) agree bit for bit on random blocks.
- Closed forms: Q2_0 (tests/test_gguf.py:34-38 of the reference), Q8_0, Q4_0, Q5_0; ksigns against ggml's first
  entries.
- Encoders restated from ggml's quantize functions (the packing side of each format) round-trip through the
  decoders: a misplaced field, a wrong shift or a transposed index fails one of them.
- Field-by-field checks of IQ3_S / IQ3_XXS / IQ4_XS: one field changed at a time moves exactly the weights it
  should, by exactly the factor it should.
- tiles_of's invariants (tests/test_blocks.py:177-195 of the reference).
- The Q2_0 table of sums: its closed form; on exact inputs the table path is the pinned float64 product rounded
  once; on random inputs within the table's float16 rounding; the lanes of a row only reorder its sum.
- The committed vectors of tests/golden/ (the oracle's own output at a fixed seed) are reproduced bit for bit.
"""

import os
import re

import numpy as np
import pytest

from oracle import blocks as O
from oracle import grids

ROOT_TABLES = "strata_mlx_amd/csrc/tables.h"


def _c_table(name):
    import os

    text = open(os.path.join(os.path.dirname(os.path.dirname(__file__)), ROOT_TABLES)).read()
    body = re.search(name + r"\[\d+\] = \{(.*?)\};", text, re.S).group(1)
    return np.array([int(v, 0) for v in re.findall(r"-?0x[0-9a-fA-F]+|-?\d+", body)], dtype=np.int64)


@pytest.mark.parametrize("name, grid, values, count", [
    ("kStrataIq3xxsGrid", grids.iq3xxs_grid, {4, 12, 20, 28, 36, 44, 52, 62}, 256),
    ("kStrataIq3sGrid", grids.iq3s_grid, set(range(1, 16, 2)), 512)])
def test_the_two_grid_transcriptions_agree_and_have_ggml_structure(name, grid, values, count):
    g = grid()
    assert g.shape == (count, 4)
    assert set(np.unique(g).tolist()) <= values
    words = (g[:, 0].astype(np.int64) | g[:, 1].astype(np.int64) << 8 | g[:, 2].astype(np.int64) << 16
             | g[:, 3].astype(np.int64) << 24)
    assert (np.diff(words) > 0).all()  # distinct and ascending, as ggml lays them out
    assert (g[0] == min(values)).all()  # entry 0 is the all-smallest point
    np.testing.assert_array_equal(_c_table(name), words)


def test_kvalues_are_the_library_table():
    np.testing.assert_array_equal(_c_table("kStrataKvaluesIq4nl"), grids.KVALUES_IQ4NL)


def test_ksigns_closed_form():
    ks = grids.ksigns()
    assert ks[:16].tolist() == [0, 129, 130, 3, 132, 5, 6, 135, 136, 9, 10, 139, 12, 141, 142, 15]  # ggml's first row
    assert all(bin(int(v)).count("1") % 2 == 0 for v in ks)  # eight signs of even parity
    assert ((ks & 127) == np.arange(128)).all()


KINDS = ["Q2_0", "IQ4_NL", "IQ4_XS", "IQ3_S", "IQ3_XXS", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "Q5_0"]


@pytest.mark.parametrize("kind", KINDS)
def test_numpy_and_c_restatements_agree_bit_for_bit(kind):
    from oracle import c_library

    lib = c_library()
    tid, per, size = O.BY_NAME[kind]
    rng = np.random.default_rng(tid)
    rows, cols = 6, 2560
    data = O.random_blocks(kind, rows * cols // per, rng)
    grid = {"IQ3_S": grids.iq3s_grid(), "IQ3_XXS": grids.iq3xxs_grid()}.get(kind, np.zeros((1, 4), np.uint8))
    grid = np.ascontiguousarray(grid)
    out = np.empty((rows, cols), np.float32)
    assert lib.oracle_dequant(tid, data.ctypes.data, rows, cols, cols // per * size, grid.ctypes.data,
                              out.ctypes.data) == 0
    want = O.dequantize(data, kind, (rows, cols))
    np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kind", ["IQ3_S", "Q2_0", "Q4_K"])
def test_c_matvec_is_the_float64_product(kind):
    from oracle import c_library

    lib = c_library()
    tid, per, size = O.BY_NAME[kind]
    rng = np.random.default_rng(3)
    E, rows, cols = 3, 4, 512
    data = O.random_blocks(kind, E * rows * cols // per, rng)
    w = O.dequantize(data, kind, (E, rows, cols))
    idx = np.array([2, 0, 1, 1], dtype=np.uint32)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    grid = np.ascontiguousarray(grids.iq3s_grid())
    out = np.empty((4, rows), np.float32)
    assert lib.oracle_matvec(tid, data.ctypes.data, rows, cols, cols // per * size, idx.ctypes.data, 4,
                             x.ctypes.data, 2, grid.ctypes.data, out.ctypes.data) == 0
    want = O.expert_matvec(w, idx, x, 2)
    assert np.abs(out - want).max() <= 1e-5 * np.abs(w).max() * np.sqrt(cols)


def _f16(v):
    return np.array([v], dtype="<f2").view(np.uint8)


def test_q2_0_closed_form():
    rng = np.random.default_rng(0)
    data = O.random_blocks("Q2_0", 40, rng).reshape(40, 18)
    d = data[:, :2].copy().view("<f2").astype(np.float64)
    codes = np.zeros((40, 64))
    for m in range(16):
        for j in range(4):
            codes[:, 4 * m + j] = (data[:, 2 + m] >> (2 * j)) & 3
    np.testing.assert_array_equal(O.dequantize(data.reshape(-1), "Q2_0", (40, 64)), (d * (codes - 1)).astype(np.float32))


def test_q8_0_q4_0_q5_0_known_blocks():
    q8 = np.zeros(34, np.uint8)
    q8[:2] = _f16(0.5)
    q8[2:] = np.arange(-16, 16, dtype=np.int8).view(np.uint8)
    np.testing.assert_array_equal(O.dequantize(q8, "Q8_0", (1, 32))[0], np.arange(-16, 16) * 0.5)
    q4 = np.zeros(18, np.uint8)
    q4[:2] = _f16(2.0)
    q4[2:] = (np.arange(16) | (np.arange(16)[::-1] << 4)).astype(np.uint8)
    want = np.concatenate([np.arange(16), np.arange(16)[::-1]]) - 8.0
    np.testing.assert_array_equal(O.dequantize(q4, "Q4_0", (1, 32))[0], 2 * want)
    q5 = np.zeros(22, np.uint8)
    q5[:2] = _f16(1.0)
    q5[2:6] = np.array([0xFFFF0000], dtype="<u4").view(np.uint8)  # fifth bits set for weights 16..31
    q5[6:] = 0x21  # low nibble 1, high nibble 2
    want = np.concatenate([np.full(16, 1 - 16), np.full(16, 2 + 16 - 16)]).astype(np.float32)
    np.testing.assert_array_equal(O.dequantize(q5, "Q5_0", (1, 32))[0], want)


# ---- encoders restated from ggml's quantize functions (the packing side), round-tripped through the decoders

def encode_q4_k(d, dmin, sc, mn, q):
    """ggml quantize_row_q4_K packing: sc, mn (8,) 6-bit; q (256,) 4-bit codes."""
    b = np.zeros(144, np.uint8)
    b[0:2], b[2:4] = _f16(d), _f16(dmin)
    s = np.zeros(12, np.int64)
    for j in range(8):
        if j < 4:
            s[j], s[j + 4] = sc[j], mn[j]
        else:
            s[j + 4] = (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    b[4:16] = s
    for j in range(0, 256, 64):
        for l in range(32):
            b[16 + j // 2 + l] = q[j + l] | (q[j + l + 32] << 4)
    return b


def test_q4_k_round_trip():
    rng = np.random.default_rng(1)
    for _ in range(20):
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        d, dmin = float(np.float16(rng.uniform(0.001, 0.1))), float(np.float16(rng.uniform(0.001, 0.1)))
        got = O.dequantize(encode_q4_k(d, dmin, sc, mn, q), "Q4_K", (1, 256))[0]
        want = (np.float32(d) * np.repeat(sc, 32).astype(np.float32)) * q.astype(np.float32) \
            - np.float32(dmin) * np.repeat(mn, 32).astype(np.float32)
        np.testing.assert_array_equal(got, want.astype(np.float32))


def encode_q5_k(d, dmin, sc, mn, q):
    """ggml quantize_row_q5_K packing: Q4_K's fields for the low four bits of q (256,) 5-bit codes, their
    fifth bits in 32 bytes after the scales (weight l of sub-block s at bit s of byte l)."""
    b4 = encode_q4_k(d, dmin, sc, mn, q & 15)
    qh = np.zeros(32, np.int64)
    for s in range(8):
        qh |= (q[32 * s:32 * s + 32] >> 4) << s
    return np.concatenate([b4[:16], qh.astype(np.uint8), b4[16:]])


def test_q5_k_round_trip():
    """A misplaced fifth bit (bit l of byte s rather than bit s of byte l) or a dropped one fails here."""
    rng = np.random.default_rng(2)
    for _ in range(20):
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 32, 256)
        d, dmin = float(np.float16(rng.uniform(0.001, 0.1))), float(np.float16(rng.uniform(0.001, 0.1)))
        block = encode_q5_k(d, dmin, sc, mn, q)
        assert block.size == O.BY_NAME["Q5_K"][2]
        got = O.dequantize(block, "Q5_K", (1, 256))[0]
        want = (np.float32(d) * np.repeat(sc, 32).astype(np.float32)) * q.astype(np.float32) \
            - np.float32(dmin) * np.repeat(mn, 32).astype(np.float32)
        np.testing.assert_array_equal(got, want.astype(np.float32))
        # with every fifth bit clear it is the Q4_K block of the same fields
        low = O.dequantize(encode_q5_k(d, dmin, sc, mn, q & 15), "Q5_K", (1, 256))[0]
        np.testing.assert_array_equal(low, O.dequantize(encode_q4_k(d, dmin, sc, mn, q & 15), "Q4_K", (1, 256))[0])


def encode_q6_k(d, scales, codes):
    """ggml quantize_row_q6_K packing: codes (256,) in -32..31, scales (16,) int8."""
    b = np.zeros(210, np.uint8)
    L = (codes + 32).astype(np.int64)
    for h in range(2):
        for l in range(32):
            q1, q2, q3, q4 = (L[128 * h + l + 32 * i] for i in range(4))
            b[64 * h + l] = (q1 & 15) | ((q3 & 15) << 4)
            b[64 * h + 32 + l] = (q2 & 15) | ((q4 & 15) << 4)
            b[128 + 32 * h + l] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    b[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    b[208:210] = _f16(d)
    return b


def test_q6_k_round_trip():
    rng = np.random.default_rng(2)
    for _ in range(20):
        codes = rng.integers(-32, 32, 256)
        scales = rng.integers(-128, 128, 16)
        d = float(np.float16(rng.uniform(-0.01, 0.01)))
        got = O.dequantize(encode_q6_k(d, scales, codes), "Q6_K", (1, 256))[0]
        want = codes.astype(np.float64) * np.repeat(scales, 16) * d
        np.testing.assert_array_equal(got, want.astype(np.float32))


def encode_q3_k(d, scales, values):
    """ggml quantize_row_q3_K packing: scales (16,) in -32..31, values (256,) in -4..3."""
    b = np.zeros(110, np.uint8)
    s = np.zeros(12, np.int64)
    for j in range(16):
        l = int(scales[j]) + 32
        if j < 8:
            s[j] = l & 0xF
        else:
            s[j - 8] |= (l & 0xF) << 4
        s[j % 4 + 8] |= (l >> 4) << (2 * (j // 4))
    b[96:108] = s
    L = (np.asarray(values) + 4).astype(np.int64)
    hmask = np.zeros(32, np.int64)
    m, hm = 0, 1
    for j in range(256):
        if L[j] > 3:
            hmask[m] |= hm
            L[j] -= 4
        m += 1
        if m == 32:
            m, hm = 0, hm << 1
    b[0:32] = hmask
    for j in range(0, 256, 128):
        for l in range(32):
            b[32 + j // 4 + l] = L[j + l] | (L[j + l + 32] << 2) | (L[j + l + 64] << 4) | (L[j + l + 96] << 6)
    b[108:110] = _f16(d)
    return b


def test_q3_k_round_trip():
    rng = np.random.default_rng(3)
    for _ in range(20):
        scales, values = rng.integers(-32, 32, 16), rng.integers(-4, 4, 256)
        d = float(np.float16(rng.uniform(-0.01, 0.01)))
        got = O.dequantize(encode_q3_k(d, scales, values), "Q3_K", (1, 256))[0]
        want = (d * np.repeat(scales, 16)) * values.astype(np.float64)
        np.testing.assert_array_equal(got, want.astype(np.float32))


def test_iq4_xs_scale_fields():
    """IQ4_XS: the 6-bit scale of run ib is its nibble of scales_l and its two bits of scales_h, less 32."""
    rng = np.random.default_rng(4)
    ls = rng.integers(0, 64, 8)
    b = np.zeros(136, np.uint8)
    b[0:2] = _f16(1.0)
    high = sum(int(ls[ib] >> 4) << (2 * ib) for ib in range(8))
    b[2:4] = np.array([high], dtype="<u2").view(np.uint8)
    for ib in range(8):
        b[4 + ib // 2] |= (ls[ib] & 15) << (4 * (ib % 2))
    q = rng.integers(0, 16, 256)
    for ib in range(8):
        for i in range(16):
            b[8 + 16 * ib + i] = q[32 * ib + i] | (q[32 * ib + 16 + i] << 4)
    got = O.dequantize(b, "IQ4_XS", (1, 256))[0]
    want = np.repeat(ls - 32, 32) * grids.KVALUES_IQ4NL[q]
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_iq3_s_fields_one_at_a_time():
    grid = grids.iq3s_grid().astype(np.float64)
    b = np.zeros(110, np.uint8)
    b[0:2] = _f16(1.0)
    base = O.dequantize(b, "IQ3_S", (1, 256))[0]
    np.testing.assert_array_equal(base, np.tile(grid[0], 64))  # scale nibble 0: dl = 1
    for ib, l in ((0, 0), (3, 5), (7, 7)):
        for idx in (1, 200, 255 + 256):
            c = b.copy()
            c[2 + 8 * ib + l] = idx & 255
            c[66 + ib] = ((idx >> 8) & 1) << l
            w = O.dequantize(c, "IQ3_S", (1, 256))[0]
            at = 32 * ib + 4 * l
            np.testing.assert_array_equal(w[at:at + 4], grid[idx])
            mask = np.ones(256, bool)
            mask[at:at + 4] = False
            np.testing.assert_array_equal(w[mask], base[mask])
    for ib in range(8):  # scale nibbles: run ib is multiplied by 1 + 2 s
        c = b.copy()
        c[106 + ib // 2] = 5 << (4 * (ib % 2))
        w = O.dequantize(c, "IQ3_S", (1, 256))[0]
        np.testing.assert_array_equal(w[32 * ib:32 * ib + 32], 11 * base[32 * ib:32 * ib + 32])
    for k in range(32):  # sign bit k of the run's four sign bytes flips weight k of the run
        c = b.copy()
        c[74 + 4 * 2 + k // 8] = 1 << (k % 8)
        w = O.dequantize(c, "IQ3_S", (1, 256))[0]
        assert w[64 + k] == -base[64 + k] and np.array_equal(np.delete(w, 64 + k), np.delete(base, 64 + k))


def test_iq3_xxs_fields_one_at_a_time():
    grid = grids.iq3xxs_grid().astype(np.float64)
    ks = grids.ksigns()
    b = np.zeros(98, np.uint8)
    b[0:2] = _f16(1.0)
    base = O.dequantize(b, "IQ3_XXS", (1, 256))[0]
    np.testing.assert_array_equal(base, np.tile(grid[0], 64) * 0.25)  # (0.5 + 0) * 0.5
    for ib in range(8):
        aux = (7 << 28) | (5 << 7)  # scale 7; sign index 5 for the run's second pair of groups
        c = b.copy()
        c[66 + 4 * ib:70 + 4 * ib] = np.array([aux], dtype="<u4").view(np.uint8)
        c[2 + 8 * ib + 3] = 77
        w = O.dequantize(c, "IQ3_XXS", (1, 256))[0][32 * ib:32 * ib + 32]
        dl = 7.5 * 0.5
        signs = int(ks[5])  # groups 2 and 3 take its low and high nibble
        for l in range(8):
            g = grid[77 if l == 3 else 0]
            s = (signs >> (4 * (l % 2))) if l in (2, 3) else 0
            for j in range(4):
                assert w[4 * l + j] == (-1 if (s >> j) & 1 else 1) * dl * g[j]


@pytest.mark.parametrize("tokens, k, experts", [(211, 3, 7), (5, 2, 40), (64, 10, 512), (1, 1, 3)])
def test_tiles_hold_every_pair_with_its_expert(tokens, k, experts):
    rng = np.random.default_rng(tokens)
    idx = rng.integers(0, experts, (1, tokens, k))
    idx[0, :tokens // 3] = 1
    if tokens >= 33 and experts > 4:
        idx[0, -33:, 0] = np.repeat([3, 4], [16, 17])
    tile_expert, token, where = O.tiles_of(idx, experts)
    flat = idx.reshape(-1)
    assert len(tile_expert) * 16 == len(token) and len(where) == len(flat)
    assert len(set(where.tolist())) == len(flat)
    np.testing.assert_array_equal(tile_expert[where // 16], flat)
    np.testing.assert_array_equal(token[where], np.arange(len(flat)) // k)
    used = np.zeros(len(tile_expert), bool)
    used[where // 16] = True
    assert (tile_expert[~used] == experts).all() and (tile_expert[used] < experts).all()
    assert used.sum() == sum(-(-c // 16) for c in np.bincount(flat))


def test_swiglu_rounding_is_within_half_ulps_of_silu():
    rng = np.random.default_rng(5)
    g = rng.standard_normal(10000).astype(np.float16)
    u = rng.standard_normal(10000).astype(np.float16)
    got = O.swiglu_rounded(g, u, np.float16).astype(np.float64)
    gf, uf = g.astype(np.float64), u.astype(np.float64)
    exact = gf / (1 + np.exp(-gf)) * uf
    assert np.abs(got - exact).max() <= 4 * 2 ** -11 * np.abs(exact).max()


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_vectors.npz")


def test_the_oracle_still_gives_the_committed_vectors():
    """tests/golden/oracle_vectors.npz (written by tests/golden/make_golden.py): every decoder, the routed matvec,
    the tile layout and the SwiGLU give the committed numbers, bit for bit."""
    gold = np.load(GOLDEN)
    kinds = sorted({k.split("/")[0] for k in gold.files if k.endswith("/blocks") and "/" in k} - {"matvec"})
    assert len(kinds) == 12
    for kind in kinds:
        data = gold[f"{kind}/blocks"]
        per = O.BY_NAME[kind][1]
        n = data.size // O.BY_NAME[kind][2]
        assert np.array_equal(O.dequantize(data, kind, (1, n * per)).astype(np.float32), gold[f"{kind}/weights"])
    w = O.dequantize(gold["matvec/blocks"], "IQ3_S", (3, 2, 256))
    assert np.array_equal(O.expert_matvec(w, gold["matvec/idx"], gold["matvec/x"], 2), gold["matvec/out"])
    te, token, where = O.tiles_of(gold["tiles/indices"], 5, 16)
    assert np.array_equal(te, gold["tiles/tile_expert"]) and np.array_equal(token, gold["tiles/token"])
    assert np.array_equal(where, gold["tiles/where"])
    g, u = gold["swiglu/g"], gold["swiglu/u"]
    assert np.array_equal(O.swiglu_rounded(g, u, np.float16), gold["swiglu/h16"])
    assert np.array_equal(O.swiglu_rounded(g.astype(np.float32), u.astype(np.float32), np.float32),
                          gold["swiglu/h32"])



# ---- the router, its choice and the combine (oracle/fused.py)

def test_top_k_is_a_brute_force_selection_with_ties_to_the_lower_index():
    from oracle import fused as OF

    rng = np.random.default_rng(2)
    logits = rng.integers(-3, 4, (50, 40)).astype(np.float32)  # many ties
    got = OF.top_k(logits, 7)
    for r in range(len(logits)):
        left = list(range(40))
        for q in range(7):
            best = max(left, key=lambda j: (logits[r, j], -j))
            assert got[r, q] == best
            left.remove(best)


def test_softmax_of_the_chosen_has_its_closed_forms():
    from oracle import fused as OF

    eq = np.zeros((1, 16), np.float32)
    idx = OF.top_k(eq, 4)
    assert np.array_equal(idx[0], [0, 1, 2, 3]) and np.allclose(OF.softmax_k(eq, idx), 0.25)
    far = np.array([[0.0, 200.0, 1.0, -5.0]], np.float32)
    idx = OF.top_k(far, 3)
    assert np.array_equal(idx[0], [1, 2, 0]) and OF.softmax_k(far, idx)[0, 0] == 1.0


def test_combine_adds_the_experts_in_the_references_order():
    """fused.py:448-466: experts j, j + 8, ... into partial sum j (each product rounded first), then the partial
    sums in order. With k = 9, partial sum 0 holds the two tiny products (2^-24 each) and reaches 2^-23 before
    the product 1 + 2^-11 (a float16 midpoint) is added: 1 + 2^-11 + 2^-23 rounds up to 1 + 2^-10 in float16. A
    plain left-to-right sum loses each 2^-24 against 1 + 2^-11 and rounds to 1. One-hot weights give y exactly;
    g = -inf drops the shared expert, g = 0 halves it."""
    from oracle import fused as OF

    y = np.ones((1, 9, 256), np.float16)
    w = np.zeros((1, 9), np.float32)
    w[0, 0] = w[0, 8] = 2.0 ** -24
    w[0, 1] = 1.0 + 2.0 ** -11
    s = np.full((1, 256), 3.0, np.float16)
    out = OF.moe_combine(y, w, np.array([-np.inf], np.float16), s)
    assert (out == np.float16(1.0 + 2.0 ** -10)).all()
    rng = np.random.default_rng(1)
    y = rng.standard_normal((2, 8, 256)).astype(np.float16)
    onehot = np.zeros((2, 8), np.float32)
    onehot[0, 5] = onehot[1, 2] = 1.0
    out = OF.moe_combine(y, onehot, np.array([-np.inf, -np.inf], np.float16), s.repeat(2, 0))
    assert np.array_equal(out[0], y[0, 5]) and np.array_equal(out[1], y[1, 2])
    half = OF.moe_combine(np.zeros_like(y), onehot, np.array([0.0, 0.0], np.float16), s.repeat(2, 0))
    assert (half == np.float16(1.5)).all()


# ---- the Q2_0 table of sums (oracle/lookup.py)

def _q2_exact_stack(rng, experts, rows, cols):
    """Q2_0 blocks whose scales are powers of two: with activations that are integers over four, every sum of the
    table path is exact in float32 and float16."""
    data = O.random_blocks("Q2_0", experts * rows * cols // 64, rng).reshape(-1, 18)
    d = (2.0 ** -rng.integers(0, 4, len(data))) * rng.choice([-1.0, 1.0], len(data))
    data[:, :2] = d.astype("<f2").reshape(-1, 1).view(np.uint8)
    return data.reshape(-1)


def test_the_table_has_its_closed_form():
    from oracle import lookup as LK

    rng = np.random.default_rng(5)
    x = (rng.integers(-40, 41, (3, 64)) / 4).astype(np.float16)
    t = LK.lookup_table(x)
    assert t.shape == (3, 32, 16) and t.dtype == np.float16
    for c in range(16):
        want = ((c & 3) - 1) * x[:, 0::2].astype(np.float64) + ((c >> 2) - 1) * x[:, 1::2].astype(np.float64)
        assert np.array_equal(t[:, :, c].astype(np.float64), want)
    # the table of silu(g) * u is the table of those values
    g, u = rng.standard_normal((2, 3, 64)).astype(np.float16)
    h = (g.astype(np.float32) / (1 + np.exp(-g.astype(np.float32))) * u.astype(np.float32)).astype(np.float32)
    glu = LK.lookup_table_glu(g, u)
    for c in range(16):
        want = (np.float32((c & 3) - 1) * h[:, 0::2] + np.float32((c >> 2) - 1) * h[:, 1::2]).astype(np.float16)
        assert np.array_equal(glu[:, :, c], want)


@pytest.mark.parametrize("rows,cols,share,per_row", [(8, 64, 1, 1), (5, 640, 2, 4), (3, 2048, 4, 8), (2, 4096, 8, 32)])
def test_lookup_on_exact_values_is_the_product_of_the_weights(rows, cols, share, per_row):
    """Exact inputs: every sum of the table path is exact, so it gives the float64 product of the decoded weights
    rounded once to float16, bit for bit."""
    from oracle import lookup as LK

    rng = np.random.default_rng(rows + cols)
    experts, pairs = 3, 2 * share
    data = _q2_exact_stack(rng, experts, rows, cols)
    w = O.dequantize(data, "Q2_0", (experts, rows, cols))
    idx = rng.integers(0, experts, pairs)
    x = (rng.integers(-12, 13, (pairs // share, cols)) / 4).astype(np.float16)
    got = LK.lookup_matvec(data, (experts, rows, cols), idx, LK.lookup_table(x), share, per_row)
    want = O.expert_matvec(w, idx, x.astype(np.float64), share)
    assert np.array_equal(got, want.astype(np.float16))


def test_lookup_on_random_values_is_the_product_within_the_tables_rounding():
    from oracle import lookup as LK

    rng = np.random.default_rng(11)
    experts, rows, cols, pairs = 4, 24, 1024, 6
    data = O.random_blocks("Q2_0", experts * rows * cols // 64, rng)
    w = O.dequantize(data, "Q2_0", (experts, rows, cols))
    idx = rng.integers(0, experts, pairs)
    x = rng.standard_normal((pairs, cols)).astype(np.float16)
    got = LK.lookup_matvec(data, (experts, rows, cols), idx, LK.lookup_table(x), 1, 8).astype(np.float64)
    want = O.expert_matvec(w, idx, x.astype(np.float64), 1)
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert 1e-5 < err < 2e-3  # the sums' float16 rounding, and no more


def test_the_lanes_of_a_row_only_reorder_its_sum():
    from oracle import lookup as LK

    rng = np.random.default_rng(2)
    data = _q2_exact_stack(rng, 2, 4, 1024)
    idx, x = np.array([1, 0]), (rng.integers(-8, 9, (2, 1024)) / 4).astype(np.float16)
    table = LK.lookup_table(x)
    outs = [LK.lookup_matvec(data, (2, 4, 1024), idx, table, 1, p) for p in (1, 2, 8, 32)]
    assert all(np.array_equal(o, outs[0]) for o in outs)


def test_q3k_planes_give_the_weights_of_the_blocks():
    """The planes' own formula on the rearranged parts gives what the pinned Q3_K decoder gives on the blocks."""
    rng = np.random.default_rng(8)
    rows, cols = 6, 768
    data = O.random_blocks("Q3_K", rows * cols // 256, rng)
    planes = O.q3k_planes(data, rows, cols)
    assert planes["hm"].shape == (18, 8) and planes["qs"].shape == (18, 16) and planes["sc"].shape == (18, 16)
    assert planes["sc"].min() >= -32 and planes["sc"].max() <= 31
    got = O.q3k_planes_weights(planes, rows, cols)
    assert np.array_equal(got, O.dequantize(data, "Q3_K", (rows, cols)))
