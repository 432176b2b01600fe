"""CPU oracle for the expert dequant-matmul path: every block decoder and the products on them.

TEST INFRASTRUCTURE ONLY. Only tests, the smoke check and the benchmark's CPU-baseline leg use
this module, as the checker. The library never imports it.

Each decoder restates the reference's per-type decode, vectorised over blocks in numpy:
  - the ten expert types from `unpack32` (strata_mlx/blocks.py:57-194);
  - the dense types from `to_affine` / `q6k_parts` (strata_mlx/gguf.py:150-276).
Every weight is an exact float32 value (an fp16 scale times small integers), so decoding in
float64 and rounding once to float32 is exactly the reference's float32 result. Q4_K and Q5_K are the
exception: `code * (d * sc) + -(dmin * mn)`, one rounding at the add; those are computed in float32
in the reference's order (strata_mlx/gguf.py:207-217, test_gguf.py:55).

What pins each function (tests/test_oracle.py; the reference holds no golden vectors for this path):
  - every decoder: a second, scalar C restatement (unpack.c) agrees bit for bit; closed forms for Q2_0
    (test_gguf.py:34-38 of the reference), Q8_0, Q4_0, Q5_0; encoders restated from ggml's quantize packing
    round-trip through Q4_K, Q6_K, Q3_K; IQ3_S, IQ3_XXS, IQ4_XS moved one field at a time.
  - IQ3_S / IQ3_XXS codebook values: parity unpinned against the reference's own tables (gguf-py 0.19.0, which
    builds them at run time, is absent here). Two transcriptions in different encodings agree entry by entry and
    have ggml's structure; no vector from the reference confirms them.
  - expert_matvec / tile_matmul: float64 products of the decoded weights (the reference's test oracles,
    test_blocks.py:35, 107); the summation order of the reference's Q4_K / Q8_0 products (mlx) is not restated.
  - tiles_of: the invariants of test_blocks.py:177-195.
  - swiglu_rounded: the rounding steps of strata_mlx/blocks.py:222-238, checked against float64 silu within the
    half-ulp bounds those steps allow.
"""

import numpy as np

from . import grids

# GGUF type id -> (name, weights per block, bytes per block); strata_mlx/gguf.py:25-33
TYPES = {
    2: ("Q4_0", 32, 18), 6: ("Q5_0", 32, 22), 8: ("Q8_0", 32, 34),
    11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210),
    20: ("IQ4_NL", 32, 18), 23: ("IQ4_XS", 256, 136), 42: ("Q2_0", 64, 18),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 21: ("IQ3_S", 256, 110),
    22: ("IQ2_S", 256, 82), 29: ("IQ1_M", 256, 56),
}
BY_NAME = {name: (tid, per, size) for tid, (name, per, size) in TYPES.items()}
# the expert types of strata_mlx/blocks.py:36-38
BLOCK = {k: BY_NAME[k][1:] for k in ("IQ4_NL", "IQ4_XS", "IQ3_S", "IQ3_XXS", "IQ2_S", "IQ2_XS", "IQ2_XXS",
                                     "IQ1_M", "Q2_0", "Q3_K")}
# types whose codebooks are not available here (their grids were not transcribed)
NO_GRID = ("IQ2_S", "IQ2_XS", "IQ2_XXS", "IQ1_M")
# where each block keeps its fp16 scales (tests/test_gguf.py:12-14)
SCALE_BYTES = {"Q2_0": [0], "Q4_0": [0], "Q5_0": [0], "Q8_0": [0], "IQ4_NL": [0], "IQ4_XS": [0],
               "Q4_K": [0, 2], "Q5_K": [0, 2], "Q3_K": [108], "Q6_K": [208],
               "IQ3_S": [0], "IQ3_XXS": [0], "IQ2_S": [0], "IQ2_XS": [0], "IQ2_XXS": [0], "IQ1_M": []}


def _f16(b: np.ndarray, at: int) -> np.ndarray:
    return np.ascontiguousarray(b[:, at:at + 2]).view("<f2")[:, 0].astype(np.float64)


def _u16(b: np.ndarray, at: int) -> np.ndarray:
    return b[:, at].astype(np.uint32) | (b[:, at + 1].astype(np.uint32) << 8)


def _u32(b: np.ndarray, at: int) -> np.ndarray:
    return _u16(b, at) | (_u16(b, at + 2) << 16)


def _signed(values: np.ndarray, sign_bits: np.ndarray) -> np.ndarray:
    return np.where(sign_bits.astype(bool), -values, values)


def _q2_0(b):
    # blocks.py:58-68: run n of a row is block n/2, code bytes 2 + 8(n%2); w[4i+j] = d((q[i] >> 2j & 3) - 1)
    d = _f16(b, 0)
    code = np.stack([(b[:, 2:18] >> s) & 3 for s in (0, 2, 4, 6)], axis=2).reshape(-1, 64)
    return d[:, None] * (code.astype(np.float64) - 1)


def _iq4_nl(b):
    # blocks.py:69-77
    d = _f16(b, 0)
    q = b[:, 2:18]
    kv = grids.KVALUES_IQ4NL.astype(np.float64)
    return d[:, None] * np.concatenate([kv[q & 15], kv[q >> 4]], axis=1)


def _iq4_xs(b):
    # blocks.py:78-88
    n = len(b)
    d = _f16(b, 0)
    kv = grids.KVALUES_IQ4NL.astype(np.float64)
    out = np.empty((n, 8, 32))
    high = _u16(b, 2)
    for ib in range(8):
        ls = ((b[:, 4 + ib // 2].astype(np.uint32) >> (4 * (ib % 2))) & 15) | (((high >> (2 * ib)) & 3) << 4)
        dl = d * (ls.astype(np.float64) - 32)
        q = b[:, 8 + 16 * ib: 24 + 16 * ib]
        out[:, ib] = dl[:, None] * np.concatenate([kv[q & 15], kv[q >> 4]], axis=1)
    return out.reshape(n, 256)


def _iq3_s(b):
    # blocks.py:89-102
    n = len(b)
    grid = grids.iq3s_grid().astype(np.float64)
    d = _f16(b, 0)
    out = np.empty((n, 8, 8, 4))
    for ib in range(8):
        dl = d * (1 + 2 * ((b[:, 106 + ib // 2].astype(np.uint32) >> (4 * (ib % 2))) & 15)).astype(np.float64)
        high = b[:, 66 + ib].astype(np.uint32)
        for l in range(8):
            g = grid[b[:, 2 + 8 * ib + l].astype(np.uint32) | (((high >> l) & 1) << 8)]
            sign = b[:, 74 + 4 * ib + l // 2].astype(np.uint32) >> (4 * (l % 2))
            for j in range(4):
                out[:, ib, l, j] = _signed(dl * g[:, j], (sign >> j) & 1)
    return out.reshape(n, 256)


def _iq3_xxs(b):
    # blocks.py:103-116
    n = len(b)
    grid = grids.iq3xxs_grid().astype(np.float64)
    ks = grids.ksigns().astype(np.uint32)
    d = _f16(b, 0)
    out = np.empty((n, 8, 8, 4))
    for ib in range(8):
        aux = _u32(b, 66 + 4 * ib)
        dl = d * (0.5 + (aux >> 28).astype(np.float64)) * 0.5
        for l in range(8):
            g = grid[b[:, 2 + 8 * ib + l]]
            sign = ks[(aux >> (7 * (l // 2))) & 127] >> (4 * (l % 2))
            for j in range(4):
                out[:, ib, l, j] = _signed(dl * g[:, j], (sign >> j) & 1)
    return out.reshape(n, 256)


def _q3k_scale(s: np.ndarray, k: int) -> np.ndarray:
    # blocks.py:49-53: the k-th 6-bit scale, less 32
    p, word = k % 4, k // 4
    low = (s[:, 4 * word + p].astype(np.int64) & 15) if word < 2 else (s[:, 4 * (word - 2) + p].astype(np.int64) >> 4)
    return (low | (((s[:, 8 + p].astype(np.int64) >> (2 * word)) & 3) << 4)) - 32


def _q3_k(b):
    # blocks.py:164-175
    n = len(b)
    d = _f16(b, 108)
    out = np.empty((n, 8, 32))
    for r in range(8):
        q = b[:, 32 + 32 * (r // 4): 64 + 32 * (r // 4)].astype(np.int64)
        shift = 2 * (r % 4)
        s0 = d * _q3k_scale(b[:, 96:108], 2 * r)
        s1 = d * _q3k_scale(b[:, 96:108], 2 * r + 1)
        v = ((q >> shift) & 3) - np.where((b[:, 0:32].astype(np.int64) >> r) & 1, 0, 4)
        out[:, r, :16] = s0[:, None] * v[:, :16]
        out[:, r, 16:] = s1[:, None] * v[:, 16:]
    return out.reshape(n, 256)


def _k4_scales(p):
    # gguf.py:174-179
    p = p.astype(np.uint8)
    sc = np.concatenate([p[:, :4] & 63, (p[:, 8:12] & 15) | ((p[:, :4] >> 6) << 4)], axis=1)
    mn = np.concatenate([p[:, 4:8] & 63, (p[:, 8:12] >> 4) | ((p[:, 4:8] >> 6) << 4)], axis=1)
    return sc.astype(np.float32), mn.astype(np.float32)


def _nibbles(qs, run=16):
    # gguf.py:168-171
    qs = qs.reshape(-1, run)
    return np.concatenate([qs & 15, qs >> 4], axis=1)


def _q4_k(b):
    # gguf.py:207-213, in float32 as the reference multiplies and adds
    n = len(b)
    d = _f16(b, 0).astype(np.float32)[:, None]
    dmin = _f16(b, 2).astype(np.float32)[:, None]
    sc, mn = _k4_scales(b[:, 4:16])
    scales, biases = d * sc, -(dmin * mn)
    codes = _nibbles(b[:, 16:144], 32).reshape(n, 8, 32).astype(np.float32)
    return (codes * scales[:, :, None] + biases[:, :, None]).reshape(n, 256)


def _q5_k(b):
    # gguf.py:207-218
    n = len(b)
    d = _f16(b, 0).astype(np.float32)[:, None]
    dmin = _f16(b, 2).astype(np.float32)[:, None]
    sc, mn = _k4_scales(b[:, 4:16])
    scales, biases = d * sc, -(dmin * mn)
    qh = b[:, 16:48]
    high = np.stack([(qh >> s) & 1 for s in range(8)], axis=1)
    codes = (_nibbles(b[:, 48:176], 32).reshape(n, 8, 32) | (high << 4)).astype(np.float32)
    return (codes * scales[:, :, None] + biases[:, :, None]).reshape(n, 256)


def _q6_k(b):
    # gguf.py:150-165 (q6k_parts) and 143-146 (to_float): w = code * scale * d
    n = len(b)
    ql, qh = b[:, :128].reshape(-1, 2, 64), b[:, 128:192].reshape(-1, 2, 32)
    hi = np.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], axis=2)
    lo = np.stack([ql[..., :32] & 15, ql[..., 32:] & 15, ql[..., :32] >> 4, ql[..., 32:] >> 4], axis=2)
    codes = ((lo | (hi << 4)).astype(np.int64) - 32).reshape(n, 256)
    scales = np.ascontiguousarray(b[:, 192:208]).view(np.int8).astype(np.float64)
    d = _f16(b, 208)
    return codes * np.repeat(scales, 16, axis=1) * d[:, None]


def _q8_0(b):
    # gguf.py:203-206: (q + 128) d - 128 d = q d, exact
    return _f16(b, 0)[:, None] * np.ascontiguousarray(b[:, 2:34]).view(np.int8).astype(np.float64)


def _q4_0(b):
    # gguf.py:195-197
    return _f16(b, 0)[:, None] * (_nibbles(b[:, 2:18]).astype(np.float64) - 8)


def _q5_0(b):
    # gguf.py:198-202
    high = (_u32(b, 2)[:, None] >> np.arange(32, dtype=np.uint32)) & 1
    codes = _nibbles(b[:, 6:22]).astype(np.uint32) | (high << 4)
    return _f16(b, 0)[:, None] * (codes.astype(np.float64) - 16)


_DECODE = {"Q2_0": _q2_0, "IQ4_NL": _iq4_nl, "IQ4_XS": _iq4_xs, "IQ3_S": _iq3_s, "IQ3_XXS": _iq3_xxs,
           "Q3_K": _q3_k, "Q4_K": _q4_k, "Q5_K": _q5_k, "Q6_K": _q6_k, "Q8_0": _q8_0, "Q4_0": _q4_0,
           "Q5_0": _q5_0}


def dequantize(data: np.ndarray, kind: str, shape: tuple) -> np.ndarray:
    """The weights of `data` (uint8 bytes of a tensor of `shape`, rows along the last axis) as float32.

    strata_mlx/blocks.py:515-522 (the dequant kernel) and gguf.py:135-147, 182-276 (the CPU forms)."""
    if kind not in _DECODE:
        raise ValueError(f"{kind}: no decoder in the oracle")
    _, per_block, block_bytes = BY_NAME[kind]
    if shape[-1] % per_block:
        raise ValueError(f"{kind}: rows of {shape[-1]} weights do not end on a block of {per_block}")
    b = np.asarray(data, dtype=np.uint8).reshape(-1, block_bytes)
    w = _DECODE[kind](b)
    return w.astype(np.float32).reshape(shape)


def random_blocks(kind: str, n_blocks: int, rng: np.random.Generator, lo: float = -0.05, hi: float = 0.05,
                  scale: str = "uniform") -> np.ndarray:
    """Random blocks as the reference's tests make them (tests/test_gguf.py:17-30): uniform bytes, the fp16
    scales replaced by U(lo, hi), or by |N(0,1)| * 0.01 when scale == "normal" (the benchmark inputs)."""
    _, _, block_bytes = BY_NAME[kind]
    b = rng.integers(0, 256, (n_blocks, block_bytes), dtype=np.uint8)

    def draw(size):
        if scale == "normal":
            return (np.abs(rng.standard_normal(size)) * 0.01).astype("<f2")
        return rng.uniform(lo, hi, size).astype("<f2")

    for at in SCALE_BYTES[kind]:
        b[:, at:at + 2] = draw((n_blocks, 1)).view(np.uint8)
    if kind == "IQ1_M":
        d = draw(n_blocks).view("<u2")
        words = b[:, 48:56].copy().view("<u2")
        for i in range(4):
            words[:, i] = (words[:, i] & 0x0FFF) | (((d >> (4 * i)) & 15) << 12)
        b[:, 48:56] = words.view(np.uint8)
    return b.reshape(-1)


# ---- products on the weights (float64 oracles, as the reference's tests compute them)

def expert_matvec(w: np.ndarray, idx: np.ndarray, x: np.ndarray, share: int) -> np.ndarray:
    """out[p] = W[idx[p]] . x[p // share] in float64; w (E, rows, cols). strata_mlx/blocks.py:196-220, 538-554."""
    idx = np.asarray(idx).reshape(-1)
    xs = np.asarray(x, dtype=np.float64).reshape(-1, w.shape[-1])
    rows = xs[np.arange(len(idx)) // share]
    out = np.empty((len(idx), w.shape[1]))
    for e in np.unique(idx):  # an expert at a time: memory of one expert's weights, whatever the pair count
        at = np.nonzero(idx == e)[0]
        out[at] = rows[at] @ w[e].astype(np.float64).T
    return out


def swiglu_rounded(g: np.ndarray, u: np.ndarray, dtype) -> np.ndarray:
    """silu(g) * u as mlx-lm rounds it (strata_mlx/blocks.py:222-238): the sigmoid in float32 rounded to the
    activations' type, then g * sig and that times u, each product rounded to that type."""
    g = np.asarray(g).astype(dtype)
    u = np.asarray(u).astype(dtype)
    gf = g.astype(np.float64)
    y = 1.0 / (1.0 + np.exp(np.abs(gf)))
    sig = np.where(gf < 0, y, 1 - y).astype(np.float32).astype(dtype)
    a = (gf * sig.astype(np.float64)).astype(dtype)
    return (a.astype(np.float64) * u.astype(np.float64)).astype(dtype)


def tiles_of(indices: np.ndarray, experts: int, tile: int = 16):
    """The pairs of `indices` laid out in tiles of `tile`, each tile one expert's; strata_mlx/blocks.py:657-681.

    Returns (tile_expert, token, where), the tile count P // tile + min(E, P) whatever the routing. Slots within
    an expert go in pair order."""
    k = indices.shape[-1] if np.ndim(indices) else 1
    flat = np.asarray(indices).reshape(-1).astype(np.int64)
    pairs = len(flat)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=experts)[:experts]
    tiles = (counts + tile - 1) // tile
    tile_end, pair_end = np.cumsum(tiles), np.cumsum(counts)
    expert = flat[order]
    slot = (tile_end - tiles)[expert] * tile + np.arange(pairs) - (pair_end - counts)[expert]
    most = pairs // tile + min(experts, pairs)
    token = np.zeros(most * tile, dtype=np.int64)
    token[slot] = order // k
    where = np.zeros(pairs, dtype=np.int64)
    where[order] = slot
    tile_expert = (tile_end[None] <= np.arange(most)[:, None]).sum(axis=1)
    return tile_expert.astype(np.uint32), token.astype(np.uint32), where.astype(np.uint32)


def tile_matmul(w: np.ndarray, a: np.ndarray, tile_expert: np.ndarray, round_to=None, tile: int = 16) -> np.ndarray:
    """c[p] = W[expert of p's tile] . a[p]; weights rounded to `round_to` first (strata_mlx/blocks.py:634-654).
    Tiles naming no expert (>= E) give zeros here; the reference leaves those rows undefined."""
    experts = w.shape[0]
    wf = w.astype(round_to).astype(np.float64) if round_to is not None else w.astype(np.float64)
    out = np.zeros((len(a), w.shape[1]))
    for t, e in enumerate(np.asarray(tile_expert)):
        if e < experts:
            out[t * tile:(t + 1) * tile] = a[t * tile:(t + 1) * tile].astype(np.float64) @ wf[e].T
    return out


# ---- Q3_K held as planes (strata_mlx/blocks.py:397-512)

def q3k_planes(data: np.ndarray, rows: int, cols: int) -> dict:
    """The planes of a Q3_K tensor's bytes: hm (blocks, 8) uint32, qs (blocks, 16) uint32, sc (blocks, 16) int8
    (the 6-bit scales decoded, less 32), dd (blocks,) float16. strata_mlx/blocks.py:403-414."""
    b = np.asarray(data, np.uint8).reshape(-1, 110)[: rows * cols // 256]
    sc = np.stack([_q3k_scale(b[:, 96:108], k) for k in range(16)], axis=1).astype(np.int8)
    return {"hm": np.ascontiguousarray(b[:, 0:32]).view("<u4").copy(),
            "qs": np.ascontiguousarray(b[:, 32:96]).view("<u4").copy(),
            "sc": sc,
            "dd": np.ascontiguousarray(b[:, 108:110]).view("<f2")[:, 0].copy()}


def q3k_planes_weights(planes: dict, rows: int, cols: int) -> np.ndarray:
    """The weights the planes give by the planes' own formula (strata_mlx/blocks.py:419-422, 464-479): weight
    4w + k of run rr = 4n + j is d * sc[2rr + (w >= 4)] * (((qs[8n + w] >> (8k + 2j)) & 3) - (bit 8k + rr of
    hm[w] ? 0 : 4)); float32."""
    hm, qs = planes["hm"].astype(np.int64), planes["qs"].astype(np.int64)
    sc, d = planes["sc"].astype(np.float64), planes["dd"].astype(np.float64)
    out = np.empty((len(d), 8, 32))
    for rr in range(8):
        n, j = divmod(rr, 4)
        for w in range(8):
            for k in range(4):
                v = ((qs[:, 8 * n + w] >> (8 * k + 2 * j)) & 3) - np.where((hm[:, w] >> (8 * k + rr)) & 1, 0, 4)
                out[:, rr, 4 * w + k] = d * sc[:, 2 * rr + (w >= 4)] * v
    return out.reshape(rows, cols).astype(np.float32)
