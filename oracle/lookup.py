"""CPU oracle for the Q2_0 table of sums (strata_mlx/blocks.py:697-928).

TEST INFRASTRUCTURE ONLY. Only tests use this module, as the checker. The library never imports it.

The restatement follows the reference's kernels step by step in float32 (numpy rounds every float32 operation):
  - lookup_table: entry c of input pair g is (c & 3 - 1) * a + (c >> 2 - 1) * b in float32, rounded to float16
    (blocks.py:718-726);
  - lookup_table_glu: the same of a = g / (1 + exp(-g)) * u in float32 (blocks.py:728-738);
  - lookup_matvec: lane `part` of `per_row` sums runs part, part + per_row, ...; a run's eight code bytes add
    (lo + hi) to s in order; the run adds d * s to the lane's sum in one fused multiply-add; the row's total is the
    lanes' sums added in lane order, rounded to float16 (blocks.py:741-761).

What pins each function (tests/test_oracle.py):
  - lookup_table: the closed form on inputs whose sums are exact.
  - lookup_matvec: on inputs and scales whose every sum is exact (integers over four, scales powers of two) it is
    the float64 product of the decoded weights (oracle/blocks.py, itself pinned) exactly, which fixes the nibble to
    input pair mapping, the runs' blocks and bytes and the pairs' tokens; on random inputs it is the float64
    product within the float16 rounding of the table's sums.
  - lookup_table_glu: parity unpinned for the sigmoid's exp (Metal's exp in the reference, numpy's float32 exp
    here); its sums are lookup_table's code on silu(g) * u, checked by the same closed form.
"""

import numpy as np


def lookup_table(x: np.ndarray) -> np.ndarray:
    """x (n, cols) float16 -> (n, cols / 2, 16) float16."""
    x = np.asarray(x, np.float16).astype(np.float32)
    return _sums(x[:, 0::2], x[:, 1::2])


def lookup_table_glu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """The table of silu(gate) * up, float32 steps, gate and up (n, cols) float16."""
    g = np.asarray(gate, np.float16).astype(np.float32)
    u = np.asarray(up, np.float16).astype(np.float32)
    with np.errstate(over="ignore"):
        h = g / (np.float32(1.0) + np.exp(-g)) * u
    return _sums(h[:, 0::2], h[:, 1::2])


def _sums(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    c = np.arange(16)
    ia = ((c & 3) - 1).astype(np.float32)
    ib = ((c >> 2) - 1).astype(np.float32)
    return (a[..., None] * ia + b[..., None] * ib).astype(np.float32).astype(np.float16)


def _fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    # a * b is exact in float64 (an 11-bit d times a 24-bit s); one rounding to float32 after the add
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def lookup_matvec(data: np.ndarray, shape: tuple, idx: np.ndarray, table: np.ndarray, share: int,
                  per_row: int) -> np.ndarray:
    """out[p, r] for a Q2_0 stack `data` (bytes) of `shape` (experts, rows, cols), idx (pairs,), table (tokens,
    cols / 2, 16) float16 -> (pairs, rows) float16."""
    experts, rows, cols = shape
    idx = np.asarray(idx, np.int64).reshape(-1)
    pairs = len(idx)
    runs = cols // 32
    blocks = np.asarray(data, np.uint8).reshape(experts, rows, cols // 64, 18)[idx]  # (pairs, rows, blocks, 18)
    d = np.ascontiguousarray(blocks[..., :2]).view("<f2")[..., 0].astype(np.float32)  # (pairs, rows, blocks)
    tab = np.asarray(table, np.float16).astype(np.float32)[np.arange(pairs) // share]  # (pairs, cols / 2, 16)
    prow = np.arange(pairs)[:, None]
    lanes = []
    for part in range(per_row):
        acc = np.zeros((pairs, rows), np.float32)
        for n in range(part, runs, per_row):
            q = blocks[:, :, n // 2, 2 + 8 * (n % 2):10 + 8 * (n % 2)]  # (pairs, rows, 8)
            s = np.zeros((pairs, rows), np.float32)
            for i in range(8):
                c = q[..., i].astype(np.int64)
                lo = tab[prow, 16 * n + 2 * i, c & 15]
                hi = tab[prow, 16 * n + 2 * i + 1, c >> 4]
                s = (s + (lo + hi).astype(np.float32)).astype(np.float32)
            acc = _fma32(d[:, :, n // 2], s, acc)
        lanes.append(acc)
    total = lanes[0]
    for k in range(1, per_row):
        total = (total + lanes[k]).astype(np.float32)
    with np.errstate(over="ignore"):
        return total.astype(np.float16)
