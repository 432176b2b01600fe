"""CPU oracle for the router, top-k and combine either side of the expert path (strata_mlx/fused.py:334-497).

TEST INFRASTRUCTURE ONLY. Only tests use this module, as the checker. The library never imports it.

What pins each function (tests/test_oracle.py):
  - router_matvec: the float64 product (the reference's kernel sums in float32 in its own order; a tolerance).
  - top_k: a brute-force selection on small inputs with many ties, and the order a stable sort gives.
  - softmax_k: closed forms (equal logits give 1/k; a logit far above the rest gives 1) and the float64 form.
  - moe_combine: the reference's order and rounding (fused.py:448-466) restated in float32 / float16 steps,
    checked on cases that fix each step: one-hot weights give y exactly, g -> -inf drops the shared expert,
    the order of the eight partial sums on values where float32 addition is not associative. The sigmoid's exp
    is parity unpinned: the reference uses Metal's fast exp, this restatement float32 numpy exp.
"""

import numpy as np


def router_matvec(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """out[t, r] = w[r, :] . x[t, :] in float64 (strata_mlx/fused.py:334-353)."""
    return np.asarray(x, np.float64) @ np.asarray(w, np.float64).T


def top_k(logits: np.ndarray, k: int) -> np.ndarray:
    """The k largest of each row, largest first, ties to the lower index (strata_mlx/fused.py:400-436)."""
    return np.argsort(-np.asarray(logits, np.float32), axis=-1, kind="stable")[..., :k].astype(np.int64)


def softmax_k(logits: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """softmax over the chosen logits (strata_mlx/fused.py:490-491), float64 rounded to float32."""
    v = np.take_along_axis(np.asarray(logits, np.float64), idx, axis=-1)
    e = np.exp(v - v.max(axis=-1, keepdims=True))
    return (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)


def moe_combine(y: np.ndarray, w: np.ndarray, g: np.ndarray, s: np.ndarray) -> np.ndarray:
    """y (rows, K, D) float16, w (rows, K) float32, g (rows,) float16, s (rows, D) float16 -> (rows, D) float16,
    each step rounded as strata_mlx/fused.py:448-466 rounds it."""
    y = np.asarray(y, np.float16).astype(np.float32)
    w = np.asarray(w, np.float32)
    rows, k, d = y.shape
    acc = np.zeros((rows, d), np.float32)
    for j in range(min(8, k)):
        part = np.zeros((rows, d), np.float32)
        for q in range(j, k, 8):
            part = (y[:, q, :] * w[:, q:q + 1]).astype(np.float32) + part
        acc = part if j == 0 else (part + acc).astype(np.float32)
    routed = acc.astype(np.float16)
    gf = np.asarray(g, np.float16).astype(np.float32).reshape(rows, 1)
    gate = (np.float32(1.0) / (np.float32(1.0) + np.exp(-gf))).astype(np.float16)
    shared = (gate.astype(np.float32) * np.asarray(s, np.float16).astype(np.float32)).astype(np.float16)
    return (routed.astype(np.float32) + shared.astype(np.float32)).astype(np.float16)
