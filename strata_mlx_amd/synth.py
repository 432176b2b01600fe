"""Synthetic inputs of the benchmark workloads, made on the GPU.

Blocks: uniform random bytes with every fp16 scale field replaced by |N(0,1)| * 0.01 (the layouts' scale
offsets, as tests/test_gguf.py:12-14 of the reference lists them). Routing: the experts get a random
permutation of Zipf(s) probabilities, and each token takes the top-k of log p + Gumbel(0, 1), i.e. k
draws without replacement; the weights are the softmax over the chosen logits (strata_mlx/fused.py:490-491).
"""

import numpy as np
import torch

from .blocks import BLOCK, DENSE

SCALE_BYTES = {"Q2_0": [0], "Q4_0": [0], "Q5_0": [0], "Q8_0": [0], "IQ4_NL": [0], "IQ4_XS": [0],
               "Q4_K": [0, 2], "Q5_K": [0, 2], "Q3_K": [108], "Q6_K": [208], "IQ3_S": [0], "IQ3_XXS": [0]}


def random_stack(kind: str, n_weights: int, device, generator: torch.Generator | None = None) -> torch.Tensor:
    """Random blocks of `kind` holding n_weights weights, as a flat uint8 tensor on `device`."""
    per_block, block_bytes = {**BLOCK, **DENSE}[kind]
    if n_weights % per_block:
        raise ValueError("not whole blocks")
    n = n_weights // per_block
    b = torch.randint(0, 256, (n, block_bytes), dtype=torch.uint8, device=device, generator=generator)
    for at in SCALE_BYTES[kind]:
        d = (torch.randn(n, device=device, generator=generator).abs() * 0.01).half()
        b[:, at:at + 2] = d.view(torch.uint8).reshape(n, 2)
    return b.reshape(-1)


def zipf_routing(tokens: int, experts: int, k: int, rng: np.random.Generator, s: float = 1.1):
    """(indices (tokens, k) int64, weights (tokens, k) float32) drawn as described above."""
    p = 1.0 / np.arange(1, experts + 1) ** s
    p = (p / p.sum())[rng.permutation(experts)]
    logits = np.log(p)[None, :] + rng.gumbel(size=(tokens, experts))
    idx = np.argsort(-logits, axis=1)[:, :k]
    chosen = np.take_along_axis(logits, idx, axis=1)
    w = np.exp(chosen - chosen.max(axis=1, keepdims=True))
    return idx.astype(np.int64), (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
