"""A GGUF file straight to the kernels (strata_mlx/load.py:235-273): the uploaded bytes are the file's, and the
layers built on them multiply as the oracle's decode of the same bytes (float64 products, the reference's
tolerances: test_blocks.py:35 for experts, test_dense.py:49 for dense layers)."""

import numpy as np
import pytest
import torch

import gguf_files as W
from oracle import blocks as O
from strata_mlx_amd import gguf as G

pytestmark = pytest.mark.gpu

IDS = {name: type_id for type_id, (name, _, _) in G.TYPES.items()}


def _model(tmp_path, rng):
    """Experts (4, 256, 1024) IQ3_S and IQ3_XXS, a Q6_K and a Q4_K layer, a Q8_0 embedding."""
    spec = [("blk.0.ffn_gate_exps.weight", (4, 256, 1024), "IQ3_S"),
            ("blk.0.ffn_down_exps.weight", (4, 256, 1024), "IQ3_XXS"),
            ("blk.0.attn_q.weight", (96, 512), "Q6_K"), ("blk.0.attn_o.weight", (64, 768), "Q4_K"),
            ("token_embd.weight", (50, 256), "Q8_0")]
    tensors = []
    for name, shape, kind in spec:
        per = O.BY_NAME[kind][1]
        n = int(np.prod(shape)) // per
        tensors.append((name, shape, IDS[kind], O.random_blocks(kind, n, rng).reshape(-1)))
    path = str(tmp_path / "model.gguf")
    W.write(path, tensors, [("general.architecture", W.STRING, "test")], alignment=64)
    return path, {name: (shape, G.TYPES[type_id][0], data) for name, shape, type_id, data in tensors}


def test_uploads_are_the_files_bytes_and_layers_multiply_as_their_weights(gpu, tmp_path):
    rng = np.random.default_rng(5)
    path, spec = _model(tmp_path, rng)
    g = G.GGUF(path)
    for name, (shape, kind, data) in spec.items():
        dev = G.upload(g[name], gpu, stage_bytes=4096)  # many chunks through the two staging buffers
        assert dev.dtype == torch.uint8 and torch.equal(dev.cpu(), torch.from_numpy(data))

    for name in ("blk.0.ffn_gate_exps.weight", "blk.0.ffn_down_exps.weight"):
        shape, kind, data = spec[name]
        lin = G.experts(g[name], gpu)
        w = O.dequantize(data, kind, shape)
        x = rng.standard_normal((3, 1, 1, shape[2])).astype(np.float32)
        idx = np.array([[0, 3], [2, 2], [1, 0]])
        got = lin(torch.from_numpy(x).to(gpu), torch.from_numpy(idx).to(gpu)).cpu().numpy().reshape(6, -1)
        want = O.expert_matvec(w, idx.reshape(-1), x.reshape(3, -1), share=2)
        assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max()

    for name in ("blk.0.attn_q.weight", "blk.0.attn_o.weight"):
        shape, kind, data = spec[name]
        layer = G.linear(g[name], gpu)
        w = O.dequantize(data, kind, shape)
        x = rng.standard_normal((2, shape[1])).astype(np.float32)
        got = layer(torch.from_numpy(x).to(gpu)).cpu().numpy()
        want = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.abs(got - want).max() <= 2e-5 * np.abs(want).max()

    shape, kind, data = spec["token_embd.weight"]
    emb = G.embedding(g["token_embd.weight"], gpu, torch.float32)
    ids = np.array([[7, 0, 49], [3, 3, 12]])
    got = emb(torch.from_numpy(ids).to(gpu)).cpu().numpy()
    assert np.array_equal(got, O.dequantize(data, kind, shape)[ids])
