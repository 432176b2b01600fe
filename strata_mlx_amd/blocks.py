"""Experts computed on the GGUF file's own blocks, on gfx950: the call surface of strata_mlx/blocks.py.

The blocks go to the GPU as the file's bytes (a uint8 tensor) and hand-written HIP kernels read them:

    matvec     out[pair, row] = W[expert of pair, row, :] . x     decode: bandwidth-bound, no MFMA
               (also with every pair's expert as an array of its own: matvec_separate)
    window     the same for one layer and a window of tokens (window_matvec, dense.BlockLinear)
    lookup     Q2_0 over float16 from a table of the 16 sums of each input pair (lookup_table, lookup_matvec,
               lookup_gate_up, lookup_down_glu)
    planes     Q3_K rearranged once into aligned planes (q3k_planes, q3k_planes_window, q3k_planes_dequantize)
    tiles      a prompt's pairs sorted by expert into tiles; weights decoded into LDS, MFMA products
    dequant    every weight of the stack as float16 or float32, bit-exact

Sums are float32 whatever the type of the activations. Arguments mirror the reference's, with torch
tensors on the GPU in place of mx.array.
"""

import torch

from . import _lib

# type -> (weights per block, bytes per block); strata_mlx/blocks.py:36-38
BLOCK = {"IQ4_NL": (32, 18), "IQ4_XS": (256, 136), "IQ3_S": (256, 110), "IQ3_XXS": (256, 98),
         "IQ2_S": (256, 82), "IQ2_XS": (256, 74), "IQ2_XXS": (256, 66), "IQ1_M": (256, 56), "Q2_0": (64, 18),
         "Q3_K": (256, 110)}
# the dense types of the loader, decoded by the same kernels (strata_mlx/gguf.py:25-33)
DENSE = {"Q4_0": (32, 18), "Q5_0": (32, 22), "Q8_0": (32, 34), "Q4_K": (256, 144), "Q5_K": (256, 176),
         "Q6_K": (256, 210)}
# these types' codebooks are not in the package (no source of them to pin against): the kernels refuse them
NO_GRID = ("IQ2_S", "IQ2_XS", "IQ2_XXS", "IQ1_M")

TOKENS_TILE = 16  # slots of a tile (strata_mlx/blocks.py:581)
TILES_FROM = 1600  # (token, expert) pairs from which a prompt goes through tiles (strata_mlx/blocks.py:580)
MATVEC_GLU_UPTO = 1 << 16  # pairs for which down takes silu(gate) * up itself (the reference: 30)


def row_bytes(kind: str, cols: int) -> int:
    per_block, block_bytes = {**BLOCK, **DENSE}[kind]
    if cols % per_block:
        raise ValueError(f"{kind}: rows of {cols} weights do not end on a block of {per_block}")
    return cols // per_block * block_bytes


def _flat_u8(blocks: torch.Tensor) -> torch.Tensor:
    if blocks.dtype != torch.uint8:
        raise ValueError("blocks must be the file's bytes, uint8")
    _lib.require_device(blocks)
    return blocks


def dequantize(blocks: torch.Tensor, kind: str, shape: tuple, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """The weights of `blocks` (uint8, a tensor of `shape` as the file holds it) as floats, bit-exact.
    strata_mlx/blocks.py:515-522."""
    *lead, rows, cols = shape
    n = 1
    for v in lead:
        n *= v
    _flat_u8(blocks)
    if blocks.numel() < n * rows * row_bytes(kind, cols):
        raise ValueError("blocks hold fewer bytes than the shape needs")
    out = torch.empty(tuple(shape), dtype=dtype, device=blocks.device)
    if dtype not in (torch.float32, torch.float16):
        raise ValueError("dequantize gives float32 or float16")
    _lib.check(_lib.library().strata_dequant(_lib.kind_id(kind), blocks.data_ptr(), n, rows, cols, out.data_ptr(),
                                             _lib.dtype_id(dtype), _lib.stream()), f"dequantize {kind}")
    return out


def _idx32(indices: torch.Tensor) -> torch.Tensor:
    return indices.reshape(-1).to(torch.int32).contiguous()


class BlockSwitchLinear:
    """The experts' matrices of one projection (gate, up or down) as the GGUF bytes of an (experts, out, in) stack
    on the GPU, with the call signature of mlx-lm's routed linear: each (token, expert) pair multiplies its token's
    row by its expert's matrix. strata_mlx/blocks.py:525-558."""

    unpack_from = 5000  # pairs from which the reference multiplies unpacked floats; here a kernel either way

    def __init__(self, blocks: torch.Tensor, kind: str, shape: tuple, per_row: int | None = None):
        self.blocks, self.kind = _flat_u8(blocks), kind
        self.num_experts, self.output_dims, self.input_dims = shape
        self.row_bytes = row_bytes(kind, self.input_dims)
        if blocks.numel() < self.num_experts * self.output_dims * self.row_bytes:
            raise ValueError("blocks hold fewer bytes than the shape needs")
        self.per_row = per_row  # accepted for the reference's signature; the kernel sets its own split

    def __call__(self, x: torch.Tensor, indices: torch.Tensor, sorted_indices: bool = False) -> torch.Tensor:
        """The routed products for `indices`: x is (..., 1, in); every index multiplies the row of x it belongs to
        (one row per index, or one row shared by the k indices of a token). Returns (..., k, 1, out)."""
        indices = torch.as_tensor(indices, device=x.device)
        batch, k = tuple(x.shape[:-2]), (indices.shape[-1] if indices.ndim else 1)
        ishape = tuple(indices.shape)
        if batch == ishape:
            share = 1
        elif batch == (*ishape[:-1], 1):
            share = k
        else:
            x, share = x.expand(*ishape, 1, self.input_dims), 1
        pairs = indices.numel()
        x2 = x.reshape(-1, self.input_dims).contiguous()
        out = torch.empty((pairs, self.output_dims), dtype=x.dtype, device=x.device)
        idx = _idx32(indices)
        _lib.check(_lib.library().strata_expert_matvec(
            _lib.kind_id(self.kind), self.blocks.data_ptr(), self.num_experts, self.output_dims, self.input_dims,
            idx.data_ptr(), pairs, x2.data_ptr(), _lib.dtype_id(x.dtype), share, out.data_ptr(), _lib.stream()),
            f"matvec {self.kind}")
        return out.reshape(*ishape, 1, self.output_dims)


def gate_up(gate: BlockSwitchLinear, up: BlockSwitchLinear, x: torch.Tensor, idx: torch.Tensor, share: int):
    """(gate . x, up . x) for every pair in one launch; x (pairs / share, in), idx (pairs,) -> two (pairs, out)."""
    if (gate.kind, gate.output_dims, gate.input_dims, gate.num_experts) != (up.kind, up.output_dims, up.input_dims,
                                                                             up.num_experts):
        raise ValueError("gate and up differ in type or shape")
    pairs = idx.numel()
    x2 = x.reshape(-1, gate.input_dims).contiguous()
    g = torch.empty((pairs, gate.output_dims), dtype=x.dtype, device=x.device)
    u = torch.empty_like(g)
    idx = _idx32(idx)
    _lib.check(_lib.library().strata_expert_matvec2(
        _lib.kind_id(gate.kind), gate.blocks.data_ptr(), up.blocks.data_ptr(), gate.num_experts, gate.output_dims,
        gate.input_dims, idx.data_ptr(), pairs, x2.data_ptr(), _lib.dtype_id(x.dtype), share, g.data_ptr(),
        u.data_ptr(), _lib.stream()), f"gate/up {gate.kind}")
    return g, u


def gate_up_swiglu(gate: BlockSwitchLinear, up: BlockSwitchLinear, x: torch.Tensor, idx: torch.Tensor, share: int):
    """gate_up with silu(gate) * up as well, rounded as mlx-lm rounds it: three (pairs, out). IQ3_S, IQ3_XXS and
    Q2_0 in float16 do it in one launch (a lane ends with both sums of a row); other types and dtypes add a small
    elementwise launch. The gate and up calls of strata_mlx/blocks.py:969-975 with the SwiGLU of its down call."""
    if (gate.kind, gate.output_dims, gate.input_dims, gate.num_experts) != (up.kind, up.output_dims, up.input_dims,
                                                                             up.num_experts):
        raise ValueError("gate and up differ in type or shape")
    pairs = idx.numel()
    x2 = x.reshape(-1, gate.input_dims).contiguous()
    g = torch.empty((pairs, gate.output_dims), dtype=x.dtype, device=x.device)
    u, h = torch.empty_like(g), torch.empty_like(g)
    idx = _idx32(idx)
    _lib.check(_lib.library().strata_expert_gate_up_swiglu(
        _lib.kind_id(gate.kind), gate.blocks.data_ptr(), up.blocks.data_ptr(), gate.num_experts, gate.output_dims,
        gate.input_dims, idx.data_ptr(), pairs, x2.data_ptr(), _lib.dtype_id(x.dtype), share, g.data_ptr(),
        u.data_ptr(), h.data_ptr(), _lib.stream()), f"gate/up/swiglu {gate.kind}")
    return g, u, h


def gate_up_swiglu_shared(gate: BlockSwitchLinear, up: BlockSwitchLinear, x: torch.Tensor, idx: torch.Tensor,
                          shared_gate, shared_up, with_shared_gu: bool = False):
    """gate_up_swiglu at one token with a shared expert's gate and up (layers of the file's Q4_K blocks with
    `blocks`, `kind`, `output_dims`, `input_dims`: dense.BlockLinear) in the same launch: (g, u, h) of the pairs
    and the shared expert's h (1, shared rows), and its own gate . x and up . x (1, shared rows) after those if
    with_shared_gu. None where the launch does not take the case (other types, several tokens, inputs other than
    4096): the caller then makes the two calls apart. The routed experts' and the shared expert's gate and up of
    strata_mlx/fused.py:492-493, with the SwiGLU of their down calls."""
    if (gate.kind, gate.output_dims, gate.input_dims, gate.num_experts) != (up.kind, up.output_dims, up.input_dims,
                                                                             up.num_experts):
        raise ValueError("gate and up differ in type or shape")
    if (shared_gate.kind, shared_gate.output_dims, shared_gate.input_dims) != (
            shared_up.kind, shared_up.output_dims, shared_up.input_dims) or shared_gate.input_dims != gate.input_dims:
        raise ValueError("the shared expert's gate and up differ in type or shape from each other or the token")
    if getattr(shared_gate, "blocks", None) is None or getattr(shared_up, "blocks", None) is None or \
            getattr(shared_gate, "to_file", None) is not None or getattr(shared_up, "to_file", None) is not None:
        raise ValueError("the shared expert's layers as the file's blocks, inputs in the file's order")
    pairs = idx.numel()
    x2 = x.reshape(-1, gate.input_dims).contiguous()
    if x2.shape[0] != 1:
        return None
    g = torch.empty((pairs, gate.output_dims), dtype=x.dtype, device=x.device)
    u, h = torch.empty_like(g), torch.empty_like(g)
    sh = torch.empty((1, shared_gate.output_dims), dtype=x.dtype, device=x.device)
    sgu = (torch.empty_like(sh), torch.empty_like(sh)) if with_shared_gu else (None, None)
    idx = _idx32(idx)
    rc = _lib.library().strata_expert_gate_up_swiglu_shared(
        _lib.kind_id(gate.kind), gate.blocks.data_ptr(), up.blocks.data_ptr(), gate.num_experts, gate.output_dims,
        gate.input_dims, idx.data_ptr(), pairs, x2.data_ptr(), _lib.dtype_id(x.dtype), g.data_ptr(), u.data_ptr(),
        h.data_ptr(), _lib.kind_id(shared_gate.kind), shared_gate.blocks.data_ptr(), shared_up.blocks.data_ptr(),
        shared_gate.output_dims, sh.data_ptr(), _lib.ptr(sgu[0]), _lib.ptr(sgu[1]), _lib.stream())
    if rc in (_lib.ERR_SHAPE, _lib.ERR_DTYPE):
        return None
    _lib.check(rc, f"gate/up/swiglu with the shared expert {gate.kind} + {shared_gate.kind}")
    return (g, u, h, sh, *sgu) if with_shared_gu else (g, u, h, sh)


def moe_gate_up_swiglu_shared(gate: BlockSwitchLinear, up: BlockSwitchLinear, x: torch.Tensor, logits: torch.Tensor,
                              experts: int, k: int, shared_gate, shared_up):
    """gate_up_swiglu_shared at one token with the experts chosen in the launch from the router's float32 logits
    (1, rows >= experts: the experts' first, then rows such as the shared expert's gate), the choice top_k makes:
    (h (k, rows), idx (k,) int32, w (k,) float32 the softmax of the chosen logits, the shared expert's h (1, rows),
    the logits past the experts' as float16 (1, rows - experts) or None), or None where the launch does not take
    the case (then route_gated and gate_up_swiglu_shared). strata_mlx/fused.py:488-493 with blocks.py:969-975."""
    if (gate.kind, gate.output_dims, gate.input_dims, gate.num_experts) != (up.kind, up.output_dims, up.input_dims,
                                                                             up.num_experts):
        raise ValueError("gate and up differ in type or shape")
    if (shared_gate.kind, shared_gate.output_dims, shared_gate.input_dims) != (
            shared_up.kind, shared_up.output_dims, shared_up.input_dims) or shared_gate.input_dims != gate.input_dims:
        raise ValueError("the shared expert's gate and up differ in type or shape from each other or the token")
    if getattr(shared_gate, "blocks", None) is None or getattr(shared_up, "blocks", None) is None or \
            getattr(shared_gate, "to_file", None) is not None or getattr(shared_up, "to_file", None) is not None:
        raise ValueError("the shared expert's layers as the file's blocks, inputs in the file's order")
    x2 = x.reshape(-1, gate.input_dims).contiguous()
    lg = logits.reshape(-1).contiguous()
    if x2.shape[0] != 1 or lg.dtype != torch.float32 or lg.numel() < experts or experts != gate.num_experts:
        return None
    dev = x.device
    h = torch.empty((k, gate.output_dims), dtype=x.dtype, device=dev)
    idx = torch.empty(k, dtype=torch.int32, device=dev)
    w = torch.empty(k, dtype=torch.float32, device=dev)
    sh = torch.empty((1, shared_gate.output_dims), dtype=x.dtype, device=dev)
    nx = lg.numel() - experts
    extra = torch.empty((1, nx), dtype=torch.float16, device=dev) if nx > 0 else None
    rc = _lib.library().strata_moe_gate_up_swiglu_shared(
        _lib.kind_id(gate.kind), gate.blocks.data_ptr(), up.blocks.data_ptr(), gate.num_experts, gate.output_dims,
        gate.input_dims, lg.data_ptr(), lg.numel(), k, x2.data_ptr(), _lib.dtype_id(x.dtype), h.data_ptr(),
        idx.data_ptr(), w.data_ptr(), _lib.kind_id(shared_gate.kind), shared_gate.blocks.data_ptr(),
        shared_up.blocks.data_ptr(), shared_gate.output_dims, sh.data_ptr(), _lib.ptr(extra), _lib.stream())
    if rc in (_lib.ERR_SHAPE, _lib.ERR_DTYPE, _lib.ERR_KIND):
        return None
    _lib.check(rc, f"gate/up with the choice and the shared expert {gate.kind} + {shared_gate.kind}")
    return h, idx, w, sh, extra


def expert_matvec_shared(lin: BlockSwitchLinear, idx: torch.Tensor, shared):
    """The down call of one token's routed experts, out[pair] = W[idx[pair]] . x[pair] (x (pairs, in), each pair
    its own h), with a shared expert's down (a layer of the file's Q4_K blocks with `blocks`, `kind`,
    `output_dims`, `input_dims`: dense.BlockLinear) of its token shared_x (1, in) in the same launch: (out of
    the pairs, the shared expert's (1, shared rows)), called as f(x, shared_x). None where the launch does not
    take the case (other types, inputs other than 1536): the caller then makes the two calls apart. The routed
    and shared experts' down calls of strata_mlx/fused.py:492-493."""
    if getattr(shared, "blocks", None) is None or getattr(shared, "to_file", None) is not None:
        raise ValueError("the shared expert's layer as the file's blocks, inputs in the file's order")
    if shared.input_dims != lin.input_dims:
        raise ValueError("the shared expert's down takes the routed down's input width")

    def call(x: torch.Tensor, shared_x: torch.Tensor):
        pairs = idx.numel()
        x2 = x.reshape(-1, lin.input_dims).contiguous()
        s2 = shared_x.reshape(-1, shared.input_dims).contiguous()
        if x2.shape[0] != pairs or s2.shape[0] != 1 or s2.dtype != x2.dtype:
            return None
        out = torch.empty((pairs, lin.output_dims), dtype=x.dtype, device=x.device)
        s_out = torch.empty((1, shared.output_dims), dtype=x.dtype, device=x.device)
        ix = _idx32(idx)
        rc = _lib.library().strata_expert_matvec_shared(
            _lib.kind_id(lin.kind), lin.blocks.data_ptr(), lin.num_experts, lin.output_dims, lin.input_dims,
            ix.data_ptr(), pairs, x2.data_ptr(), _lib.dtype_id(x.dtype), out.data_ptr(), _lib.kind_id(shared.kind),
            shared.blocks.data_ptr(), shared.output_dims, s2.data_ptr(), s_out.data_ptr(), _lib.stream())
        if rc in (_lib.ERR_SHAPE, _lib.ERR_DTYPE, _lib.ERR_KIND):
            return None
        _lib.check(rc, f"down with the shared expert {lin.kind} + {shared.kind}")
        return out, s_out

    return call


LAYER_SPIN = 100000  # polls of memory (about a microsecond each) before a wait of expert_layer gives up
_layer_workspaces = {}


def _layer_workspace(device: torch.device, pairs: int, ffn: int) -> torch.Tensor:
    """The workspace of expert_layer for one device, stream and shape, zeroed when first made and kept."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream, pairs, ffn)
    ws = _layer_workspaces.get(key)
    if ws is None:
        size = _lib.library().strata_expert_layer_workspace(pairs, ffn)
        if size < 0:
            raise ValueError(f"expert_layer: {pairs} pairs of {ffn} rows not taken")
        ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _layer_workspaces[key] = ws
    return ws


def layer_status(device: torch.device | None = None) -> int:
    """The status bits that expert_layer's launches on `device` set since the last call (bit 0: a wait gave up and
    wrote NaN rows), cleared on return. Waits for the device."""
    status = 0
    for (index, _, _, _), ws in _layer_workspaces.items():
        if device is None or index == torch.device(device).index:
            word = ws[:4].view(torch.int32)
            status |= int(word.item())
            word.zero_()
    return status


def expert_layer(gate: BlockSwitchLinear, up: BlockSwitchLinear, down: BlockSwitchLinear, x: torch.Tensor,
                 idx: torch.Tensor, with_h: bool = False):
    """down(silu(gate . x) * (up . x)) for every pair of one token, in one launch: x (1, in) float16, idx (pairs,)
    -> (pairs, out), or (y, h) with h (pairs, ffn) if with_h. The same bits as gate_up_swiglu followed by
    expert_matvec on down. None where the launch does not take the case (other types or shapes, several tokens):
    the caller then makes those two calls. The per-pair path of strata_mlx/blocks.py:958-986 at one token."""
    if (gate.kind, gate.output_dims, gate.input_dims, gate.num_experts) != (up.kind, up.output_dims, up.input_dims,
                                                                             up.num_experts):
        raise ValueError("gate and up differ in type or shape")
    if (down.kind, down.num_experts, down.input_dims, down.output_dims) != (gate.kind, gate.num_experts,
                                                                             gate.output_dims, gate.input_dims):
        return None
    x2 = x.reshape(-1, gate.input_dims)
    pairs = idx.numel()
    if x2.shape[0] != 1 or x.dtype != torch.float16 or not 1 <= pairs <= 16:
        return None
    x2 = x2.contiguous()
    lib = _lib.library()
    if lib.strata_expert_layer_workspace(pairs, gate.output_dims) < 0:
        return None
    ws = _layer_workspace(x.device, pairs, gate.output_dims)
    y = torch.empty((pairs, down.output_dims), dtype=x.dtype, device=x.device)
    h = torch.empty((pairs, gate.output_dims), dtype=x.dtype, device=x.device) if with_h else None
    idx = _idx32(idx)
    rc = lib.strata_expert_layer(
        _lib.kind_id(gate.kind), gate.blocks.data_ptr(), up.blocks.data_ptr(), down.blocks.data_ptr(),
        gate.num_experts, gate.input_dims, gate.output_dims, idx.data_ptr(), pairs, x2.data_ptr(),
        _lib.dtype_id(x.dtype), _lib.ptr(h), y.data_ptr(), ws.data_ptr(), LAYER_SPIN, _lib.stream())
    if rc in (_lib.ERR_KIND, _lib.ERR_SHAPE):
        return None
    _lib.check(rc, f"expert layer {gate.kind}")
    return (y, h) if with_h else y


def expert_matvec(lin: BlockSwitchLinear, idx: torch.Tensor, x: torch.Tensor, share: int = 1) -> torch.Tensor:
    """out[pair] = W[idx[pair]] . x[pair / share]: x (pairs / share, in) -> (pairs, out)."""
    pairs = idx.numel()
    x2 = x.reshape(-1, lin.input_dims).contiguous()
    out = torch.empty((pairs, lin.output_dims), dtype=x.dtype, device=x.device)
    idx = _idx32(idx)
    _lib.check(_lib.library().strata_expert_matvec(
        _lib.kind_id(lin.kind), lin.blocks.data_ptr(), lin.num_experts, lin.output_dims, lin.input_dims,
        idx.data_ptr(), pairs, x2.data_ptr(), _lib.dtype_id(x.dtype), share, out.data_ptr(), _lib.stream()),
        f"matvec {lin.kind}")
    return out


def matvec_glu(lin: BlockSwitchLinear, idx: torch.Tensor, gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """`lin(swiglu(gate, up), idx)`, one pair to each row of gate and up: (pairs, out). The SwiGLU is rounded as
    mlx-lm rounds it. strata_mlx/blocks.py:939-955."""
    pairs = idx.numel()
    gate, up = gate.reshape(pairs, -1).contiguous(), up.reshape(pairs, -1).contiguous()
    out = torch.empty((pairs, lin.output_dims), dtype=gate.dtype, device=gate.device)
    idx = _idx32(idx)
    _lib.check(_lib.library().strata_expert_matvec_swiglu(
        _lib.kind_id(lin.kind), lin.blocks.data_ptr(), lin.num_experts, lin.output_dims, lin.input_dims,
        idx.data_ptr(), pairs, gate.data_ptr(), up.data_ptr(), _lib.dtype_id(gate.dtype), out.data_ptr(),
        _lib.stream()), f"matvec_glu {lin.kind}")
    return out


def matvec_separate(experts: list, kind: str, rows: int, cols: int, x: torch.Tensor, share: int) -> torch.Tensor:
    """out[pair] = W[pair] . x, every pair bringing its expert's blocks as a tensor of its own.
    x (pairs / share, cols). Returns (pairs, rows). strata_mlx/blocks.py:331-346."""
    n = len(experts)
    for e in experts:
        _flat_u8(e)
    ptrs = torch.tensor([e.data_ptr() for e in experts], dtype=torch.int64, device=x.device)
    x2 = x.reshape(-1, cols).contiguous()
    out = torch.empty((n, rows), dtype=x.dtype, device=x.device)
    _lib.check(_lib.library().strata_expert_matvec_ptrs(
        _lib.kind_id(kind), ptrs.data_ptr(), rows, cols, n, x2.data_ptr(), _lib.dtype_id(x.dtype), share,
        out.data_ptr(), _lib.stream()), f"matvec_separate {kind}")
    return out


def window_matvec(blocks: torch.Tensor, kind: str, rows: int, cols: int, x: torch.Tensor,
                  per_row: int | None = None, row_ids: torch.Tensor | None = None,
                  out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """out[t] = W . x[t] for one layer `blocks` of (rows, cols) and x (tokens, cols): (tokens, rows), or
    (tokens, len(row_ids)) over the listed rows only. strata_mlx/blocks.py:383-394."""
    _flat_u8(blocks)
    x2 = x.reshape(-1, cols).contiguous()
    tokens = x2.shape[0]
    n = rows if row_ids is None else row_ids.numel()
    out_dtype = out_dtype or x.dtype
    out = torch.empty((tokens, n), dtype=out_dtype, device=x.device)
    ids = None if row_ids is None else row_ids.reshape(-1).to(torch.int32).contiguous()
    _lib.check(_lib.library().strata_dense_matvec(
        _lib.kind_id(kind), blocks.data_ptr(), rows, cols, x2.data_ptr(), tokens, _lib.dtype_id(x.dtype),
        out.data_ptr(), _lib.dtype_id(out_dtype), _lib.ptr(ids), n if ids is not None else 0, _lib.stream()),
        f"window {kind}")
    return out


# ---- Q3_K held as planes (strata_mlx/blocks.py:397-512): the blocks rearranged once into aligned arrays of their
# parts (high-bit words, value words, decoded scales, d), 114 bytes a block where the file has 110.

Q3K_PLANE_BYTES = 114
PLANES_MAX_TOKENS = 8  # tokens a launch of the planes window kernel takes; more go 8 at a time
PLANES_MAX_X_BYTES = 48 * 1024  # and at most this much of their activations (staged in LDS)


def q3k_planes(blocks: torch.Tensor, rows: int, cols: int) -> dict:
    """A Q3_K tensor's blocks (rows, cols as the file has them) -> its planes, on the GPU. strata_mlx/blocks.py:403-414."""
    _flat_u8(blocks)
    if cols % 256 or blocks.numel() < rows * row_bytes("Q3_K", cols):
        raise ValueError(f"Q3_K planes: blocks of a ({rows}, {cols}) tensor")
    n = rows * cols // 256
    dev = blocks.device
    planes = {"hm": torch.empty(n * 8, dtype=torch.int32, device=dev),
              "qs": torch.empty(n * 16, dtype=torch.int32, device=dev),
              "sc": torch.empty(n * 16, dtype=torch.int8, device=dev),
              "dd": torch.empty(n, dtype=torch.float16, device=dev)}
    _lib.check(_lib.library().strata_q3k_planes(blocks.data_ptr(), rows, cols, planes["hm"].data_ptr(),
                                                planes["qs"].data_ptr(), planes["sc"].data_ptr(),
                                                planes["dd"].data_ptr(), _lib.stream()), "q3k_planes")
    return planes


def _planes_per_row(rows: int, cols: int) -> int:
    """Lanes a row by the tensor's shape, never by the window, so that a token gets the same bits alone as in a
    window (strata_mlx/blocks.py:484-490): here as many as a row has half blocks, up to 16, since a wave of 64
    lanes and 256 CUs want more lanes than the reference's rule (2 for 10,240 rows) gives."""
    per_row, halves = 1, 2 * cols // 256
    while per_row < 16 and per_row < halves:
        per_row *= 2
    return per_row


def q3k_planes_window(planes: dict, rows: int, cols: int, x: torch.Tensor) -> torch.Tensor:
    """out[t] = W . x[t] for a Q3_K tensor held as planes, x (tokens, cols). Returns (tokens, rows) in x's type.
    strata_mlx/blocks.py:482-501."""
    x = x.reshape(-1, cols).contiguous()
    tokens = x.shape[0]
    out = torch.empty((tokens, rows), dtype=x.dtype, device=x.device)
    per_row = _planes_per_row(rows, cols)
    step = max(1, min(PLANES_MAX_TOKENS, PLANES_MAX_X_BYTES // (cols * x.element_size())))
    for t0 in range(0, tokens, step):
        t1 = min(tokens, t0 + step)
        _lib.check(_lib.library().strata_q3k_planes_window(
            planes["hm"].data_ptr(), planes["qs"].data_ptr(), planes["sc"].data_ptr(), planes["dd"].data_ptr(),
            rows, cols, x[t0:t1].data_ptr(), t1 - t0, _lib.dtype_id(x.dtype), per_row, out[t0:t1].data_ptr(),
            _lib.stream()), "q3k_planes_window")
    return out


def q3k_planes_dequantize(planes: dict, rows: int, cols: int, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Every weight of a tensor held as planes, bit-exact (float32 / float16). strata_mlx/blocks.py:504-512."""
    if dtype not in (torch.float32, torch.float16):
        raise ValueError("q3k_planes_dequantize gives float32 or float16")
    out = torch.empty((rows, cols), dtype=dtype, device=planes["dd"].device)
    _lib.check(_lib.library().strata_q3k_planes_dequant(
        planes["hm"].data_ptr(), planes["qs"].data_ptr(), planes["sc"].data_ptr(), planes["dd"].data_ptr(), rows,
        cols, out.data_ptr(), _lib.dtype_id(dtype), _lib.stream()), "q3k_planes_dequantize")
    return out


# ---- Q2_0 from a table of sums (strata_mlx/blocks.py:697-928): two weights of a nibble make one of 16 sums of
# their two inputs; with those sums in a float16 table a code byte costs two table reads. float16 only.

LOOKUP_FROM = 1  # (token, expert) pairs from which Q2_0 experts over float16 go this way (blocks.py:711)
# switch_glu sends Q2_0 experts over float16 to the table of sums when True, as the reference's dispatch does
# (blocks.py:963-964); its sums are rounded to float16 (about 2e-3 relative L2 off the exact products at a decode
# layer's shape). By default they take the register-decode kernels instead: exact products and float32 sums (within
# 1e-3), and one launch fewer a layer.
LOOKUP_GLU = False
LOOKUP_MAX_COLS = 4096  # a token's table, 16 * cols bytes, is held in LDS


def _threads_per_row(runs: int) -> int:
    """Lanes the lookup kernels give a row: doubled while the row's runs still split evenly and every lane keeps
    four runs or more, at most 32 (the rule of strata_mlx/blocks.py:303-308, which fixes the summation order)."""
    p = 1
    while p < 32 and runs % (2 * p) == 0 and runs // (2 * p) >= 4:
        p *= 2
    return p


def _lookup_per_row(cols: int, pairs: int) -> int:
    """Lanes a row of lookup_matvec / lookup_gate_up: strata_mlx/blocks.py:797-803."""
    per_row = _threads_per_row(cols // 32)
    if cols >= 2048:
        per_row = min(per_row, 8 if pairs <= 40 else 2)
    elif pairs > 20:
        per_row = min(per_row, 4)
    return per_row


def lookable(lin, dtype: torch.dtype) -> bool:
    """strata_mlx/blocks.py:764-765, and rows whose table fits LDS."""
    return lin.kind == "Q2_0" and dtype == torch.float16 and lin.input_dims <= LOOKUP_MAX_COLS


def lookup_table(x: torch.Tensor) -> torch.Tensor:
    """The Q2_0 table of sums: for each token of x (n, cols) float16 and each pair of its inputs (a, b), the 16
    values (c & 3 - 1) a + (c >> 2 - 1) b, one for each nibble c of two 2-bit codes: (n, cols / 2, 16) float16.
    strata_mlx/blocks.py:768-777."""
    if x.dtype != torch.float16:
        raise ValueError("lookup_table takes float16 activations")
    _lib.require_device(x)
    n, cols = x.shape
    x = x.contiguous()
    table = torch.empty((n, cols // 2, 16), dtype=torch.float16, device=x.device)
    _lib.check(_lib.library().strata_q2_lookup_table(x.data_ptr(), n, cols, table.data_ptr(), _lib.stream()),
               "lookup_table")
    return table


def lookup_table_glu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """The table of silu(gate) * up, both (n, cols) float16. strata_mlx/blocks.py:780-789."""
    if gate.dtype != torch.float16 or up.dtype != torch.float16 or gate.shape != up.shape:
        raise ValueError("lookup_table_glu takes float16 gate and up of one shape")
    n, cols = gate.shape
    gate, up = gate.contiguous(), up.contiguous()
    table = torch.empty((n, cols // 2, 16), dtype=torch.float16, device=gate.device)
    _lib.check(_lib.library().strata_q2_lookup_table_glu(gate.data_ptr(), up.data_ptr(), n, cols, table.data_ptr(),
                                                         _lib.stream()), "lookup_table_glu")
    return table


def _lookup(lins: tuple, idx: torch.Tensor, table: torch.Tensor, share: int) -> tuple:
    lin = lins[0]
    if any(not lookable(l, torch.float16) for l in lins) or table.dtype != torch.float16:
        raise ValueError("the table path takes Q2_0 stacks of at most "
                         f"{LOOKUP_MAX_COLS} inputs and a float16 table")
    idx = _idx32(idx)
    pairs = idx.numel()
    outs = [torch.empty((pairs, lin.output_dims), dtype=torch.float16, device=table.device) for _ in lins]
    b = lins[1].blocks.data_ptr() if len(lins) > 1 else None
    ob = outs[1].data_ptr() if len(lins) > 1 else None
    _lib.check(_lib.library().strata_q2_lookup_matvec(
        lin.blocks.data_ptr(), b, lin.num_experts, lin.output_dims, lin.input_dims, idx.data_ptr(), pairs,
        table.contiguous().data_ptr(), share, _lookup_per_row(lin.input_dims, pairs), outs[0].data_ptr(), ob,
        _lib.stream()), "lookup_matvec")
    return tuple(outs)


def lookup_matvec(lin, idx: torch.Tensor, table: torch.Tensor, share: int) -> torch.Tensor:
    """The routed Q2_0 product read through a table of sums: row r of pair p is the sum, over the row's code
    nibbles, of the entries of token p / share's `lookup_table` that they select, times each block's d.
    (pairs, rows) float16. strata_mlx/blocks.py:792-812."""
    return _lookup((lin,), idx, table, share)[0]


def lookup_gate_up(gate, up, idx: torch.Tensor, table: torch.Tensor, share: int) -> tuple:
    """(`lookup_matvec(gate, ...)`, `lookup_matvec(up, ...)`) in one launch, the same bits; gate and up of one shape.
    strata_mlx/blocks.py:829-848."""
    if (gate.num_experts, gate.output_dims, gate.input_dims) != (up.num_experts, up.output_dims, up.input_dims):
        raise ValueError("lookup_gate_up takes gate and up of one shape")
    return _lookup((gate, up), idx, table, share)


def lookup_down_glu(lin, idx: torch.Tensor, gate: torch.Tensor, up: torch.Tensor):
    """`lookup_matvec(lin, idx, lookup_table_glu(gate, up), 1)` in one launch (the same bits), or None where a
    pair's table does not fit LDS. strata_mlx/blocks.py:889-914."""
    if not lookable(lin, gate.dtype) or up.dtype != torch.float16:
        return None
    idx = _idx32(idx)
    pairs = idx.numel()
    # lookup_matvec's lanes a row, so that the two give the same bits. The reference's own rule for down
    # (blocks.py:893-895) leaves out the rule for rows of 2048 inputs or more; below 2048, where down's rows are,
    # the two rules agree.
    per_row = _lookup_per_row(lin.input_dims, pairs)
    gate = gate.reshape(pairs, lin.input_dims).contiguous()
    up = up.reshape(pairs, lin.input_dims).contiguous()
    out = torch.empty((pairs, lin.output_dims), dtype=torch.float16, device=gate.device)
    _lib.check(_lib.library().strata_q2_lookup_down_glu(
        lin.blocks.data_ptr(), lin.num_experts, lin.output_dims, lin.input_dims, idx.data_ptr(), pairs,
        gate.data_ptr(), up.data_ptr(), per_row, out.data_ptr(), _lib.stream()), "lookup_down_glu")
    return out


def _lookup_glu(x: torch.Tensor, indices: torch.Tensor, up, gate, down) -> torch.Tensor:
    """strata_mlx/blocks.py:917-928: one table for gate and up, gate and up in one launch, down building the table
    of silu(gate) * up itself."""
    k = indices.shape[-1] if indices.ndim else 1
    idx = _idx32(indices)
    table = lookup_table(x.reshape(-1, x.shape[-1]))
    if (gate.output_dims, gate.input_dims, gate.num_experts) == (up.output_dims, up.input_dims, up.num_experts):
        g, u = lookup_gate_up(gate, up, idx, table, k)
    else:
        g, u = lookup_matvec(gate, idx, table, k), lookup_matvec(up, idx, table, k)
    out = lookup_down_glu(down, idx, g, u)
    if out is None:
        out = lookup_matvec(down, idx, lookup_table_glu(g, u), 1)
    return out.reshape(*indices.shape, down.output_dims)


def switch_glu(x: torch.Tensor, indices: torch.Tensor, up: BlockSwitchLinear, gate: BlockSwitchLinear,
               down: BlockSwitchLinear) -> torch.Tensor:
    """down(silu(gate(x)) * up(x)) through each token's experts: x (..., in), indices (..., k) -> (..., k, out).
    The argument order is the reference's (x, indices, up, gate, down); strata_mlx/blocks.py:958-986.

    Decode windows take the matvec kernels: gate and up in one launch reading x once and writing silu(gate) * up
    (rounded as mlx-lm rounds it), then down on that; Q2_0 stacks over float16 too, unless LOOKUP_GLU sends them to
    the table of sums as the reference's dispatch does (blocks.py:963-964). Prompt chunks (from TILES_FROM pairs) take
    the tiles: the pairs sorted by expert on the GPU, gate and up with the SwiGLU in one MFMA launch, down written
    straight to the pairs."""
    indices = torch.as_tensor(indices, device=x.device)
    k = indices.shape[-1] if indices.ndim else 1
    flat = indices.reshape(-1)
    xs = x.reshape(-1, x.shape[-1])
    if flat.numel() >= TILES_FROM and all(tileable(lin.kind, lin.output_dims, lin.input_dims)
                                          for lin in (up, gate, down)):
        return _tiled_glu(x, indices, up, gate, down)
    if LOOKUP_GLU and flat.numel() >= LOOKUP_FROM and all(lookable(lin, x.dtype) for lin in (up, gate, down)):
        return _lookup_glu(x, indices, up, gate, down)
    if (gate.kind, gate.output_dims, gate.input_dims, gate.num_experts) == (up.kind, up.output_dims, up.input_dims,
                                                                             up.num_experts):
        _, _, h = gate_up_swiglu(gate, up, xs, flat, k)
        return expert_matvec(down, flat, h).reshape(*indices.shape, down.output_dims)
    else:
        g = gate(xs.reshape(-1, 1, 1, xs.shape[-1]).expand(-1, 1, 1, -1), indices.reshape(-1, k)).reshape(flat.numel(), -1)
        u = up(xs.reshape(-1, 1, 1, xs.shape[-1]).expand(-1, 1, 1, -1), indices.reshape(-1, k)).reshape(flat.numel(), -1)
    out = matvec_glu(down, flat, g, u)
    return out.reshape(*indices.shape, down.output_dims)


class BlockSwitchGLU:
    """gate, up and down of one layer's expert stacks behind mlx-lm's `SwitchGLU` call (x, indices) -> y, which
    `switch_glu` computes; strata_mlx/blocks.py:989-996."""

    def __init__(self, gate: BlockSwitchLinear, up: BlockSwitchLinear, down: BlockSwitchLinear):
        self.gate_proj, self.up_proj, self.down_proj = gate, up, down

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        return switch_glu(x, indices, self.up_proj, self.gate_proj, self.down_proj)


ROWS_TILE, COLS_TILE = 64, 64  # what a tile takes (strata_mlx/blocks.py:581, 629-631)


def tileable(kind: str, rows: int, cols: int) -> bool:
    """True when rows and cols are whole 64 x 64 tiles, cols whole blocks of the type, and the type has a decoder
    here: the stacks `tile_matmul` multiplies (strata_mlx/blocks.py:629-631)."""
    per_block = {**BLOCK, **DENSE}[kind][0]
    return rows % ROWS_TILE == 0 and cols % COLS_TILE == 0 and cols % per_block == 0 and kind not in NO_GRID


def _route(indices: torch.Tensor, experts: int) -> tuple:
    """tiles_of's layout and the pair of each slot (slot_pair, -1 for an empty slot), all int32 on the GPU."""
    k = indices.shape[-1] if indices.ndim else 1
    flat = _idx32(indices)
    pairs = flat.numel()
    lib = _lib.library()
    n_tiles = lib.strata_route_tiles_max(pairs, experts, TOKENS_TILE)
    dev = indices.device
    tile_expert = torch.empty(n_tiles, dtype=torch.int32, device=dev)
    token = torch.empty(n_tiles * TOKENS_TILE, dtype=torch.int32, device=dev)
    slot_pair = torch.empty(n_tiles * TOKENS_TILE, dtype=torch.int32, device=dev)
    where = torch.empty(pairs, dtype=torch.int32, device=dev)
    ws = torch.empty(max(1, lib.strata_route_tiles_workspace(pairs, experts)), dtype=torch.uint8, device=dev)
    _lib.check(lib.strata_route_tiles(flat.data_ptr(), pairs, k, experts, TOKENS_TILE, tile_expert.data_ptr(),
                                      token.data_ptr(), where.data_ptr(), slot_pair.data_ptr(), ws.data_ptr(),
                                      _lib.stream()), "tiles_of")
    return tile_expert, token, where, slot_pair, flat


def tiles_of(indices: torch.Tensor, experts: int) -> tuple:
    """Groups a prompt's (token, expert) pairs by expert into tiles of TOKENS_TILE slots, on the GPU and without
    waiting for it. Returns three int32 arrays: tile -> expert (`experts` marks an unused tile), slot -> token, and
    pair -> slot. The tile count, P // 16 + min(E, P), is fixed by the pair count alone, so no routing can overflow
    it. Within an expert, slots follow the pairs' order. strata_mlx/blocks.py:657-681."""
    return _route(indices, experts)[:3]


def rows_to_f16(a: torch.Tensor) -> tuple:
    """Rows of 16-bit (or float32) activations scaled into float16 by a power of two each, so that each row's
    largest magnitude lands in [2^14, 2^15): (the float16 rows, each row's largest magnitude as int32 float bits).
    Exact for every value within 2^31 of its row's largest; the MFMA kernels scale their sums back."""
    a = a.reshape(-1, a.shape[-1]).contiguous()
    _lib.require_device(a)
    rows, cols = a.shape
    out = torch.empty((rows, cols), dtype=torch.float16, device=a.device)
    row_max = torch.empty(rows, dtype=torch.int32, device=a.device)
    _lib.check(_lib.library().strata_rows_to_f16(a.data_ptr(), rows, cols, _lib.dtype_id(a.dtype), out.data_ptr(),
                                                 row_max.data_ptr(), _lib.stream()), "rows_to_f16")
    return out, row_max


def rows_from_f32(c: torch.Tensor, row_max: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Products of rows scaled by rows_to_f16 (c float32 (rows, cols), row_max its second output) scaled back by
    each row's power of two and rounded once to `dtype`."""
    c = c.contiguous()
    _lib.require_device(c)
    rows, cols = c.shape
    out = torch.empty((rows, cols), dtype=dtype, device=c.device)
    for r0 in range(0, rows, 65535):  # the launch takes 65535 rows at a time
        n = min(65535, rows - r0)
        _lib.check(_lib.library().strata_rows_from_f32(c[r0:].data_ptr(), n, cols, row_max[r0:].data_ptr(),
                                                       _lib.dtype_id(dtype), out[r0:].data_ptr(), _lib.stream()),
                   "rows_from_f32")
    return out


def tile_matmul(blocks: torch.Tensor, kind: str, shape: tuple, a: torch.Tensor, tile_expert: torch.Tensor,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """The grouped product of a prompt's tiles on MFMA: row p of the result is W[e] . a[p], e the expert that p's
    tile belongs to, W the (experts, rows, cols) stack in `blocks`.

    a has P rows of cols activations, P a whole number of tiles; tile_expert holds one expert per tile. A tile whose
    entry is experts or more is skipped, and its rows of the result keep what the buffer held (`out`, when given). float16 activations multiply weights as float16 (exact for IQ3_S / IQ3_XXS /
    Q2_0 rows of whole 256-weight steps: integer codes times the run's own scale, with d on the float32 sums;
    rounded to float16 for the other types); bfloat16 rows are first scaled into float16 by a power of two each
    (rows_to_f16) and the sums scaled back, so they multiply exactly too; float32 activations multiply exact
    weights in float32. Sums are float32. Returns (P, rows) float32. strata_mlx/blocks.py:634-654."""
    experts, rows, cols = shape
    _flat_u8(blocks)
    a = a.contiguous()
    p = a.shape[0]
    if p % TOKENS_TILE:
        raise ValueError(f"{p} rows of activations are not whole tiles of {TOKENS_TILE}")
    te = tile_expert.reshape(-1).to(torch.int32).contiguous()
    if te.numel() * TOKENS_TILE != p:
        raise ValueError("one expert to every tile of activations")
    a_max = None
    if a.dtype == torch.bfloat16:
        a, a_max = rows_to_f16(a)
    if out is None:
        out = torch.empty((p, rows), dtype=torch.float32, device=a.device)
    _lib.check(_lib.library().strata_grouped_matmul(
        _lib.kind_id(kind), blocks.data_ptr(), experts, rows, cols, a.data_ptr(), _lib.dtype_id(a.dtype),
        _lib.ptr(a_max), te.data_ptr(), te.numel(), TOKENS_TILE, out.data_ptr(), _lib.stream()), f"tile_matmul {kind}")
    return out


PROMPT_KINDS = ("IQ3_S", "IQ3_XXS", "Q2_0")  # the kinds of the fused prompt kernels (rows of whole 256-weight steps)


def _prompt_fused(lin, dtype: torch.dtype) -> bool:
    return lin.kind in PROMPT_KINDS and lin.input_dims % 256 == 0 and dtype in (torch.float16, torch.bfloat16)


def _tiled_glu(x: torch.Tensor, indices: torch.Tensor, up, gate, down) -> torch.Tensor:
    """The three products of a prompt's pairs through the tiles (strata_mlx/blocks.py:684-694): the pairs sorted by
    expert on the GPU, gate and up in one launch with the SwiGLU (float32 products, rounded once to the activations'
    type) written in slot order, and down written straight to the pairs. bfloat16 rows go to the float16 MFMA
    scaled by a power of two each (rows_to_f16). Types the fused kernels do not take, and float32, go through
    tile_matmul and the reference's steps."""
    tiles, token, where, slot_pair, flat = _route(indices, gate.num_experts)
    xs = x.reshape(-1, x.shape[-1]).contiguous()
    lib = _lib.library()
    n_slots = token.numel()
    same = (gate.kind, gate.output_dims, gate.input_dims, gate.num_experts) == (up.kind, up.output_dims,
                                                                                 up.input_dims, up.num_experts)
    if same and _prompt_fused(gate, x.dtype):
        x16, x_max = rows_to_f16(xs) if x.dtype == torch.bfloat16 else (xs, None)
        h = torch.empty((n_slots, gate.output_dims), dtype=x.dtype, device=x.device)
        _lib.check(lib.strata_prompt_gate_up_swiglu(
            _lib.kind_id(gate.kind), gate.blocks.data_ptr(), up.blocks.data_ptr(), gate.num_experts, gate.output_dims,
            gate.input_dims, x16.data_ptr(), _lib.ptr(x_max), token.data_ptr(), tiles.data_ptr(), tiles.numel(),
            TOKENS_TILE, h.data_ptr(), _lib.dtype_id(x.dtype), _lib.stream()), f"prompt gate/up {gate.kind}")
    else:
        a = xs[token.long()]

        def product(lin):
            return tile_matmul(lin.blocks, lin.kind, (lin.num_experts, lin.output_dims, lin.input_dims), a, tiles)

        h = (torch.nn.functional.silu(product(gate)) * product(up)).to(x.dtype)
    if _prompt_fused(down, x.dtype):
        h16, h_max = rows_to_f16(h) if x.dtype == torch.bfloat16 else (h, None)
        y = torch.empty((flat.numel(), down.output_dims), dtype=x.dtype, device=x.device)
        _lib.check(lib.strata_prompt_down(
            _lib.kind_id(down.kind), down.blocks.data_ptr(), down.num_experts, down.output_dims, down.input_dims,
            h16.data_ptr(), _lib.ptr(h_max), tiles.data_ptr(), tiles.numel(), TOKENS_TILE, slot_pair.data_ptr(),
            flat.data_ptr(), flat.numel(), y.data_ptr(), _lib.dtype_id(x.dtype), _lib.stream()), f"prompt down {down.kind}")
    else:
        c = tile_matmul(down.blocks, down.kind, (down.num_experts, down.output_dims, down.input_dims), h, tiles)
        y = c[where.long().clamp(min=0)].to(x.dtype)
        y = torch.where((where >= 0)[:, None], y, torch.full_like(y, float("nan")))  # a pair naming no expert
    return y.reshape(*indices.shape, down.output_dims)
