"""Dense layers on the file's blocks: the call surface of strata_mlx/dense.py, over `strata_dense_matvec`.

    ScaledLinear   a Q6_K layer given as the reference holds it (codes, scales, d; dense.py:109-167). The parts
                   are packed back into the file's Q6_K blocks once, on the GPU, and every product reads those
                   210-byte blocks (6.56 bits a weight, where the parts take 8.56).
    BlockLinear    a layer kept as the file's blocks, any type the kernels decode (dense.py:205-242); `inputs`
                   reorders the activations as the reference's does. Q3_K layers are held as planes
                   (blocks.q3k_planes), as the reference holds them.
    BlockEmbedding rows of an embedding decoded when their tokens come (dense.py:245-258).

Up to MAX_TOKENS tokens a product is a window of the matvec kernel (each block decoded once for every token). A
longer chunk (a prompt's) of float16 or bfloat16 tokens is multiplied as the reference multiplies it
(dense.py:234-241): the layer dequantized for the chunk (strata_dequantize, each weight exact in float32 and
rounded once to float16) and let go, then a library product with float32 sums (torch.mm; 4-6 times the tile
kernels' speed at 2048 tokens). bfloat16 tokens are scaled into float16 rows by a power of two each, exactly, and
the sums scaled back. float32 tokens go through the tile kernels as a stack of one matrix (exact weights on MFMA).
"""

import torch

from . import blocks as B

MAX_TOKENS = 8  # more than a window: a chunk of a prompt, multiplied as floats (dense.py:33)
# Q3_K layers held as planes (blocks.q3k_planes), as the reference holds them (dense.py:190, 214-215), when True;
# by default they stay the file's blocks, which the register decode reads at twice the planes window's speed
PLANES = False


def q6k_blocks(codes: torch.Tensor, scales: torch.Tensor, d: torch.Tensor) -> torch.Tensor:
    """The Q6_K blocks (rows * cols / 256 * 210 bytes, uint8) whose parts are `codes` int8 (rows, cols) in
    [-32, 31], `scales` int8 (rows, cols / 16) and `d` float16 (rows, cols / 256): the inverse of q6k_parts
    (strata_mlx/gguf.py:150-165). In a block, weight 128h + 32r + i has its low four bits in ql[64h + i] (r = 0,
    2: low / high nibble) or ql[64h + 32 + i] (r = 1, 3), its high two in bits 2r of qh[32h + i]."""
    rows, cols = codes.shape
    if cols % 256 or scales.shape != (rows, cols // 16) or d.shape != (rows, cols // 256):
        raise ValueError(f"Q6_K parts of a ({rows}, {cols}) layer must be codes (rows, cols), scales "
                         f"(rows, cols/16), d (rows, cols/256)")
    nb = cols // 256
    q = (codes.to(torch.int16) + 32).to(torch.uint8).reshape(rows, nb, 2, 4, 32)
    lo, hi = q & 15, q >> 4
    ql = torch.cat([lo[:, :, :, 0] | (lo[:, :, :, 2] << 4), lo[:, :, :, 1] | (lo[:, :, :, 3] << 4)], dim=3)
    qh = hi[:, :, :, 0] | (hi[:, :, :, 1] << 2) | (hi[:, :, :, 2] << 4) | (hi[:, :, :, 3] << 6)
    sc = scales.contiguous().view(torch.uint8).reshape(rows, nb, 16)
    dd = d.to(torch.float16).contiguous().view(torch.uint8).reshape(rows, nb, 2)
    return torch.cat([ql.reshape(rows, nb, 128), qh.reshape(rows, nb, 64), sc, dd], dim=2).reshape(-1)


class BlockLinear:
    """A dense projection (attention, a shared expert, lm_head) whose weight rows stay GGUF blocks on the GPU, one
    row per output, with nn.Linear's call (x (..., in) -> (..., out)). When the file stores the inputs in another
    order, `inputs` gives each input's column in the file's row, and x is permuted to match before the product.
    strata_mlx/dense.py:205-242."""

    def __init__(self, blocks: torch.Tensor, kind: str, shape: tuple, inputs=None):
        self.blocks, self.kind = B._flat_u8(blocks), kind
        self.output_dims, self.input_dims = shape
        if blocks.numel() < self.output_dims * B.row_bytes(kind, self.input_dims):
            raise ValueError("blocks hold fewer bytes than the shape needs")
        self.to_file = None
        if inputs is not None:
            self.to_file = torch.argsort(torch.as_tensor(inputs, device=blocks.device)).to(torch.int64)
        self.planes = None
        if kind == "Q3_K" and PLANES:  # held as planes instead: aligned words for the window kernel
            self.planes, self.blocks = B.q3k_planes(blocks, *shape), None

    @property
    def nbytes(self) -> int:
        if self.planes is not None:
            return sum(a.numel() * a.element_size() for a in self.planes.values())
        return self.blocks.numel()

    def floats(self, dtype: torch.dtype) -> torch.Tensor:
        """The weights (out, in), each exact in float32 and rounded once to `dtype`."""
        half = torch.float16 if dtype == torch.float16 else torch.float32
        if self.planes is not None:
            w = B.q3k_planes_dequantize(self.planes, self.output_dims, self.input_dims, half)
        else:
            w = B.dequantize(self.blocks, self.kind, (self.output_dims, self.input_dims), half)
        return w if w.dtype == dtype else w.to(dtype)

    def __call__(self, x: torch.Tensor, row_ids: torch.Tensor | None = None) -> torch.Tensor:
        rows, cols = self.output_dims, self.input_dims
        lead = x.shape[:-1]
        x2 = x.reshape(-1, cols)
        if self.to_file is not None:
            x2 = x2[:, self.to_file]
        tokens = x2.shape[0]
        if self.planes is not None:
            if tokens <= MAX_TOKENS:
                out = B.q3k_planes_window(self.planes, rows, cols, x2)
            else:
                out = x2 @ self.floats(x.dtype).T
            if row_ids is not None:
                out = out[:, row_ids.reshape(-1).long()]
        elif tokens <= MAX_TOKENS or row_ids is not None:
            out = B.window_matvec(self.blocks, self.kind, rows, cols, x2, row_ids=row_ids)
        elif x2.dtype in (torch.float16, torch.bfloat16):
            out = float16_chunk(self.floats(torch.float16), x2)
        elif B.tileable(self.kind, rows, cols):
            out = tiled_chunk(self.blocks, self.kind, rows, cols, x2)
        else:
            out = x2 @ self.floats(x.dtype).T
        return out.reshape(*lead, out.shape[-1])


def float16_chunk(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """x (tokens, cols) float16 or bfloat16 times float16 weights w (rows, cols), as the reference multiplies a
    prompt chunk (dense.py:234-241: the weights unpacked for the chunk, then a library product): float32 sums,
    (tokens, rows) in x's type. bfloat16 rows are scaled into float16 by a power of two each (rows_to_f16: exact),
    and the sums scaled back."""
    if x.dtype == torch.float16:
        return torch.mm(x, w.t())  # float32 sums, rounded once to float16
    x16, x_max = B.rows_to_f16(x)
    return B.rows_from_f32(torch.mm(x16, w.t(), out_dtype=torch.float32), x_max, x.dtype)


def tiled_chunk(blocks: torch.Tensor, kind: str, rows: int, cols: int, x: torch.Tensor) -> torch.Tensor:
    """out[t] = W . x[t] for a chunk of tokens x (tokens, cols) through the tile kernels, W one matrix of blocks:
    (tokens, rows) in x's type, float32 sums."""
    tokens = x.shape[0]
    tiles = (tokens + B.TOKENS_TILE - 1) // B.TOKENS_TILE
    a = x
    if tiles * B.TOKENS_TILE != tokens:  # the last tile's empty slots multiply zeros
        a = torch.zeros((tiles * B.TOKENS_TILE, cols), dtype=x.dtype, device=x.device)
        a[:tokens] = x
    te = torch.zeros(tiles, dtype=torch.int32, device=x.device)
    c = B.tile_matmul(blocks, kind, (1, rows, cols), a, te)
    return c[:tokens].to(x.dtype)


class FusedLinear(BlockLinear):
    """Several layers of one block type that read the same input (q, k and v; a shared expert's gate and up) kept
    as one matrix: their rows one after another, so a token's products are one launch (one kernel's fixed cost
    in place of one a layer). Called like the layers it fuses, it returns their outputs in order. No counterpart in
    the reference, whose engine calls the layers one by one (dense.py:109-167, 205-242); the products are the
    layers' own."""

    def __init__(self, layers):
        layers = list(layers)
        first = layers[0]
        if any(l.kind != first.kind or l.input_dims != first.input_dims or l.to_file is not None or l.planes is not None
               for l in layers):
            raise ValueError("fused layers share one block type and input width, as the file's blocks")
        self.sizes = [l.output_dims for l in layers]
        rb = B.row_bytes(first.kind, first.input_dims)
        blocks = torch.cat([l.blocks[:l.output_dims * rb] for l in layers])
        super().__init__(blocks, first.kind, (sum(self.sizes), first.input_dims))

    def __call__(self, x: torch.Tensor, row_ids=None):
        if row_ids is not None:
            raise ValueError("a fused layer takes every row")
        return tuple(torch.split(super().__call__(x), self.sizes, dim=-1))


def gate_up_swiglu(gate: BlockLinear, up: BlockLinear, x: torch.Tensor) -> tuple:
    """A dense (shared) expert's gate and up at the same tokens, with silu(gate) * up rounded as mlx-lm rounds it,
    in one launch: (gate . x, up . x, h), each (tokens, rows). The layers are read as one-expert stacks."""
    if (gate.kind, gate.output_dims, gate.input_dims) != (up.kind, up.output_dims, up.input_dims):
        raise ValueError("gate and up differ in type or shape")
    if gate.blocks is None or up.blocks is None or gate.to_file is not None or up.to_file is not None:
        raise ValueError("gate_up_swiglu takes layers kept as the file's blocks, inputs in the file's order")
    shape = (1, gate.output_dims, gate.input_dims)
    g = B.BlockSwitchLinear(gate.blocks, gate.kind, shape)
    u = B.BlockSwitchLinear(up.blocks, up.kind, shape)
    x2 = x.reshape(-1, gate.input_dims)
    idx = torch.zeros(x2.shape[0], dtype=torch.int32, device=x.device)
    return B.gate_up_swiglu(g, u, x2, idx, 1)


class ScaledLinear(BlockLinear):
    """A Q6_K layer given as codes, scales and d (strata_mlx/dense.py:109-167), kept as the file's Q6_K blocks.
    d_step (weights to a d) must be 256: layers whose inputs were reordered are BlockLinear with `inputs`."""

    def __init__(self, codes: torch.Tensor, scales: torch.Tensor, d: torch.Tensor):
        rows, cols = codes.shape
        if d.shape[1] * 256 != cols:
            raise ValueError(f"a d to every {cols // max(1, d.shape[1])} weights: only 256 (the file's blocks)")
        super().__init__(q6k_blocks(codes, scales, d), "Q6_K", (rows, cols))

    @classmethod
    def from_blocks(cls, blocks: torch.Tensor, shape: tuple) -> "ScaledLinear":
        """A layer straight from the file's Q6_K bytes."""
        self = cls.__new__(cls)
        BlockLinear.__init__(self, blocks, "Q6_K", shape)
        return self


class BlockEmbedding:
    """Token embeddings left as GGUF blocks on the GPU: looking tokens up decodes just their rows, so the table is
    never expanded to floats. strata_mlx/dense.py:245-258."""

    def __init__(self, blocks: torch.Tensor, kind: str, shape: tuple, dtype: torch.dtype):
        self.num_embeddings, self.dims = shape
        self.kind, self.dtype = kind, dtype
        self.rows = B._flat_u8(blocks).reshape(self.num_embeddings, -1)

    @property
    def nbytes(self) -> int:
        return self.rows.numel()

    def __call__(self, ids: torch.Tensor) -> torch.Tensor:
        ids = torch.as_tensor(ids, device=self.rows.device)
        taken = self.rows.index_select(0, ids.reshape(-1).to(torch.int64)).reshape(-1)
        dt = torch.float16 if self.dtype == torch.float16 else torch.float32
        out = B.dequantize(taken, self.kind, (ids.numel(), 1, self.dims), dt)
        return out.to(self.dtype).reshape(*ids.shape, self.dims)
