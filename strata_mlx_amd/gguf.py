"""GGUF files straight to the kernels: the reader of strata_mlx/gguf.py:63-133 and the block uploads of
strata_mlx/load.py:235-273, with torch tensors in HBM in place of mx.array.

A GGUF file (versions 2 and 3; little-endian) is

    "GGUF"  u32 version  u64 n_tensors  u64 n_kv
    n_kv x       (string key, u32 value type, value)
    n_tensors x  (string name, u32 n_dims, u64 dims[n_dims] (fastest axis first), u32 type, u64 offset)
    padding to `general.alignment` (32 when absent), then the data; each tensor at data + offset

with a string as u64 length + UTF-8 bytes and an array as (u32 element type, u64 count, elements). A tensor's
`shape` here is numpy order (the dims reversed), so an expert stack reads (experts, rows, cols) and row r of
expert e starts at byte (e * rows + r) * row_bytes of its data: the layout every kernel of this package takes.

The reader maps the file and holds each tensor as a numpy view of its bytes (nothing is read until used);
`upload` copies those bytes to the GPU unchanged, through pinned staging buffers, so an expert stack is in HBM
in the file's own blocks without a conversion. `experts`, `linear` and `embedding` then wrap them in the layers
of blocks.py / dense.py.
"""

import mmap
import re
import struct
from dataclasses import dataclass

import numpy as np
import torch

from . import blocks as B
from . import dense as D

# GGUF type id -> (name, weights per block, bytes per block); strata_mlx/gguf.py:25-33
TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 30: ("BF16", 1, 2),
    2: ("Q4_0", 32, 18), 6: ("Q5_0", 32, 22), 8: ("Q8_0", 32, 34),
    11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210),
    20: ("IQ4_NL", 32, 18), 23: ("IQ4_XS", 256, 136), 42: ("Q2_0", 64, 18),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 21: ("IQ3_S", 256, 110),
    22: ("IQ2_S", 256, 82), 29: ("IQ1_M", 256, 56),
}
FLOAT_TYPES = ("F32", "F16", "BF16")

# metadata value types: id -> struct code (8 string and 9 array are read by hand)
_SCALARS = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}
_STRING, _ARRAY = 8, 9
_NUMPY = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 10: "<u8", 11: "<i8", 12: "<f8"}
DEFAULT_ALIGNMENT = 32

STAGE_BYTES = 64 << 20  # bytes of each of the two pinned buffers an upload streams through


@dataclass
class Tensor:
    """A tensor of the file: its bytes as a read-only uint8 view into the mapped file (strata_mlx/gguf.py:38-50)."""

    name: str
    shape: tuple  # numpy order: the last axis is the one a row runs along
    type: str
    data: np.ndarray  # the raw bytes, a view into the file
    path: str = ""  # the file, and where in it the bytes start
    offset: int = 0

    @property
    def quantized(self) -> bool:
        return self.type not in FLOAT_TYPES

    @property
    def nbytes(self) -> int:
        return int(self.data.size)


def tensor_bytes(type_id: int, shape: tuple) -> int:
    """Bytes of a tensor of `shape` (numpy order) in type `type_id`; its rows must end on a block."""
    name, per_block, block_bytes = TYPES[type_id]
    cols = shape[-1] if shape else 1
    if cols % per_block:
        raise ValueError(f"{name}: rows of {cols} weights do not end on a block of {per_block}")
    n = 1
    for v in shape:
        n *= int(v)
    return n // per_block * block_bytes


class _Cursor:
    """Reads little-endian fields from a buffer, raising ValueError past its end."""

    def __init__(self, buf, path: str):
        self.buf, self.pos, self.path, self.size = buf, 0, path, len(buf)

    def take(self, n: int) -> int:
        at = self.pos
        if n < 0 or at + n > self.size:
            raise ValueError(f"{self.path}: truncated GGUF header (needs byte {at + n}, file has {self.size})")
        self.pos = at + n
        return at

    def scalar(self, code: str):
        at = self.take(struct.calcsize("<" + code))
        return struct.unpack_from("<" + code, self.buf, at)[0]

    def string(self) -> str:
        n = self.scalar("Q")
        at = self.take(n)
        return bytes(self.buf[at : at + n]).decode("utf-8", "replace")

    def value(self, vtype: int):
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            etype, count = self.scalar("I"), self.scalar("Q")
            if etype in _NUMPY:  # arrays of numbers in one read
                width = np.dtype(_NUMPY[etype]).itemsize
                at = self.take(count * width)
                return np.frombuffer(self.buf, dtype=_NUMPY[etype], count=count, offset=at).tolist()
            return [self.value(etype) for _ in range(count)]
        if vtype not in _SCALARS:
            raise ValueError(f"{self.path}: GGUF metadata value type {vtype} is not defined")
        return self.scalar(_SCALARS[vtype])


class GGUF:
    """A GGUF file, mapped: `meta` (key -> value) and `tensors` (name -> Tensor). strata_mlx/gguf.py:63-125.

    A malformed file (wrong magic, a version before 2, a header past the end, a tensor type not in TYPES, a row
    that does not end on a block, a tensor past the end of the file) raises ValueError."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        try:
            self._map = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError:  # an empty file cannot be mapped
            self._f.close()
            raise ValueError(f"{path} is not a GGUF file (empty)")
        cur = _Cursor(self._map, path)
        if len(self._map) < 4 or bytes(self._map[:4]) != b"GGUF":
            raise ValueError(f"{path} is not a GGUF file")
        cur.take(4)
        self.version = cur.scalar("I")
        if self.version < 2:
            raise ValueError(f"{path}: GGUF version {self.version} (32-bit counts) is not read; versions 2 and 3 are")
        n_tensors, n_kv = cur.scalar("Q"), cur.scalar("Q")
        self.meta = {}
        for _ in range(n_kv):
            key = cur.string()
            self.meta[key] = cur.value(cur.scalar("I"))
        infos = []
        for _ in range(n_tensors):
            name = cur.string()
            n_dims = cur.scalar("I")
            dims = [cur.scalar("Q") for _ in range(n_dims)]
            type_id, offset = cur.scalar("I"), cur.scalar("Q")
            infos.append((name, tuple(reversed(dims)), type_id, offset))
        self.alignment = int(self.meta.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0:
            raise ValueError(f"{path}: alignment {self.alignment}")
        self.data_start = (cur.pos + self.alignment - 1) // self.alignment * self.alignment
        raw = np.frombuffer(self._map, dtype=np.uint8)
        self.tensors = {}
        for name, shape, type_id, offset in infos:
            if type_id not in TYPES:
                raise ValueError(f"{name}: GGUF tensor type {type_id} is not supported")
            start = self.data_start + offset
            n = tensor_bytes(type_id, shape)
            if start + n > raw.size:
                raise ValueError(f"{name}: bytes {start}..{start + n} lie past the end of {path} ({raw.size})")
            self.tensors[name] = Tensor(name, shape, TYPES[type_id][0], raw[start : start + n], path, start)

    def __getitem__(self, name: str) -> Tensor:
        return self.tensors[name]

    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def __iter__(self):
        return iter(self.tensors.values())


_SPLIT = re.compile(r"-(\d{5})-of-(\d{5})\.gguf$")


def shards(path: str) -> list:
    """A model's files: the one named and, where its name says it is one of several (`-00001-of-00003.gguf`),
    the others beside it. strata_mlx/gguf.py:128-133."""
    m = _SPLIT.search(path)
    count = int(m.group(2)) if m else 1
    return [GGUF(path)] + [GGUF(_SPLIT.sub(f"-{i:05d}-of-{m.group(2)}.gguf", path)) for i in range(2, count + 1)]


def upload(t: Tensor, device, stage_bytes: int = STAGE_BYTES) -> torch.Tensor:
    """The tensor's bytes in device memory, unchanged (uint8, flat), as strata_mlx/load.py:263 hands the file's
    blocks to the GPU. Chunks of the mapped file go through two pinned buffers, the copy of one chunk to the GPU
    overlapping the read of the next from the file; returns when the bytes are on the device."""
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("upload copies to a GPU")
    n = t.nbytes
    out = torch.empty(n, dtype=torch.uint8, device=device)
    if n == 0:
        return out
    chunk = max(1, min(stage_bytes, n))
    stages = [torch.empty(chunk, dtype=torch.uint8, pin_memory=True) for _ in range(1 if n <= chunk else 2)]
    views = [s.numpy() for s in stages]
    done = [None] * len(stages)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device)
        for i, at in enumerate(range(0, n, chunk)):
            b = i % len(stages)
            if done[b] is not None:
                done[b].synchronize()  # the copy out of this buffer has ended
            m = min(chunk, n - at)
            views[b][:m] = t.data[at : at + m]
            out[at : at + m].copy_(stages[b][:m], non_blocking=True)
            done[b] = torch.cuda.Event()
            done[b].record(stream)
        stream.synchronize()
    return out


def experts(t: Tensor, device) -> B.BlockSwitchLinear:
    """A stack of experts (experts, rows, cols) kept as the file's blocks. strata_mlx/load.py:259-263."""
    if t.type not in B.BLOCK or len(t.shape) != 3:
        raise ValueError(f"{t.name}: {t.type} experts of shape {t.shape} are not supported")
    return B.BlockSwitchLinear(upload(t, device), t.type, t.shape)


def linear(t: Tensor, device):
    """A dense layer (rows, cols) on the file's blocks, called like a Linear: Q6_K as ScaledLinear, the other
    block types as BlockLinear (strata_mlx/load.py:235-256; every type here stays the file's blocks, where the
    reference converts some to MLX's affine form). Float tensors are not layers of this package: to_float."""
    if len(t.shape) != 2:
        raise ValueError(f"{t.name}: a linear layer is 2-D, not {t.shape}")
    if t.type == "Q6_K":
        return D.ScaledLinear.from_blocks(upload(t, device), t.shape)
    if t.type in B.BLOCK or t.type in B.DENSE:
        return D.BlockLinear(upload(t, device), t.type, t.shape)
    raise ValueError(f"{t.name}: {t.type} layers are not kept as blocks")


def embedding(t: Tensor, device, dtype: torch.dtype = torch.float16) -> D.BlockEmbedding:
    """An embedding (vocabulary, dims) whose rows are decoded as tokens come. strata_mlx/load.py:266-273."""
    if len(t.shape) != 2 or not (t.type in B.BLOCK or t.type in B.DENSE):
        raise ValueError(f"{t.name}: {t.type} embedding of shape {t.shape} is not kept as blocks")
    return D.BlockEmbedding(upload(t, device), t.type, t.shape, dtype)


def to_float(t: Tensor) -> np.ndarray:
    """A float tensor as float32 on the host (strata_mlx/gguf.py:135-147, its float types)."""
    if t.type == "F32":
        return t.data.view("<f4").reshape(t.shape).copy()
    if t.type == "F16":
        return t.data.view("<f2").astype(np.float32).reshape(t.shape)
    if t.type == "BF16":
        return (t.data.view("<u2").astype(np.uint32) << 16).view(np.float32).reshape(t.shape)
    raise ValueError(f"{t.name}: {t.type} is not a float type")
