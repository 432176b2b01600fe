"""The GGUF reader (strata_mlx/gguf.py:63-133) on the CPU: a file assembled byte by byte from the format, files of
every type, alignment and metadata type from tests/gguf_files.py, shards, float tensors (test_gguf.py:62-66 of the
reference), and malformed files, which raise ValueError."""

import struct

import numpy as np
import pytest

import gguf_files as W
from strata_mlx_amd import gguf as G


def _u32(v):
    return struct.pack("<I", v)


def _u64(v):
    return struct.pack("<Q", v)


def test_a_file_laid_out_by_hand(tmp_path):
    # header 24 B; "general.alignment" u32 64: 8 + 17 + 4 + 4 = 33 B; "a" [i32 -1, 2, 3]: 8 + 1 + 4 + 4 + 8 + 12
    # = 37 B; tensor "w" Q2_0 (3, 64): 8 + 1 + 4 + 16 + 4 + 8 = 41 B. 135 B of header; data at 192.
    head = b"GGUF" + _u32(3) + _u64(1) + _u64(2)
    head += _u64(17) + b"general.alignment" + _u32(4) + _u32(64)
    head += _u64(1) + b"a" + _u32(9) + _u32(5) + _u64(3) + struct.pack("<3i", -1, 2, 3)
    head += _u64(1) + b"w" + _u32(2) + _u64(64) + _u64(3) + _u32(42) + _u64(0)
    assert len(head) == 135
    data = np.arange(54, dtype=np.uint8) * 3
    path = tmp_path / "hand.gguf"
    path.write_bytes(head + bytes(192 - 135) + data.tobytes())
    g = G.GGUF(str(path))
    assert g.version == 3 and g.alignment == 64 and g.data_start == 192
    assert g.meta == {"general.alignment": 64, "a": [-1, 2, 3]}
    t = g["w"]
    assert (t.name, t.shape, t.type, t.offset, t.nbytes) == ("w", (3, 64), "Q2_0", 192, 54)
    assert np.array_equal(t.data, data) and t.quantized and "w" in g and "v" not in g


@pytest.mark.parametrize("alignment", [None, 64, 256])
@pytest.mark.parametrize("version", [2, 3])
def test_every_type_reads_back_where_it_was_written(tmp_path, alignment, version):
    rng = np.random.default_rng(version * 7 + (alignment or 0))
    tensors = []
    for type_id, (name, per_block, block_bytes) in sorted(G.TYPES.items()):
        rows, blocks_a_row = int(rng.integers(1, 5)), int(rng.integers(1, 4))
        shape = (rows, blocks_a_row * per_block * (8 if per_block == 1 else 1))
        if type_id == 21:  # an expert stack too
            shape = (3, rows, shape[1])
        n = G.tensor_bytes(type_id, shape)
        tensors.append((f"t.{name}", shape, type_id, rng.integers(0, 256, n, dtype=np.uint8)))
    path = str(tmp_path / "all.gguf")
    where = W.write(path, tensors, alignment=alignment, version=version)
    g = G.GGUF(path)
    assert len(g.tensors) == len(tensors)
    for name, shape, type_id, data in tensors:
        t = g[name]
        assert t.shape == shape and t.type == G.TYPES[type_id][0] and t.offset == where[name]
        assert t.offset % (alignment or 32) == 0
        assert np.array_equal(t.data, data)


def test_metadata_of_every_value_type(tmp_path):
    meta = [("u8", W.U8, 200), ("i8", W.I8, -100), ("u16", W.U16, 60000), ("i16", W.I16, -30000),
            ("u32", W.U32, 4_000_000_000), ("i32", W.I32, -2_000_000_000), ("f32", W.F32, 0.5),
            ("bool", W.BOOL, True), ("str", W.STRING, "qwen ✓"), ("u64", W.U64, 1 << 63),
            ("i64", W.I64, -(1 << 62)), ("f64", W.F64, 1e-300),
            ("tokens", W.ARRAY, (W.STRING, ["<s>", "", "é"])), ("ids", W.ARRAY, (W.U32, [1, 2, 3])),
            ("nested", W.ARRAY, (W.ARRAY, [(W.I16, [1, -1]), (W.I16, [])])), ("empty", W.ARRAY, (W.F32, []))]
    path = str(tmp_path / "meta.gguf")
    W.write(path, [], meta)
    got = G.GGUF(path).meta
    assert got == {"u8": 200, "i8": -100, "u16": 60000, "i16": -30000, "u32": 4_000_000_000,
                   "i32": -2_000_000_000, "f32": 0.5, "bool": True, "str": "qwen ✓", "u64": 1 << 63,
                   "i64": -(1 << 62), "f64": 1e-300, "tokens": ["<s>", "", "é"], "ids": [1, 2, 3],
                   "nested": [[1, -1], []], "empty": []}


def test_shards_are_found_beside_the_first(tmp_path):
    for i in (1, 2, 3):
        W.write(str(tmp_path / f"m-{i:05d}-of-00003.gguf"), [(f"t{i}", (1, 32), 8, np.full(34, i, np.uint8))])
    files = G.shards(str(tmp_path / "m-00001-of-00003.gguf"))
    assert [list(f.tensors) for f in files] == [["t1"], ["t2"], ["t3"]]
    W.write(str(tmp_path / "one.gguf"), [])
    assert len(G.shards(str(tmp_path / "one.gguf"))) == 1


def test_float_tensors():
    bits = np.array([0x3F80, 0xBF00, 0x37FB, 0x4480], dtype="<u2")  # 1, -0.5, about 3e-5, 1024
    want = (bits.astype(np.uint32) << 16).view(np.float32)
    assert want[0] == 1.0 and want[3] == 1024.0
    np.testing.assert_array_equal(G.to_float(G.Tensor("t", (4,), "BF16", bits.view(np.uint8))), want)
    h = np.array([1.0, -2.5, 65504.0], np.float16)
    np.testing.assert_array_equal(G.to_float(G.Tensor("t", (3,), "F16", h.view(np.uint8))), h.astype(np.float32))
    f = np.array([[1.5, -0.0]], np.float32)
    np.testing.assert_array_equal(G.to_float(G.Tensor("t", (1, 2), "F32", f.reshape(-1).view(np.uint8))), f)
    with pytest.raises(ValueError):
        G.to_float(G.Tensor("t", (1, 32), "Q8_0", np.zeros(34, np.uint8)))


def _good(tmp_path):
    path = str(tmp_path / "good.gguf")
    W.write(path, [("w", (2, 64), 42, np.zeros(36, np.uint8))], [("k", W.STRING, "v")])
    return path


def test_malformed_files_raise(tmp_path):
    good = open(_good(tmp_path), "rb").read()
    G.GGUF(_good(tmp_path))  # reads
    cases = {"magic": b"GGUF"[::-1] + good[4:], "version": good[:4] + _u32(1) + good[8:], "empty": b""}
    for cut in (3, 10, 30, 60, len(good) - 40, len(good) - 1):  # truncated header, truncated data
        cases[f"cut{cut}"] = good[:cut]
    for name, blob in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(blob)
        with pytest.raises(ValueError):
            G.GGUF(str(p))
    for type_id, shape in ((99, (2, 64)), (42, (2, 48))):  # a type not defined; rows not ending on a block
        p = str(tmp_path / f"bad{type_id}.gguf")
        W.write(p, [("w", shape, type_id, np.zeros(36, np.uint8))])
        with pytest.raises(ValueError):
            G.GGUF(p)


def test_layers_refuse_what_the_kernels_do_not_take(tmp_path):
    path = str(tmp_path / "types.gguf")
    W.write(path, [("f", (4, 32), 1, np.zeros(256, np.uint8)), ("q", (2, 4, 256), 12, np.zeros(1152, np.uint8))])
    g = G.GGUF(path)
    with pytest.raises(ValueError):
        G.experts(g["f"], "cuda:0")  # float experts
    with pytest.raises(ValueError):
        G.experts(g["q"], "cuda:0")  # Q4_K is a dense type of the loader, not an expert block type
    with pytest.raises(ValueError):
        G.linear(g["f"], "cuda:0")
    with pytest.raises(ValueError):
        G.linear(g["q"], "cuda:0")  # 3-D
    with pytest.raises(ValueError):
        G.upload(g["q"], "cpu")
