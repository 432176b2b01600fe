"""Writes GGUF files for the tests of strata_mlx_amd.gguf, field by field as the GGUF format (version 3) lays
them out: header, metadata, tensor infos, padding to the alignment, data. A helper, not a test module."""

import struct

import numpy as np

# metadata value type ids of the format
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_CODES = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", BOOL: "?", U64: "Q", I64: "q",
          F64: "d"}


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _string(v)
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack("<" + _CODES[vtype], v)


def write(path: str, tensors: list, meta: list = (), alignment: int | None = None, version: int = 3) -> dict:
    """tensors: (name, shape in numpy order, type id, uint8 bytes); meta: (key, value type, value). Returns
    {name: absolute byte offset of its data}. `alignment` None leaves general.alignment out (the format's 32)."""
    meta = list(meta)
    if alignment is not None:
        meta.append(("general.alignment", U32, alignment))
    align = alignment or 32
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for key, vtype, v in meta:
        head += _string(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offsets, at = [], 0
    for _, _, _, data in tensors:
        offsets.append(at)
        at = (at + len(data) + align - 1) // align * align
    for (name, shape, type_id, _), off in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(shape)) + struct.pack(f"<{len(shape)}Q", *reversed(shape))
        head += struct.pack("<IQ", type_id, off)
    start = (len(head) + align - 1) // align * align
    body = bytearray(head + bytes(start - len(head)))
    for (_, _, _, data), off in zip(tensors, offsets):
        body += bytes(start + off - len(body))
        body += np.asarray(data, np.uint8).tobytes()
    with open(path, "wb") as f:
        f.write(bytes(body))
    return {t[0]: start + off for t, off in zip(tensors, offsets)}
