"""Minimal GGUF writer for tests: the on-disk layout of GGUF versions 1-3
(little endian), written with `struct` from the format description and
independent of the reader under test.

    header   b"GGUF", u32 version, tensor count, metadata count
             (u32 each in version 1, u64 from version 2)
    metadata key string, u32 value type, value
    tensors  name, u32 n_dims, dims (u32 in v1, u64 after; ggml order, the
             contiguous dimension first), u32 ggml type, u64 offset
    data     aligned to `alignment` (general.alignment, default 32); each
             tensor's offset is relative to the data start and aligned too

The reference builds its GGUF fixtures the same way through candle's
gguf_file::write (qwen3_8/ggml_tests.rs:72-212): architecture string, U32
hyper-parameters, F32 values, Q4K / Q8_0 / F32 tensors.
"""
from __future__ import annotations

import struct

VT = {"U8": 0, "I8": 1, "U16": 2, "I16": 3, "U32": 4, "I32": 5, "F32": 6, "BOOL": 7,
      "STRING": 8, "ARRAY": 9, "U64": 10, "I64": 11, "F64": 12}
_SCALAR = {"U8": "<B", "I8": "<b", "U16": "<H", "I16": "<h", "U32": "<I", "I32": "<i",
           "F32": "<f", "BOOL": "<?", "U64": "<Q", "I64": "<q", "F64": "<d"}
# ggml type id, elements per block, bytes per block
GGML = {"F32": (0, 1, 4), "F16": (1, 1, 2), "Q4_0": (2, 32, 18), "Q8_0": (8, 32, 34),
        "Q4K": (12, 256, 144), "Q6K": (14, 256, 210), "BF16": (30, 1, 2)}


def _len(n: int, version: int) -> bytes:
    return struct.pack("<I" if version == 1 else "<Q", n)


def _str(s: str, version: int, nul: bool = False) -> bytes:
    b = s.encode() + (b"\0" if nul else b"")
    return _len(len(b), version) + b


def _value(vtype: str, value, version: int, nul: bool) -> bytes:
    if vtype == "STRING":
        return _str(value, version, nul)
    if vtype == "ARRAY":
        etype, items = value
        out = struct.pack("<I", VT[etype]) + _len(len(items), version)
        return out + b"".join(_value(etype, v, version, nul) for v in items)
    return struct.pack(_SCALAR[vtype], value)


def tensor_nbytes(ggml: str, dims) -> int:
    _, bs, ts = GGML[ggml]
    n = 1
    for d in dims:
        n *= d
    return n // bs * ts


def write_gguf(path, metadata, tensors, version: int = 3, alignment: int = 32,
               nul_strings: bool = False, ggml_type_ids=None, truncate: int = 0,
               check_sizes: bool = True) -> int:
    """metadata: [(key, value type name, value)] (ARRAY values are
    (element type name, [items])); tensors: [(name, ggml type name, dims in
    candle order [outer, ..., contiguous], raw bytes)].  A general.alignment
    entry in `metadata` must agree with `alignment`.  ggml_type_ids overrides
    the type id written per tensor name; truncate drops that many bytes from
    the end; check_sizes=False writes tensor infos whose bytes do not match
    their dims (for reader error tests).  Returns the data start offset."""
    head = b"GGUF" + struct.pack("<I", version) + _len(len(tensors), version) + _len(len(metadata), version)
    body = b""
    for key, vtype, value in metadata:
        body += _str(key, version, nul_strings) + struct.pack("<I", VT[vtype]) + _value(vtype, value, version, nul_strings)
    offsets, off = [], 0
    for name, ggml, dims, raw in tensors:
        assert not check_sizes or len(raw) == tensor_nbytes(ggml, dims), (name, len(raw))
        offsets.append(off)
        off += len(raw)
        off = (off + alignment - 1) // alignment * alignment
    for (name, ggml, dims, raw), toff in zip(tensors, offsets):
        tid = (ggml_type_ids or {}).get(name, GGML[ggml][0])
        body += _str(name, version, nul_strings) + struct.pack("<I", len(dims))
        for d in reversed(dims):  # ggml order: contiguous dimension first
            body += struct.pack("<I" if version == 1 else "<Q", d)
        body += struct.pack("<I", tid) + struct.pack("<Q", toff)
    blob = head + body
    data_start = (len(blob) + alignment - 1) // alignment * alignment
    blob += b"\0" * (data_start - len(blob))
    for (name, ggml, dims, raw), toff in zip(tensors, offsets):
        blob += b"\0" * (data_start + toff - len(blob)) + raw
    if truncate:
        blob = blob[:-truncate]
    with open(path, "wb") as f:
        f.write(blob)
    return data_start
