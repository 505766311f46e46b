"""cuVS index files: a 4-byte dtype prefix, then every scalar and array as
one NumPy ``.npy`` (format 1.0) record, little endian.

The layout of reference python/mlxvs/cuvs/_serialize.py, which follows
RAFT's ``numpy_serializer``: the header dict is written without a trailing
comma and padded with 1 to 64 spaces and a newline so that magic, version,
length and header end on a multiple of 64 bytes; one-byte types (and bool)
carry no byte order, binary16 is ``<e2`` (``<f2`` in a prefix of format 6 or
later).  Readers accept any valid format 1.0 record.
"""

from __future__ import annotations

import ast
import struct

import numpy as np

MAGIC = b"\x93NUMPY"

_DESCR = {
    np.dtype(np.float32): "<f4",
    np.dtype(np.float64): "<f8",
    np.dtype(np.float16): "<e2",
    np.dtype(np.int8): "|i1",
    np.dtype(np.uint8): "|u1",
    np.dtype(np.bool_): "|u1",
    np.dtype(np.int32): "<i4",
    np.dtype(np.uint32): "<u4",
    np.dtype(np.int64): "<i8",
    np.dtype(np.uint64): "<u8",
}
_TYPES = {
    "<f4": np.float32, "<f8": np.float64, "<e2": np.float16, "<f2": np.float16,
    "|i1": np.int8, "|u1": np.uint8, "<i4": np.int32, "<u4": np.uint32,
    "<i8": np.int64, "<u8": np.uint64, "|b1": np.bool_,
}


def _shape_text(shape) -> str:
    dims = [str(int(s)) for s in shape]
    if not dims:
        return "()"
    if len(dims) == 1:
        return f"({dims[0]},)"
    return "(" + ", ".join(dims) + ")"


def header_bytes(dtype, shape) -> bytes:
    """The record header of an array of `dtype` and `shape`."""
    text = (f"{{'descr': '{_DESCR[np.dtype(dtype)]}', 'fortran_order': False, "
            f"'shape': {_shape_text(shape)}}}")
    fixed = len(MAGIC) + 2 + 2
    spaces = 64 - (fixed + len(text) + 1) % 64  # 1 .. 64
    body = text.encode("latin1") + b" " * spaces + b"\n"
    return MAGIC + b"\x01\x00" + struct.pack("<H", len(body)) + body


def write_scalar(f, value, dtype) -> None:
    f.write(header_bytes(dtype, ()))
    f.write(np.asarray(value, dtype=dtype).astype(np.dtype(dtype).newbyteorder("<")).tobytes())


def write_array(f, a, dtype=None) -> None:
    a = np.ascontiguousarray(a, dtype=dtype)
    f.write(header_bytes(a.dtype, a.shape))
    f.write(a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes())


def read_header(f):
    """(dtype, shape) of the next record."""
    head = f.read(10)
    if len(head) < 10 or head[:6] != MAGIC:
        raise ValueError("not a cuVS index file: missing a NumPy record")
    if head[6] != 1:
        raise ValueError(f"unsupported NumPy record version {head[6]}.{head[7]}")
    (hlen,) = struct.unpack("<H", head[8:10])
    d = ast.literal_eval(f.read(hlen).decode("latin1").strip())
    if d.get("fortran_order"):
        raise ValueError("Fortran-ordered arrays are not supported")
    if d["descr"] not in _TYPES:
        raise ValueError(f"unsupported dtype {d['descr']!r}")
    return np.dtype(_TYPES[d["descr"]]), tuple(d["shape"])


def read_scalar(f):
    dtype, shape = read_header(f)
    if shape:
        raise ValueError(f"expected a scalar, found shape {shape}")
    raw = f.read(dtype.itemsize)
    if len(raw) != dtype.itemsize:
        raise ValueError("truncated cuVS index file")
    return np.frombuffer(raw, dtype=dtype.newbyteorder("<"))[0].item()


def read_array(f) -> np.ndarray:
    dtype, shape = read_header(f)
    count = int(np.prod(shape)) if shape else 1
    raw = f.read(count * dtype.itemsize)
    if len(raw) != count * dtype.itemsize:
        raise ValueError("truncated cuVS index file")
    return np.frombuffer(raw, dtype=dtype.newbyteorder("<")).astype(dtype).reshape(shape)


def dtype_prefix(dtype, version: int) -> bytes:
    """The 4-byte dtype prefix of an index file."""
    s = _DESCR[np.dtype(dtype)]
    if s == "<e2" and version >= 6:
        s = "<f2"
    return s.encode().ljust(4, b"\0")


def read_prefix(f) -> np.dtype:
    s = f.read(4).rstrip(b"\0").decode("latin1")
    if s not in _TYPES:
        raise ValueError(f"unknown dtype prefix {s!r}")
    return np.dtype(_TYPES[s])
