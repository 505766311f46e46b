"""The record framing of cuVS / RAFT index files.

An index file starts with a 4-byte type tag (the dataset's element type as
text, NUL padded) and continues as a run of NumPy ``.npy`` format-1.0
records, one per scalar or array, all little endian.  RAFT's
``numpy_serializer`` (which cuVS uses, and which the reference's Python
package reproduces in python/mlxvs/cuvs/_serialize.py) frames them in a way
NumPy's own writer does not, and cuVS's readers expect that framing:

* the header dictionary has no trailing comma after its last entry;
* it is followed by 1 to 64 spaces and a newline, so that the payload
  starts on a 64-byte boundary of the record;
* one-byte types carry no byte order (``|u1``, ``|i1``; a bool is written
  as ``|u1``), and binary16 is ``<e2`` -- except in the type tag of files of
  format version 6 and later, where it reads ``<f2``.

NumPy's reader (``numpy.lib.format``) accepts every record written here.
"""

from __future__ import annotations

import ast
import struct
from typing import BinaryIO

import numpy as np

# element types and the type text written for each
_CODES = (
    (np.float32, "<f4"),
    (np.float64, "<f8"),
    (np.float16, "<e2"),
    (np.int8, "|i1"),
    (np.uint8, "|u1"),
    (np.int32, "<i4"),
    (np.uint32, "<u4"),
    (np.int64, "<i8"),
    (np.uint64, "<u8"),
)
_TEXT_OF = {np.dtype(t): text for t, text in _CODES}
_TEXT_OF[np.dtype(np.bool_)] = "|u1"
_TYPE_OF = {text: np.dtype(t) for t, text in _CODES}
_TYPE_OF["<f2"] = np.dtype(np.float16)
_TYPE_OF["|b1"] = np.dtype(np.bool_)

_LEAD = b"\x93NUMPY\x01\x00"  # magic string and format version 1.0
_ALIGN = 64


def _type_text(dtype) -> str:
    try:
        return _TEXT_OF[np.dtype(dtype)]
    except KeyError:
        raise ValueError(f"no cuVS record type for {np.dtype(dtype)}") from None


def record_header(dtype, shape) -> bytes:
    """Lead, header length and padded header dictionary of one record."""
    shape = tuple(int(s) for s in shape)
    meta = f"{{'descr': '{_type_text(dtype)}', 'fortran_order': False, 'shape': {shape}}}"
    used = len(_LEAD) + 2 + len(meta) + 1  # the newline ends the header
    meta += " " * (_ALIGN - used % _ALIGN) + "\n"
    return _LEAD + struct.pack("<H", len(meta)) + meta.encode("latin1")


class RecordWriter:
    """Appends records to a binary file object."""

    def __init__(self, f: BinaryIO):
        self._f = f

    def scalar(self, value, dtype) -> None:
        dt = np.dtype(dtype)
        self._f.write(record_header(dt, ()))
        self._f.write(np.asarray(value, dtype=dt).astype(dt.newbyteorder("<")).tobytes())

    def array(self, a, dtype=None) -> None:
        a = np.ascontiguousarray(a, dtype=dtype)
        self._f.write(record_header(a.dtype, a.shape))
        self._f.write(a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes())


class RecordReader:
    """Takes records from a binary file object, one at a time."""

    def __init__(self, f: BinaryIO):
        self._f = f

    def _take(self, count: int) -> bytes:
        raw = self._f.read(count)
        if len(raw) != count:
            raise ValueError("the cuVS index file ends inside a record")
        return raw

    def header(self):
        """(dtype, shape) of the next record."""
        lead = self._take(len(_LEAD) + 2)
        if lead[:6] != _LEAD[:6]:
            raise ValueError("not a cuVS index file: expected a NumPy record")
        if lead[6] != 1:
            raise ValueError(f"NumPy record format {lead[6]}.{lead[7]} is not read here "
                             "(RAFT writes 1.0)")
        (size,) = struct.unpack("<H", lead[8:10])
        meta = ast.literal_eval(self._take(size).decode("latin1").strip())
        if not isinstance(meta, dict) or meta.get("fortran_order", False):
            raise ValueError("cuVS records hold C-ordered arrays only")
        dt = _TYPE_OF.get(meta.get("descr"))
        if dt is None:
            raise ValueError(f"record type {meta.get('descr')!r} is not a cuVS type")
        return dt, tuple(int(s) for s in meta["shape"])

    def _payload(self, dt: np.dtype, shape) -> np.ndarray:
        count = int(np.prod(shape, dtype=np.int64)) if shape else 1
        raw = self._take(count * dt.itemsize)
        return np.frombuffer(raw, dtype=dt.newbyteorder("<")).astype(dt).reshape(shape)

    def scalar(self):
        dt, shape = self.header()
        if shape:
            raise ValueError(f"expected a scalar record, found one of shape {shape}")
        return self._payload(dt, shape).item()

    def array(self) -> np.ndarray:
        dt, shape = self.header()
        return self._payload(dt, shape)


def type_tag(dtype, version: int) -> bytes:
    """The 4-byte type tag that opens an index file of format `version`."""
    text = _type_text(dtype)
    if text == "<e2" and version >= 6:
        text = "<f2"
    return text.encode("latin1").ljust(4, b"\0")


def read_type_tag(f: BinaryIO) -> np.dtype:
    """The element type named by a file's opening tag."""
    text = f.read(4).rstrip(b"\0").decode("latin1")
    if text not in _TYPE_OF:
        raise ValueError(f"the file's type tag {text!r} names no cuVS type")
    return _TYPE_OF[text]
