"""The TEXMEX vector files around the k-NN path (ANN benchmark datasets).

``.fvecs`` / ``.ivecs`` / ``.bvecs``: every vector is stored as its dimension
(int32, little endian) followed by its components (float32, int32 or
uint8).  The reference reads base and query rows from ``.fvecs`` and writes
the exact neighbours as ``.ivecs`` (reference examples/ground_truth.py:19-31);
:func:`ground_truth` is that script's computation on this engine.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

__all__ = ["read_fvecs", "write_fvecs", "read_ivecs", "write_ivecs", "read_bvecs",
           "write_bvecs", "ground_truth"]


def _read_vecs(path, dtype) -> np.ndarray:
    raw = np.fromfile(path, dtype=np.uint8)
    if raw.size == 0:
        return np.zeros((0, 0), dtype=dtype)
    d = int(raw[:4].view("<i4")[0])
    item = np.dtype(dtype).itemsize
    rec = 4 + d * item
    if d < 1 or raw.size % rec != 0:
        raise ValueError(f"{path}: not a vector file of dimension {d} "
                         f"({raw.size} bytes, records of {rec})")
    rows = raw.reshape(-1, rec)
    dims = rows[:, :4].copy().view("<i4").ravel()
    if (dims != d).any():
        raise ValueError(f"{path}: vectors of different dimensions")
    return np.ascontiguousarray(rows[:, 4:]).view(np.dtype(dtype).newbyteorder("<")).astype(
        dtype, copy=False)


def _write_vecs(path, a, dtype) -> None:
    a = np.asarray(a)
    if a.ndim != 2:
        raise ValueError("vectors must be 2-D [n, d]")
    n, d = a.shape
    item = np.dtype(dtype).itemsize
    out = np.empty((n, 4 + d * item), dtype=np.uint8)
    out[:, :4] = np.full((n, 1), d, dtype="<i4").view(np.uint8)
    out[:, 4:] = np.ascontiguousarray(a, dtype=np.dtype(dtype).newbyteorder("<")).view(
        np.uint8).reshape(n, d * item)
    out.tofile(path)


def read_fvecs(path) -> np.ndarray:
    """float32 [n, d] from an ``.fvecs`` file."""
    return _read_vecs(path, np.float32)


def write_fvecs(path, a) -> None:
    _write_vecs(path, a, np.float32)


def read_ivecs(path) -> np.ndarray:
    """int32 [n, d] from an ``.ivecs`` file."""
    return _read_vecs(path, np.int32)


def write_ivecs(path, a) -> None:
    """int32 [n, k] as ``.ivecs`` (each row prefixed by k)."""
    _write_vecs(path, a, np.int32)


def read_bvecs(path) -> np.ndarray:
    """uint8 [n, d] from a ``.bvecs`` file."""
    return _read_vecs(path, np.uint8)


def write_bvecs(path, a) -> None:
    _write_vecs(path, a, np.uint8)


def ground_truth(base_path, query_path, out_path, k: int = 100, metric: str = "l2"):
    """The k exact nearest base rows of every query, written as ``.ivecs``.

    The computation of reference examples/ground_truth.py:34-53: base and
    query rows from ``.fvecs``, ids from brute_force_knn.  Returns the ids.
    """
    from mlxvs_amd import brute_force_knn

    base, queries = read_fvecs(base_path), read_fvecs(query_path)
    ids, _ = brute_force_knn(base, queries, k, metric)
    write_ivecs(Path(out_path), ids)
    return ids
