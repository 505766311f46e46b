"""cuVS's ``cuvs.neighbors.brute_force`` on the exact k-NN engine.

Mirrors reference python/mlxvs/cuvs/neighbors/brute_force.py: ``build`` keeps
the rows and a cuVS distance type, ``search`` answers with the fused k-NN
(``brute_force_knn``, or ``hamming_knn`` for bit-packed rows) and returns
``(distances float32, neighbors int64)`` in cuVS's units, ``save`` / ``load``
use cuVS's brute-force file format (version 0; :mod:`mlxvs_amd.cuvs._serialize`),
which cuVS's own ``brute_force.load`` reads.

The engine's metrics are the ones this index takes: ``"sqeuclidean"``
(L2Expanded), ``"euclidean"`` / ``"l2"`` (L2SqrtExpanded),
``"inner_product"``, ``"cosine"`` (CosineExpanded) and ``"bitwise_hamming"``.
The reference's element-wise pairwise metrics (cityblock, chebyshev, ...)
and its prefilters run outside the fused path and are not part of this
engine; asking for them raises ``ValueError``.
"""

from __future__ import annotations

import numpy as np

from mlxvs_amd.cuvs import _serialize as io

__all__ = ["Index", "build", "load", "save", "search"]

# cuVS DistanceType values (reference python/mlxvs/cuvs/distance.py:12-32)
L2Expanded = 0
L2SqrtExpanded = 1
CosineExpanded = 2
InnerProduct = 6
BitwiseHamming = 20

DISTANCE_TYPES = {
    "sqeuclidean": L2Expanded,
    "euclidean": L2SqrtExpanded,
    "l2": L2SqrtExpanded,
    "inner_product": InnerProduct,
    "cosine": CosineExpanded,
    "bitwise_hamming": BitwiseHamming,
}
_NAMES = {L2Expanded: "sqeuclidean", L2SqrtExpanded: "euclidean", CosineExpanded: "cosine",
          InnerProduct: "inner_product", BitwiseHamming: "bitwise_hamming"}
# engine metric of each distance type
_ENGINE = {L2Expanded: "l2", L2SqrtExpanded: "l2", InnerProduct: "inner_product",
           CosineExpanded: "cosine"}

_SERIALIZATION_VERSION = 0


def _metric_type(metric) -> int:
    if isinstance(metric, str):
        if metric not in DISTANCE_TYPES:
            raise ValueError(f"metric {metric!r} is not supported by this engine; one of "
                             + ", ".join(repr(m) for m in DISTANCE_TYPES))
        return DISTANCE_TYPES[metric]
    t = int(metric)
    if t not in _NAMES:
        raise ValueError(f"distance type {t} is not supported by this engine")
    return t


class Index:
    """A brute-force index: the dataset and its distance type."""

    def __init__(self):
        self.trained = False
        self._dataset = None
        self._metric = L2Expanded
        self._metric_arg = 2.0

    @property
    def dataset(self):
        return self._dataset

    def __len__(self):
        return 0 if self._dataset is None else self._dataset.shape[0]

    def __repr__(self):
        return f"Index(type=BruteForce, metric={_NAMES.get(self._metric)})"


def build(dataset, metric="sqeuclidean", metric_arg=2.0, resources=None):
    """The index of ``dataset`` [n, dim] (float32 / float16 rows, or bit-packed
    uint8 rows for ``"bitwise_hamming"``), as cuVS's ``brute_force.build``."""
    x = np.asarray(dataset)
    if x.ndim != 2:
        raise ValueError("dataset must be a matrix")
    t = _metric_type(metric)
    if t == BitwiseHamming and x.dtype != np.uint8:
        raise ValueError("bitwise_hamming needs bit-packed uint8 rows")
    idx = Index()
    idx._dataset = np.ascontiguousarray(x)
    idx._metric = t
    idx._metric_arg = float(metric_arg)
    idx.trained = True
    return idx


def _to_cuvs(scores: np.ndarray, t: int) -> np.ndarray:
    """Engine outputs (squared L2, inner product, cosine similarity) as cuVS's
    distances (reference python/mlxvs/cuvs/neighbors/_common.py:39-48)."""
    if t == L2SqrtExpanded:
        return np.sqrt(np.maximum(scores, 0))
    if t == L2Expanded:
        return np.maximum(scores, 0)
    if t == CosineExpanded:
        return 1 - scores
    return scores


def search(index, queries, k, neighbors=None, distances=None, resources=None,
           prefilter=None):
    """The k nearest rows of every query, as cuVS's ``brute_force.search``.

    Returns ``(distances float32 [nq, k], neighbors int64 [nq, k])``,
    nearest first (largest inner product first); ``neighbors`` /
    ``distances`` given as arrays are filled in place.  -1 where fewer than
    k rows exist.
    """
    from mlxvs_amd import brute_force_knn, hamming_knn

    if not index.trained:
        raise ValueError("Index needs to be built before calling search.")
    if prefilter is not None and getattr(prefilter, "type", "none") != "none":
        raise ValueError("prefilters are not supported by this engine")
    q = np.asarray(queries)
    t = index._metric
    if t == BitwiseHamming:
        ids, dist = hamming_knn(index._dataset, q, k)
    else:
        ids, scores = brute_force_knn(index._dataset, q, k, _ENGINE[t])
        dist = _to_cuvs(scores, t)
    ids = np.where(ids < 0, -1, ids).astype(np.int64)
    dist = np.asarray(dist, dtype=np.float32)
    if distances is not None:
        distances[...] = dist
        dist = distances
    if neighbors is not None:
        neighbors[...] = ids
        ids = neighbors
    return dist, ids


def save(filename, index, include_dataset=True, resources=None):
    """Writes the index in cuVS's brute-force format (version 0): dtype prefix,
    version, rows, dim, distance type, metric arg, the dataset flag and rows,
    then the norms flag and the rows' norms (squared for L2, plain for
    cosine) -- reference python/mlxvs/cuvs/neighbors/brute_force.py:142-165."""
    data = np.asarray(index._dataset)
    t = index._metric
    with open(filename, "wb") as f:
        f.write(io.dtype_prefix(data.dtype, 6))
        io.write_scalar(f, _SERIALIZATION_VERSION, np.int32)
        io.write_scalar(f, data.shape[0], np.uint64)
        io.write_scalar(f, data.shape[1], np.uint64)
        io.write_scalar(f, t, np.int32)
        io.write_scalar(f, index._metric_arg, np.float32)
        io.write_scalar(f, bool(include_dataset), np.bool_)
        if include_dataset:
            io.write_array(f, data)
        has_norms = t in (L2Expanded, L2SqrtExpanded, CosineExpanded)
        io.write_scalar(f, has_norms, np.bool_)
        if has_norms:
            x = data.astype(np.float32)
            norms = np.sum(x * x, axis=1)
            if t == CosineExpanded:
                norms = np.sqrt(norms)
            io.write_array(f, norms.astype(np.float32))


def load(filename, resources=None):
    """Reads an index written by :func:`save` or by cuVS."""
    with open(filename, "rb") as f:
        dtype = io.read_prefix(f)
        ver = io.read_scalar(f)
        if ver != _SERIALIZATION_VERSION:
            raise ValueError(f"serialization version mismatch, expected "
                             f"{_SERIALIZATION_VERSION}, got {ver}")
        io.read_scalar(f)  # rows
        io.read_scalar(f)  # dim
        metric = io.read_scalar(f)
        metric_arg = io.read_scalar(f)
        if not io.read_scalar(f):
            raise ValueError("the file holds no dataset; brute force needs it")
        data = io.read_array(f).astype(dtype, copy=False)
    idx = Index()
    idx._dataset = np.ascontiguousarray(data)
    idx._metric = _metric_type(int(metric))
    idx._metric_arg = float(metric_arg)
    idx.trained = True
    return idx
