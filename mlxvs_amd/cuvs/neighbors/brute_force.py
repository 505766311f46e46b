"""cuVS's ``cuvs.neighbors.brute_force`` (build / search / save / load) on the
exact k-NN engine.

The public names and arguments are cuVS's, as the reference's compatibility
module python/mlxvs/cuvs/neighbors/brute_force.py keeps them.  Search runs
the fused k-NN (``brute_force_knn``, or ``hamming_knn`` for bit-packed rows)
and reports cuVS's distance units.  Files are cuVS's brute-force format,
version 0, readable by cuVS's own ``brute_force.load``.

Distance types served: ``"sqeuclidean"`` (L2Expanded), ``"euclidean"`` /
``"l2"`` (L2SqrtExpanded), ``"cosine"`` (CosineExpanded),
``"inner_product"`` and ``"bitwise_hamming"``.  cuVS's element-wise
pairwise metrics (cityblock, chebyshev, minkowski, ...) are evaluated
outside a fused top-k path and are not offered: they raise ``ValueError``.

Prefilters (``filters.from_bitset`` / ``from_bitmap``) run inside the fused
select (``brute_force_knn_filtered``): a row a filter leaves out never
enters a candidate list, and a query with fewer than k allowed rows gets -1
ids and the worst distance past them, as the reference's masked selection
gives (python/mlxvs/cuvs/neighbors/brute_force.py:97-136).  Bit-packed rows
with a prefilter are searched as {0, 1} float rows, whose squared L2
distance is their Hamming distance (exact in float32).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional

import numpy as np

from mlxvs_amd.cuvs._serialize import RecordReader, RecordWriter, read_type_tag, type_tag

__all__ = ["Index", "build", "load", "save", "search"]


@dataclass(frozen=True)
class _Distance:
    """A cuVS distance type and how this module serves it."""

    code: int                  # cuVS DistanceType value
    name: str                  # cuVS metric name
    engine: Optional[str]      # engine metric (None: Hamming on packed bits)
    norms: Optional[str]       # the norms record a file carries: "squared", "plain"
    units: Callable[[np.ndarray], np.ndarray]  # engine output -> cuVS distance


# cuVS DistanceType values (cuvs/distance/distance.hpp, as the reference's
# python/mlxvs/cuvs/distance.py:12-32 lists them)
_DISTANCES = (
    _Distance(0, "sqeuclidean", "l2", "squared", lambda d: np.maximum(d, 0)),
    _Distance(1, "euclidean", "l2", "squared", lambda d: np.sqrt(np.maximum(d, 0))),
    _Distance(2, "cosine", "cosine", "plain", lambda s: 1 - s),
    _Distance(6, "inner_product", "inner_product", None, lambda s: s),
    _Distance(20, "bitwise_hamming", None, None, lambda d: d),
)
_BY_CODE = {d.code: d for d in _DISTANCES}
_BY_NAME = {d.name: d for d in _DISTANCES}
_BY_NAME["l2"] = _BY_CODE[1]

FORMAT_VERSION = 0


def _distance(metric) -> _Distance:
    if isinstance(metric, str):
        found = _BY_NAME.get(metric)
    else:
        found = _BY_CODE.get(int(metric))
    if found is None:
        served = ", ".join(sorted(_BY_NAME))
        raise ValueError(f"metric {metric!r} is not supported here (served: {served})")
    return found


class Index:
    """A brute-force index: the rows and their cuVS distance type."""

    def __init__(self):
        self._rows: Optional[np.ndarray] = None
        self._distance = _BY_CODE[0]
        self._metric_arg = 2.0

    @property
    def trained(self) -> bool:
        return self._rows is not None

    @property
    def dataset(self) -> Optional[np.ndarray]:
        return self._rows

    @property
    def metric(self) -> str:
        return self._distance.name

    @property
    def distance_type(self) -> int:
        return self._distance.code

    def __len__(self):
        return 0 if self._rows is None else int(self._rows.shape[0])

    def __repr__(self):
        return f"brute_force.Index(rows={len(self)}, metric={self.metric!r})"


def _index(rows: np.ndarray, dist: _Distance, metric_arg: float) -> Index:
    if dist.code == 20 and rows.dtype != np.uint8:
        raise ValueError("bitwise_hamming indexes bit-packed uint8 rows")
    idx = Index()
    idx._rows = np.ascontiguousarray(rows)
    idx._distance = dist
    idx._metric_arg = float(metric_arg)
    return idx


def build(dataset, metric="sqeuclidean", metric_arg=2.0, resources=None) -> Index:
    """The index of ``dataset`` (float32 / float16 rows ``[n, dim]``, or
    bit-packed uint8 rows for ``"bitwise_hamming"``); the rows are kept."""
    rows = np.asarray(dataset)
    if rows.ndim != 2:
        raise ValueError(f"the dataset must be a matrix [n, dim], got {rows.ndim} dimensions")
    return _index(rows, _distance(metric), metric_arg)


def search(index, queries, k, neighbors=None, distances=None, resources=None,
           prefilter=None):
    """``(distances float32 [nq, k], neighbors int64 [nq, k])`` of every query,
    nearest first (for inner product, largest first); -1 past the rows there
    are.  Given ``neighbors`` / ``distances`` arrays are filled and returned.
    """
    from mlxvs_amd import brute_force_knn, brute_force_knn_filtered, hamming_knn

    if not getattr(index, "trained", False):
        raise ValueError("search needs a built index (see brute_force.build)")
    kind = "none" if prefilter is None else getattr(prefilter, "type", None)
    if kind not in ("none", "bitset", "bitmap"):
        raise ValueError(f"prefilter must come from cuvs.neighbors.filters, got {prefilter!r}")
    dist = index._distance
    q = np.asarray(queries)
    if kind != "none":
        words = np.asarray(prefilter.array, dtype=np.uint32)
        fkw = {kind: words}
        if dist.engine is None:
            # {0, 1} rows: squared L2 distance = Hamming distance
            bits = np.unpackbits(index._rows, axis=1).astype(np.float32)
            qbits = np.unpackbits(np.asarray(q, dtype=np.uint8), axis=1).astype(np.float32)
            ids, out = brute_force_knn_filtered(bits, qbits, k, "l2", **fkw)
        else:
            ids, raw = brute_force_knn_filtered(index._rows, q, k, dist.engine, **fkw)
            out = dist.units(raw)
    elif dist.engine is None:
        ids, out = hamming_knn(index._rows, q, k)
    else:
        ids, raw = brute_force_knn(index._rows, q, k, dist.engine)
        out = dist.units(raw)
    ids = ids.astype(np.int64)
    ids[ids < 0] = -1
    out = np.asarray(out, dtype=np.float32)
    if distances is not None:
        distances[...] = out
        out = distances
    if neighbors is not None:
        neighbors[...] = ids
        ids = neighbors
    return out, ids


def save(filename, index, include_dataset=True, resources=None) -> None:
    """Writes ``index`` as a cuVS brute-force file (format 0).

    After the type tag: version, rows, dim, distance type and metric
    argument; a flag and the dataset; a flag and, for the L2 types, the
    rows' squared norms (cosine: their norms), which cuVS reads back
    instead of recomputing them.
    """
    rows = np.asarray(index._rows)
    dist = index._distance
    with open(filename, "wb") as f:
        f.write(type_tag(rows.dtype, 6))
        w = RecordWriter(f)
        for value, dtype in ((FORMAT_VERSION, np.int32), (rows.shape[0], np.uint64),
                             (rows.shape[1], np.uint64), (dist.code, np.int32),
                             (index._metric_arg, np.float32)):
            w.scalar(value, dtype)
        w.scalar(bool(include_dataset), np.bool_)
        if include_dataset:
            w.array(rows)
        w.scalar(dist.norms is not None, np.bool_)
        if dist.norms is not None:
            x = rows.astype(np.float32)
            sq = (x * x).sum(axis=1)
            w.array((sq if dist.norms == "squared" else np.sqrt(sq)).astype(np.float32))


def load(filename, resources=None) -> Index:
    """Reads a brute-force file written by :func:`save` or by cuVS."""
    with open(filename, "rb") as f:
        dtype = read_type_tag(f)
        r = RecordReader(f)
        version = r.scalar()
        if version != FORMAT_VERSION:
            raise ValueError(f"brute-force file format {version} is not read here "
                             f"(expected {FORMAT_VERSION})")
        n, dim, code, metric_arg = r.scalar(), r.scalar(), r.scalar(), r.scalar()
        if not r.scalar():
            raise ValueError("this file was saved without its dataset, which a brute-force "
                             "index cannot do without")
        rows = r.array().astype(dtype, copy=False)
    if rows.shape != (n, dim):
        raise ValueError(f"the dataset record is {rows.shape}, the file says ({n}, {dim})")
    return _index(rows, _distance(int(code)), metric_arg)
