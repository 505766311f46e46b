"""cuVS's ``cuvs.neighbors.brute_force`` (build / search / save / load) on the
exact k-NN engine.

The public names and arguments are cuVS's, as the reference's compatibility
module python/mlxvs/cuvs/neighbors/brute_force.py keeps them.  Search runs
the fused k-NN (``brute_force_knn``, or ``hamming_knn`` for bit-packed rows)
and reports cuVS's distance units.  Files are cuVS's brute-force format,
version 0, readable by cuVS's own ``brute_force.load``.

Distance types: ``"sqeuclidean"`` (L2Expanded), ``"euclidean"`` / ``"l2"``
(L2SqrtExpanded), ``"cosine"`` (CosineExpanded), ``"inner_product"`` and
``"bitwise_hamming"`` run the fused kernels; L2Unexpanded and
L2SqrtUnexpanded (by type value) too.  The others the reference's search
computes through ``distance._pairwise`` (python/mlxvs/cuvs/distance.py:
85-151) -- ``"cityblock"`` / ``"l1"``, ``"chebyshev"``, ``"canberra"``,
``"minkowski"`` / ``"lp"`` (``metric_arg`` = p), ``"correlation"``,
``"hellinger"``, ``"braycurtis"``, ``"jensenshannon"``, ``"hamming"``,
``"kl_divergence"``, ``"russellrao"`` -- run ``pairwise_knn``: each query's
rows scored with the metric and selected exactly on the GPU, in one
kernel.  ``"jaccard"`` and ``"dice"`` build, and their search raises
``ValueError``, as the reference's does.  Search returns min(k, n) columns,
as the reference's selection does (``k = min(k, dist.shape[1])``).

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
def _same(d):
    return d


_DISTANCES = (
    _Distance(0, "sqeuclidean", "l2", "squared", lambda d: np.maximum(d, 0)),
    _Distance(1, "euclidean", "l2", "squared", lambda d: np.sqrt(np.maximum(d, 0))),
    _Distance(2, "cosine", "cosine", "plain", lambda s: 1 - s),
    _Distance(4, "l2_unexpanded", "l2", None, lambda d: np.maximum(d, 0)),
    _Distance(5, "l2_sqrt_unexpanded", "l2", None, lambda d: np.sqrt(np.maximum(d, 0))),
    _Distance(6, "inner_product", "inner_product", None, _same),
    _Distance(20, "bitwise_hamming", None, None, _same),
    # the reference's distance._pairwise metrics: pairwise_knn
    _Distance(3, "cityblock", "pairwise", None, _same),
    _Distance(7, "chebyshev", "pairwise", None, _same),
    _Distance(8, "canberra", "pairwise", None, _same),
    _Distance(9, "minkowski", "pairwise", None, _same),
    _Distance(10, "correlation", "pairwise", None, _same),
    _Distance(12, "hellinger", "pairwise", None, _same),
    _Distance(14, "braycurtis", "pairwise", None, _same),
    _Distance(15, "jensenshannon", "pairwise", None, _same),
    _Distance(16, "hamming", "pairwise", None, _same),
    _Distance(17, "kl_divergence", "pairwise", None, _same),
    _Distance(18, "russellrao", "pairwise", None, _same),
    # names the reference builds with but cannot search
    _Distance(11, "jaccard", "unsupported", None, _same),
    _Distance(19, "dice", "unsupported", None, _same),
)
_BY_CODE = {d.code: d for d in _DISTANCES}
_BY_NAME = {d.name: d for d in _DISTANCES if d.code not in (4, 5)}
_BY_NAME["l2"] = _BY_CODE[1]
_BY_NAME["l1"] = _BY_CODE[3]
_BY_NAME["lp"] = _BY_CODE[9]

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
    """``(distances float32 [nq, m], neighbors int64 [nq, m])`` of every
    query, m = min(k, rows), nearest first (for inner product, largest
    first); -1 past the rows a prefilter allows.  Given ``neighbors`` /
    ``distances`` arrays are filled and returned.  k at most 256.
    """
    from mlxvs_amd import brute_force_knn, brute_force_knn_filtered, hamming_knn, pairwise_knn

    if not getattr(index, "trained", False):
        raise ValueError("search needs a built index (see brute_force.build)")
    kind = "none" if prefilter is None else getattr(prefilter, "type", None)
    if kind not in ("none", "bitset", "bitmap"):
        raise ValueError(f"prefilter must come from cuvs.neighbors.filters, got {prefilter!r}")
    dist = index._distance
    if dist.engine == "unsupported":
        raise ValueError(f"metric {dist.name} is not supported")
    q = np.asarray(queries)
    n = len(index)
    # the reference selects min(k, n) per query (its select_k)
    k = min(int(k), n)
    if k <= 0:
        out = np.zeros((q.shape[0], 0), dtype=np.float32)
        ids = np.zeros((q.shape[0], 0), dtype=np.int64)
    elif dist.engine == "pairwise":
        fkw = {} if kind == "none" else {kind: np.asarray(prefilter.array, dtype=np.uint32)}
        ids, out = pairwise_knn(index._rows, q, k, dist.code, index._metric_arg, **fkw)
        # as the reference's pairwise branch: an infinite distance is no neighbor
        ids[np.isinf(out)] = -1
    elif kind != "none":
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
