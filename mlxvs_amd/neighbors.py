"""scikit-learn's ``NearestNeighbors`` interface over the exact k-NN engine.

The class keeps the public surface of reference python/mlxvs/_neighbors.py
(constructor arguments, ``fit``, ``kneighbors``, the fitted attributes and
scikit-learn's distance units).  Each metric name resolves to the metric
the engine computes plus a conversion into scikit-learn's units:

=============  ==============  ==========================================
name           engine metric   reported distance
=============  ==============  ==========================================
euclidean      squared L2      its square root
sqeuclidean    squared L2      as computed
l2             squared L2      as computed
cosine         cosine sim.     1 - similarity
=============  ==============  ==========================================

``kneighbors()`` without queries asks for the fitted rows' own neighbours
and leaves every row out of its own list (the single-cluster self graph of
``all_neighbors``).  The engine is exact only, so ``algorithm`` is
``"brute"``; the reference's approximate ``"nn_descent"`` graph is refused.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional

import numpy as np


@dataclass(frozen=True)
class _Units:
    engine: str                                           # engine metric name
    convert: Optional[Callable[[np.ndarray], np.ndarray]]  # None: as computed


_UNITS = {
    "euclidean": _Units("l2", np.sqrt),
    "sqeuclidean": _Units("l2", None),
    "l2": _Units("l2", None),
    "cosine": _Units("cosine", lambda sim: 1.0 - sim),
}


def _units_of(metric: str) -> _Units:
    try:
        return _UNITS[metric]
    except (KeyError, TypeError):
        known = ", ".join(_UNITS)
        raise ValueError(f"unknown metric {metric!r} for NearestNeighbors "
                         f"(known: {known})") from None


def _check_algorithm(algorithm: str) -> None:
    if algorithm == "brute":
        return
    if algorithm == "nn_descent":
        raise ValueError("algorithm 'nn_descent' builds an approximate graph, which this "
                         "exact engine does not provide; use algorithm='brute'")
    raise ValueError(f"algorithm {algorithm!r} is not available; this engine searches "
                     "with algorithm='brute'")


class NearestNeighbors:
    """Exact k nearest neighbours, scikit-learn style.

    Args:
        n_neighbors (int): Neighbours returned per query by default.
        metric (str): ``"euclidean"``, ``"sqeuclidean"``, ``"l2"`` or
          ``"cosine"``.
        algorithm (str): ``"brute"``.
        n_clusters (int): Kept for signature compatibility (the reference
          uses it with NN-Descent only).
    """

    def __init__(self, n_neighbors=5, *, metric="euclidean", algorithm="brute", n_clusters=1):
        self._units = _units_of(metric)
        _check_algorithm(algorithm)
        self.n_neighbors = n_neighbors
        self.metric = metric
        self.algorithm = algorithm
        self.n_clusters = n_clusters
        self._rows: Optional[np.ndarray] = None

    def fit(self, X, y=None):
        """Remember the rows ``X [n, d]`` (float16 rows are kept as float16
        and searched on the fp16 MFMA path); returns ``self``."""
        rows = np.asarray(X)
        if rows.ndim != 2:
            raise ValueError(f"fit expects a 2-D array of rows [n, d]; got shape {rows.shape}")
        self._rows = np.ascontiguousarray(rows)
        self.n_samples_fit_, self.n_features_in_ = rows.shape
        return self

    def _neighbours_wanted(self, n_neighbors, self_query: bool) -> int:
        k = self.n_neighbors if n_neighbors is None else int(n_neighbors)
        # a fitted row is not a candidate in its own list
        most = self.n_samples_fit_ - (1 if self_query else 0)
        if not 1 <= k <= most:
            whose = "each fitted row has" if self_query else "the fitted data has"
            raise ValueError(f"n_neighbors={k} is out of range: {whose} {most} candidate rows "
                             f"(1 <= n_neighbors <= {most})")
        return k

    def kneighbors(self, X=None, n_neighbors=None, return_distance=True):
        """Neighbours of the rows of ``X`` -- or, without ``X``, of every
        fitted row, excluding the row itself -- nearest first.

        Returns ``(distances float32, indices int64)`` of shape
        ``[queries, n_neighbors]``, or only the indices when
        ``return_distance`` is false.
        """
        from mlxvs_amd import all_neighbors, brute_force_knn

        if self._rows is None:
            raise RuntimeError("this NearestNeighbors is not fitted yet: call fit(X) first")
        k = self._neighbours_wanted(n_neighbors, X is None)
        if X is None:
            ids, raw = all_neighbors(self._rows, k, self._units.engine)
        else:
            ids, raw = brute_force_knn(self._rows, X, k, self._units.engine)
        indices = np.asarray(ids, dtype=np.int64)
        if not return_distance:
            return indices
        dist = np.asarray(raw, dtype=np.float32)
        if self._units.convert is not None:
            dist = self._units.convert(dist).astype(np.float32, copy=False)
        return dist, indices
