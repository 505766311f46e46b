"""A scikit-learn style front end over the exact k-NN engine.

Mirrors reference python/mlxvs/_neighbors.py:18-96 (``NearestNeighbors``):
``fit(X)`` keeps the rows, ``kneighbors(Q)`` returns NumPy
``(distances, indices)`` nearest first in scikit-learn's units -- Euclidean
distance for ``"euclidean"`` (the square root of the engine's squared L2),
cosine distance ``1 - cos`` for ``"cosine"``, the squared L2 as it is for
``"sqeuclidean"`` / ``"l2"`` -- and int64 indices.  ``kneighbors()`` without
queries answers for the fitted rows themselves with each row's own index
dropped (the single-cluster brute-force self graph).

Only ``algorithm="brute"`` exists here: the reference's ``"nn_descent"``
builds an approximate graph, which is outside this engine.
"""

from __future__ import annotations

import numpy as np

_METRICS = {  # reference python/mlxvs/_neighbors.py:10-15
    "euclidean": "l2",
    "sqeuclidean": "l2",
    "l2": "l2",
    "cosine": "cosine",
}


class NearestNeighbors:
    """Exact nearest neighbours with scikit-learn's interface.

    Args:
        n_neighbors (int): Neighbours per query.
        metric (str): ``"euclidean"``, ``"sqeuclidean"``, ``"l2"`` or
          ``"cosine"``.
        algorithm (str): ``"brute"``.
        n_clusters (int): Accepted for signature compatibility; must be 1.
    """

    def __init__(self, n_neighbors=5, *, metric="euclidean", algorithm="brute", n_clusters=1):
        if metric not in _METRICS:
            names = ", ".join(repr(m) for m in _METRICS)
            raise ValueError(f"unknown metric {metric!r}; one of {names}")
        if algorithm == "nn_descent":
            raise ValueError("algorithm 'nn_descent' (approximate) is not part of this "
                             "engine; use 'brute'")
        if algorithm != "brute":
            raise ValueError("algorithm must be 'brute' or 'nn_descent'")
        self.n_neighbors = n_neighbors
        self.metric = metric
        self.algorithm = algorithm
        self.n_clusters = n_clusters

    def fit(self, X, y=None):
        """Keep the rows ``X [n, d]`` (float16 rows stay float16)."""
        x = np.asarray(X)
        if x.ndim != 2:
            raise ValueError("X must be 2-D [n, d]")
        self._fit_X = np.ascontiguousarray(x)
        self.n_samples_fit_ = x.shape[0]
        self.n_features_in_ = x.shape[1]
        return self

    def kneighbors(self, X=None, n_neighbors=None, return_distance=True):
        """The neighbours of each row of ``X``, or of each fitted row.

        Without ``X`` a row is not its own neighbour, as in scikit-learn.

        Returns:
            ``(distances float32, indices int64)`` ``[nq, n_neighbors]``, or
            only the indices with ``return_distance=False``.
        """
        from mlxvs_amd import all_neighbors, brute_force_knn

        if not hasattr(self, "_fit_X"):
            raise RuntimeError("call fit(X) first")
        k = self.n_neighbors if n_neighbors is None else n_neighbors
        limit = self.n_samples_fit_ - (1 if X is None else 0)
        if not 1 <= k <= limit:
            raise ValueError(f"n_neighbors must be in [1, {limit}], got {k}")
        metric = _METRICS[self.metric]
        if X is None:
            ids, dist = all_neighbors(self._fit_X, k, metric)
        else:
            ids, dist = brute_force_knn(self._fit_X, X, k, metric)
        ids = ids.astype(np.int64)
        if not return_distance:
            return ids
        dist = np.array(dist, dtype=np.float32)
        if self.metric == "euclidean":
            dist = np.sqrt(dist)
        elif self.metric == "cosine":
            dist = 1.0 - dist
        return dist, ids
