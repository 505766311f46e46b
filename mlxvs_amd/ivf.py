"""IVF-Flat over the exact k-NN engine: the list scan and its finish.

Mirrors the reference's IVF-Flat surface (python/mlxvs/_ivf.py:12-140,
python/bindings.cpp:283-361, src/ivf.cpp:236-416):

* :func:`ivf_flat_search` -- the hot path: the ``n_probes`` nearest centers
  of each query (the fused brute-force k-NN), then every probed list scanned
  exactly on the GPU (``mlxvs_ivf_flat_search``: per-lane top-k lists fused
  into the MFMA tiles for k <= 16, candidate buffers and an exact radix
  select otherwise).  Given the same index it returns the reference's
  neighbours: best score first, then the earlier probe, then the earlier row
  of the list.
* :func:`ivf_flat_build` / :func:`ivf_flat_extend` and :class:`IvfFlatIndex`
  -- building and growing an index.  The lists come from Lloyd's k-means
  whose assignment step is :func:`mlxvs_amd.kmeans_predict` on the GPU;
  initialisation (a seeded sample of distinct rows) and the center update
  (a mean per list) run in NumPy, so an index built here clusters like the
  reference's but not identically (its start is k-means++ on an mt19937
  stream).  Rows of a list keep their input order.
* :meth:`IvfFlatIndex.save` / :meth:`IvfFlatIndex.load` -- the reference's
  ``.safetensors`` layout (tensors centers, data, indices, offsets; metadata
  format ``mlxvs.ivf_flat``, version ``1``, metric).
"""

from __future__ import annotations

import numpy as np

__all__ = ["IvfFlatIndex", "ivf_flat_build", "ivf_flat_extend", "ivf_flat_search"]

_FORMAT = "mlxvs.ivf_flat"
_METRICS = ("l2", "cosine", "inner_product")


def _metric_name(metric) -> str:
    from mlxvs_amd import Metric

    name = metric.name if isinstance(metric, Metric) else metric
    if isinstance(name, (int, np.integer)):
        name = Metric(int(name)).name
    if name not in _METRICS:
        raise ValueError(f"unknown metric {metric!r}")
    return name


def _unit_rows(x: np.ndarray) -> np.ndarray:
    # reference src/ivf.cpp:100-103 (x / max(|x|, 1e-30)), in float32
    n = np.sqrt(np.sum(x * x, axis=1, keepdims=True, dtype=np.float32))
    return (x / np.maximum(n, np.float32(1e-30))).astype(np.float32)


def ivf_flat_search(centers, data, indices, offsets, metric, queries, k, *, n_probes=20,
                    stream=None):
    """The k nearest indexed rows of every query (reference
    python/bindings.cpp:310-337).  Returns ``(ids int32 [nq, k], distances
    float32 [nq, k])`` as ``brute_force_knn``; -1 / +-inf where the scanned
    lists hold fewer than k rows."""
    from mlxvs_amd import Metric, _check, _L, _ptr

    op = "mlxvs::ivf_flat_search"
    m = Metric[_metric_name(metric)]
    c = np.ascontiguousarray(centers, dtype=np.float32)
    x = np.ascontiguousarray(data, dtype=np.float32)
    ix = np.ascontiguousarray(indices, dtype=np.int32)
    off = np.ascontiguousarray(offsets, dtype=np.int32)
    q = np.asarray(queries)
    if q.ndim == 1:
        q = q[None]
    if c.ndim != 2 or x.ndim != 2 or q.ndim != 2:
        raise ValueError(f"[{op}] centers, data and queries must be 2-D.")
    if x.shape[1] != c.shape[1] or ix.shape != (x.shape[0],) or off.shape != (c.shape[0] + 1,):
        raise ValueError(f"[{op}] the index arrays do not fit together.")
    if q.shape[1] != c.shape[1]:
        raise ValueError(f"[{op}] queries must have the index's columns.")
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = int(k)
    ids = np.empty((q.shape[0], max(k, 0)), np.int32)
    dist = np.empty((q.shape[0], max(k, 0)), np.float32)
    _check(_L().mlxvs_ivf_flat_search(_ptr(c), c.shape[0], _ptr(x), x.shape[0], _ptr(ix), _ptr(off),
                                      c.shape[1], int(m), _ptr(q), q.shape[0], k, int(n_probes),
                                      _ptr(ids), _ptr(dist)))
    return ids, dist


def _group(rows: np.ndarray, ids: np.ndarray, labels: np.ndarray, lists: int):
    order = np.argsort(labels, kind="stable")
    counts = np.bincount(labels, minlength=lists)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return (np.ascontiguousarray(rows[order], dtype=np.float32),
            np.ascontiguousarray(ids[order], dtype=np.int32), offsets)


def ivf_flat_build(rows, metric="l2", *, n_lists=1024, kmeans_n_iters=20,
                   kmeans_trainset_fraction=0.5, seed=42):
    """An IVF-Flat index of ``rows [n, d]`` (reference
    python/bindings.cpp:283-308, src/ivf.cpp:236-278): returns ``(centers,
    data, indices, offsets)``; ids are row numbers."""
    from mlxvs_amd import kmeans_predict

    op = "mlxvs::ivf_flat_build"
    name = _metric_name(metric)
    x = np.asarray(rows)
    if x.ndim != 2:
        raise ValueError(f"[{op}] rows must be 2-D [n, d].")
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[0]
    if not 1 <= n_lists <= n:
        raise ValueError(f"[{op}] n_lists must be in [1, number of rows].")
    if not 0 < kmeans_trainset_fraction <= 1:
        raise ValueError(f"[{op}] kmeans_trainset_fraction must be in (0, 1].")
    if name == "cosine":
        x = _unit_rows(x)
    rng = np.random.default_rng(seed)
    sample_n = min(n, max(64 * n_lists, int(n * kmeans_trainset_fraction)))
    sample = x[np.sort(rng.choice(n, sample_n, replace=False))] if sample_n < n else x
    centers = sample[np.sort(rng.choice(sample.shape[0], n_lists, replace=False))].copy()
    for _ in range(int(kmeans_n_iters)):
        lab = kmeans_predict(sample, centers)[:, 0]
        counts = np.bincount(lab, minlength=n_lists)
        order = np.argsort(lab, kind="stable")
        starts = np.concatenate([[0], np.cumsum(counts)[:-1]])
        sums = np.zeros(centers.shape, np.float64)
        nz = counts > 0
        sums[nz] = np.add.reduceat(sample[order].astype(np.float64), starts[nz], axis=0)
        empty = ~nz
        centers = np.where(empty[:, None], centers,
                           sums / np.maximum(counts, 1)[:, None]).astype(np.float32)
        if empty.any():  # an empty list restarts at a random sample row
            centers[empty] = sample[rng.choice(sample.shape[0], int(empty.sum()))]
    labels = kmeans_predict(x, centers)[:, 0]
    data, indices, offsets = _group(x, np.arange(n, dtype=np.int32), labels, n_lists)
    return centers, data, indices, offsets


def ivf_flat_extend(centers, data, indices, offsets, metric, new_rows, new_ids=None):
    """The index with ``new_rows`` added to the lists of their nearest centers
    (reference src/ivf.cpp:280-318); ids ``new_ids``, or the largest id plus
    1, 2, ...  Returns ``(centers, data, indices, offsets)``."""
    from mlxvs_amd import kmeans_predict

    op = "mlxvs::ivf_flat_extend"
    name = _metric_name(metric)
    c = np.asarray(centers, dtype=np.float32)
    x = np.asarray(data, dtype=np.float32)
    ix = np.asarray(indices, dtype=np.int32)
    off = np.asarray(offsets, dtype=np.int32)
    r = np.asarray(new_rows)
    if r.ndim == 1:
        r = r[None]
    r = np.ascontiguousarray(r, dtype=np.float32)
    if r.shape[1] != x.shape[1]:
        raise ValueError(f"[{op}] new_rows must have the index's columns.")
    m = r.shape[0]
    if new_ids is not None:
        new_ids = np.asarray(new_ids).astype(np.int32)
        if new_ids.shape != (m,):
            raise ValueError(f"[{op}] new_ids must hold one id per new row.")
    else:
        top = int(ix.max()) if ix.size else -1
        new_ids = np.arange(top + 1, top + 1 + m, dtype=np.int32)
    if name == "cosine":
        r = _unit_rows(r)
    lists = c.shape[0]
    old_labels = np.repeat(np.arange(lists), np.diff(off))
    new_labels = kmeans_predict(r, c)[:, 0] if m else np.zeros(0, np.int64)
    data2, ids2, off2 = _group(np.concatenate([x, r]), np.concatenate([ix, new_ids]),
                               np.concatenate([old_labels, new_labels]).astype(np.int64), lists)
    return c, data2, ids2, off2


class IvfFlatIndex:
    """An IVF-Flat index (reference python/mlxvs/_ivf.py:12-140)::

        index = mlxvs_amd.IvfFlatIndex.build(vectors, n_lists=1024)
        ids, dist = index.search(queries, k=10, n_probes=20)
        index.extend(more_vectors)
        index.save("ivf.safetensors")
    """

    def __init__(self, centers, data, indices, offsets, metric):
        self._metric = _metric_name(metric)
        self._centers = np.ascontiguousarray(centers, dtype=np.float32)
        self._data = np.ascontiguousarray(data, dtype=np.float32)
        self._indices = np.ascontiguousarray(indices, dtype=np.int32)
        self._offsets = np.ascontiguousarray(offsets, dtype=np.int32)

    @classmethod
    def build(cls, rows, n_lists=1024, metric="l2", **kwargs):
        return cls(*ivf_flat_build(rows, metric, n_lists=n_lists, **kwargs), metric)

    def search(self, queries, k=10, n_probes=20):
        return ivf_flat_search(self._centers, self._data, self._indices, self._offsets,
                               self._metric, queries, k, n_probes=n_probes)

    def extend(self, rows, ids=None):
        parts = ivf_flat_extend(self._centers, self._data, self._indices, self._offsets,
                                self._metric, rows, ids)
        self._centers, self._data, self._indices, self._offsets = parts
        return self

    def save(self, path):
        """Saves the index to a ``.safetensors`` file."""
        from safetensors.numpy import save_file

        path = str(path)
        if not path.endswith(".safetensors"):
            raise ValueError("the file name must end in .safetensors")
        save_file({"centers": self._centers, "data": self._data, "indices": self._indices,
                   "offsets": self._offsets}, path,
                  metadata={"format": _FORMAT, "version": "1", "metric": self._metric})

    @classmethod
    def load(cls, path):
        """Loads an index saved by :meth:`save` (or by the reference)."""
        from safetensors import safe_open

        with safe_open(str(path), framework="np") as f:
            meta = f.metadata() or {}
            if meta.get("format") != _FORMAT:
                raise ValueError(f"{path} is not a saved mlxvs IvfFlatIndex")
            arrays = {key: f.get_tensor(key) for key in ("centers", "data", "indices", "offsets")}
        return cls(arrays["centers"], arrays["data"], arrays["indices"], arrays["offsets"],
                   meta["metric"])

    def __len__(self):
        return self._data.shape[0]

    @property
    def centers(self):
        return self._centers

    @property
    def n_lists(self):
        return self._centers.shape[0]

    @property
    def metric(self):
        return self._metric
