"""Exact k-nearest-neighbour search on the AMD Instinct MI355X (gfx950).

Drop-in for the brute-force slice of mlxvs (mikepapadim/mlxvs 0.16.1):

    import mlxvs_amd as mlxvs
    ids, dist = mlxvs.brute_force_knn(base, queries, 10, "l2")
    ids, dist = mlxvs.hamming_knn(codes, qcodes, 100)

Same names, arguments, metric names / enum values and error types as the
reference's Python API (python/mlxvs/__init__.py:56-115,
python/bindings.cpp:37-75, 681-709); results are NumPy arrays instead of
mlx.core arrays (``numpy.asarray`` of an mlx array gives the same values).
The work runs in libmlxvs_c.so, a C-ABI library of hand-written HIP kernels;
importing this package fails when the library has not been built
(``python -m mlxvs_amd.build``): the first call then raises ImportError, and
every call raises RuntimeError when no GPU is present.
"""

from __future__ import annotations

import ctypes
import enum
from pathlib import Path

import numpy as np

__all__ = [
    "IvfFlatIndex",
    "Metric",
    "NearestNeighbors",
    "all_neighbors",
    "brute_force_knn",
    "brute_force_knn_filtered",
    "hamming_knn",
    "ivf_flat_build",
    "ivf_flat_extend",
    "ivf_flat_search",
    "kmeans_predict",
    "library_path",
    "pairwise_knn",
    "topk_merge",
    "topk_merge_device",
]
__version__ = "0.16.1"

# the in-tree build (python -m mlxvs_amd.build)
_LIB_PATH = Path(__file__).resolve().parent / "libmlxvs_c.so"

# mlxvs_status (include/mlxvs/mlxvs_c.h)
OK, INVALID_ARGUMENT, IO_ERROR, INTERNAL = 0, 1, 2, 3


def library_path() -> str:
    return str(_LIB_PATH)


def _load():
    if not _LIB_PATH.exists():
        raise ImportError(
            f"{_LIB_PATH} is missing: build it with `python -m mlxvs_amd.build` "
            "(the engine has no CPU fallback)")
    lib = ctypes.CDLL(str(_LIB_PATH))
    i64, i32, vp = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
    sig = {
        "mlxvs_brute_force_knn": [vp, i64, vp, i64, i32, i32, ctypes.c_int, vp, vp],
        "mlxvs_brute_force_knn_f16": [vp, i64, vp, i64, i32, i32, ctypes.c_int, vp, vp],
        "mlxvs_hamming_knn": [vp, i64, vp, i64, i32, i32, vp, vp],
        "mlxvs_knn_self_graph": [vp, i64, i32, i32, i32, ctypes.c_int, vp, vp],
        "mlxvs_kmeans_predict": [vp, i64, vp, i64, i32, i32, i32, vp],
        "mlxvs_ivf_flat_search": [vp, i64, vp, i64, vp, vp, i32, ctypes.c_int, vp, i64, i32, i32,
                                  vp, vp],
        "mlxvs_ivf_flat_search_device": [vp, i64, vp, i64, vp, vp, i32, ctypes.c_int, vp, i64,
                                         i32, i32, vp, vp, vp],
        "mlxvs_brute_force_knn_device": [vp, i64, vp, i64, i32, i32, i32, ctypes.c_int, vp, vp, vp],
        "mlxvs_brute_force_knn_device_noalloc": [vp, i64, vp, i64, i32, i32, i32, ctypes.c_int,
                                                 vp, vp, vp],
        "mlxvs_brute_force_knn_filtered": [vp, i64, vp, i64, i32, i32, i32, ctypes.c_int, vp, i32,
                                           vp, vp, vp],
        "mlxvs_brute_force_knn_filtered_device": [vp, i64, vp, i64, i32, i32, i32, ctypes.c_int,
                                                  vp, i32, vp, vp, vp],
        "mlxvs_pairwise_knn": [vp, i64, vp, i64, i32, i32, i32, ctypes.c_float, vp, i32, vp, vp,
                               vp],
        "mlxvs_hamming_knn_device": [vp, i64, vp, i64, i32, i32, vp, vp, vp],
        "mlxvs_knn_self_graph_device": [vp, i64, i32, i32, i32, ctypes.c_int, vp, vp, vp],
        "mlxvs_topk_merge": [vp, i64, i64, vp, vp, i32, i32, i32, vp, vp],
        "mlxvs_topk_merge_device": [vp, i64, i64, vp, vp, i32, i32, i32, vp, vp, vp],
        "mlxvs_brute_force_knn_on_stream": [vp, i64, vp, i64, i32, i32, i32, ctypes.c_int, vp,
                                            vp, vp],
        "mlxvs_hamming_knn_on_stream": [vp, i64, vp, i64, i32, i32, vp, vp, vp],
        "mlxvs_kmeans_predict_on_stream": [vp, i64, vp, i64, i32, i32, i32, vp, vp],
        "mlxvs_topk_merge_on_stream": [vp, i64, i64, vp, vp, i32, i32, i32, vp, vp, vp],
        "mlxvs_release_workspace": [],
        "mlxvs_profile": [ctypes.c_int],
        "mlxvs_profile_report": [ctypes.c_char_p, i64],
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.mlxvs_last_error.restype = ctypes.c_char_p
    lib.mlxvs_last_error.argtypes = []
    lib.mlxvs_version.restype = ctypes.c_char_p
    lib.mlxvs_version.argtypes = []
    return lib


_LIB = None


def _L():
    """The loaded library (loaded on first use, so that the pure-Python parts
    of the package -- synth -- import without it)."""
    global _LIB
    if _LIB is None:
        _LIB = _load()
    return _LIB


def _check(rc: int) -> None:
    if rc == OK:
        return
    msg = _L().mlxvs_last_error().decode()
    if rc == INVALID_ARGUMENT:
        raise ValueError(msg)
    raise RuntimeError(msg)


class Metric(enum.IntEnum):
    """How two rows compare (values of reference include/mlxvs/mlxvs_c.h:38-45)."""

    inner_product = 0
    l2 = 1
    cosine = 2


def _metric(metric) -> Metric:
    # reference python/mlxvs/__init__.py:80-87, 102-103
    if isinstance(metric, str):
        try:
            return Metric[metric]
        except KeyError:
            names = ", ".join(repr(n) for n in Metric.__members__)
            raise ValueError(f"unknown Metric {metric!r}; one of {names}") from None
    return Metric(int(metric))


def _rows(x, name: str, op: str) -> np.ndarray:
    """2-D real rows as a C-contiguous array (reference src/utils.h:18-29)."""
    a = np.asarray(x)
    if a.ndim != 2:
        raise ValueError(f"[{op}] {name} must be 2-D [n, d].")
    if a.dtype == np.bool_ or np.iscomplexobj(a) or not np.issubdtype(a.dtype, np.number):
        raise ValueError(f"[{op}] {name} must be real numbers.")
    return a


def _host_stream(stream, op: str):
    """The hipStream_t a host-array call runs on (None: the null stream).

    Takes what the reference's ``stream=`` takes the place of here: a
    hipStream_t handle as an int or ``ctypes.c_void_p``, or an object that
    carries one (``.cuda_stream``, as torch.cuda.Stream, or ``.handle``).
    The call enqueues its copies and kernels on that stream and waits for
    it before returning (reference python/bindings.cpp:55, 125)."""
    if stream is None:
        return None
    h = stream
    for attr in ("cuda_stream", "handle"):
        if hasattr(h, attr):
            h = getattr(h, attr)
            break
    if isinstance(h, ctypes.c_void_p):
        h = h.value or 0
    if isinstance(h, bool) or not isinstance(h, int) or h < 0:
        raise ValueError(f"[{op}] stream must be a hipStream_t handle (int), or None.")
    return h or None


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def brute_force_knn(base, queries, k, metric=Metric.l2, *, tile_rows=65536, stream=None):
    """Exact k-nearest neighbours of every query among the base rows.

    Mirrors reference python/bindings.cpp:37-75.  ``base`` [n, d] and
    ``queries`` [nq, d] take any real dtype and are computed in float32;
    float16 inputs (both) are multiplied on the fp16 MFMA units with float32
    accumulation, which forms the same products as float32.  Returns
    ``(ids int32 [nq, k], distances float32 [nq, k])``, nearest first:
    squared L2 ascending, otherwise similarity descending; -1 / +-inf where
    fewer than k rows exist.  ``tile_rows`` is accepted for compatibility
    (the result does not depend on it).  ``stream``: a hipStream_t handle
    (int, or an object with ``.cuda_stream``) the copies and kernels run on;
    the call waits for that stream before returning.
    """
    op = "mlxvs::brute_force_knn"
    st = _host_stream(stream, op)
    b = _rows(base, "base", op)
    q = _rows(queries, "queries", op)
    if b.shape[1] != q.shape[1]:
        raise ValueError(f"[{op}] base and queries must have the same number of columns.")
    m = _metric(metric)
    k = int(k)
    nq = q.shape[0]
    f16 = b.dtype == np.float16 and q.dtype == np.float16
    if f16:
        b = np.ascontiguousarray(b)
        q = np.ascontiguousarray(q)
        fn = _L().mlxvs_brute_force_knn_f16
    else:
        b = np.ascontiguousarray(b, dtype=np.float32)
        q = np.ascontiguousarray(q, dtype=np.float32)
        fn = _L().mlxvs_brute_force_knn
    ids = np.empty((nq, max(k, 0)), dtype=np.int32)
    dist = np.empty((nq, max(k, 0)), dtype=np.float32)
    if st is None:
        _check(fn(_ptr(b), b.shape[0], _ptr(q), nq, b.shape[1], k, int(m), _ptr(ids),
                  _ptr(dist)))
    else:
        _check(_L().mlxvs_brute_force_knn_on_stream(_ptr(b), b.shape[0], _ptr(q), nq,
                                                    b.shape[1], int(f16), k, int(m), _ptr(ids),
                                                    _ptr(dist), st))
    return ids, dist


# prefilter kinds (include/mlxvs/mlxvs_c.h MLXVS_FILTER_*)
FILTER_NONE, FILTER_BITSET, FILTER_BITMAP = 0, 1, 2


def _filter_words(mask, count: int, op: str) -> np.ndarray:
    """Filter words: a bool mask packed little-endian into uint32 words (as
    cuVS's filters pack it, reference python/mlxvs/cuvs/neighbors/
    filters.py:31-37), or uint32 words as they are; at least ceil(count / 32)
    of them."""
    a = np.asarray(mask)
    if a.dtype == np.bool_:
        b = np.packbits(a.ravel(), bitorder="little")
        a = np.pad(b, (0, -len(b) % 4)).view(np.uint32)
    elif a.dtype != np.uint32:
        raise ValueError(f"[{op}] a filter is a bool mask or uint32 words, not {a.dtype}.")
    a = np.ascontiguousarray(a.ravel())
    if len(a) < (count + 31) // 32:
        raise ValueError(f"[{op}] the filter has {len(a)} words; {(count + 31) // 32} needed.")
    return a


def brute_force_knn_filtered(base, queries, k, metric=Metric.l2, *, bitset=None, bitmap=None,
                             stream=None):
    """brute_force_knn over the rows a prefilter allows (an extension: the
    reference filters only in cuvs.neighbors.brute_force.search,
    python/mlxvs/cuvs/neighbors/brute_force.py:97-136).

    ``bitset``: the rows any query may return, a bool [n] mask or uint32
    words (bit i % 32 of word i / 32).  ``bitmap``: per query, a bool
    [nq, n] mask or uint32 words of nq * n bits, row-major, not padded per
    query.  At most one of them.  Returns ``(ids int32 [nq, k], distances
    float32 [nq, k])`` as brute_force_knn, ids numbering all rows; -1 / +-inf
    past the allowed rows there are.  The filter is applied inside the fused
    select.  ``stream``: as for brute_force_knn.
    """
    op = "mlxvs::brute_force_knn_filtered"
    st = _host_stream(stream, op)
    b = _rows(base, "base", op)
    q = _rows(queries, "queries", op)
    if b.shape[1] != q.shape[1]:
        raise ValueError(f"[{op}] base and queries must have the same number of columns.")
    if bitset is not None and bitmap is not None:
        raise ValueError(f"[{op}] give a bitset or a bitmap, not both.")
    m = _metric(metric)
    k = int(k)
    n, nq = b.shape[0], q.shape[0]
    kind, words = FILTER_NONE, None
    if bitset is not None:
        kind, words = FILTER_BITSET, _filter_words(bitset, n, op)
    elif bitmap is not None:
        bm = np.asarray(bitmap)
        if bm.dtype == np.bool_ and bm.shape != (nq, n):
            raise ValueError(f"[{op}] a bool bitmap is [nq, n] = [{nq}, {n}].")
        kind, words = FILTER_BITMAP, _filter_words(bm, nq * n, op)
    f16 = b.dtype == np.float16 and q.dtype == np.float16
    dt = np.float16 if f16 else np.float32
    b = np.ascontiguousarray(b, dtype=dt)
    q = np.ascontiguousarray(q, dtype=dt)
    ids = np.empty((nq, max(k, 0)), dtype=np.int32)
    dist = np.empty((nq, max(k, 0)), dtype=np.float32)
    _check(_L().mlxvs_brute_force_knn_filtered(
        _ptr(b), n, _ptr(q), nq, b.shape[1], int(f16), k, int(m),
        None if words is None else _ptr(words), kind, _ptr(ids), _ptr(dist), st))
    return ids, dist


# cuVS DistanceType values pairwise_knn computes (reference
# python/mlxvs/cuvs/distance.py:12-32)
PAIRWISE_DISTANCES = {
    "l1": 3, "cityblock": 3, "chebyshev": 7, "canberra": 8, "lp": 9, "minkowski": 9,
    "correlation": 10, "hellinger": 12, "braycurtis": 14, "jensenshannon": 15, "hamming": 16,
    "kl_divergence": 17, "russellrao": 18,
}


def pairwise_knn(base, queries, k, distance, metric_arg=2.0, *, bitset=None, bitmap=None,
                 stream=None):
    """Exact k-NN under one of cuVS's distances the fused kernels do not
    serve (an extension: the reference computes them in Python for
    cuvs.neighbors.brute_force.search, python/mlxvs/cuvs/distance.py:85-151,
    brute_force.py:118-136).

    ``distance``: a name of PAIRWISE_DISTANCES or its cuVS DistanceType value;
    ``metric_arg``: the exponent of ``"minkowski"`` / ``"lp"``.  Rows are
    taken as float32.  ``bitset`` / ``bitmap``: as brute_force_knn_filtered.
    Returns ``(ids int32 [nq, k], distances float32 [nq, k])``, nearest first,
    lower id first among equal distances; -1 / +inf past the rows a query may
    return.  ``stream``: as for brute_force_knn.
    """
    op = "mlxvs::pairwise_knn"
    st = _host_stream(stream, op)
    if isinstance(distance, str):
        if distance not in PAIRWISE_DISTANCES:
            raise ValueError(f"[{op}] distance {distance!r} is not one of "
                             f"{sorted(PAIRWISE_DISTANCES)}.")
        code = PAIRWISE_DISTANCES[distance]
    else:
        code = int(distance)
    b = np.ascontiguousarray(_rows(base, "base", op), dtype=np.float32)
    q = np.ascontiguousarray(_rows(queries, "queries", op), dtype=np.float32)
    if b.shape[1] != q.shape[1]:
        raise ValueError(f"[{op}] base and queries must have the same number of columns.")
    if bitset is not None and bitmap is not None:
        raise ValueError(f"[{op}] give a bitset or a bitmap, not both.")
    k = int(k)
    n, nq = b.shape[0], q.shape[0]
    kind, words = FILTER_NONE, None
    if bitset is not None:
        kind, words = FILTER_BITSET, _filter_words(bitset, n, op)
    elif bitmap is not None:
        bm = np.asarray(bitmap)
        if bm.dtype == np.bool_ and bm.shape != (nq, n):
            raise ValueError(f"[{op}] a bool bitmap is [nq, n] = [{nq}, {n}].")
        kind, words = FILTER_BITMAP, _filter_words(bm, nq * n, op)
    ids = np.empty((nq, max(k, 0)), dtype=np.int32)
    dist = np.empty((nq, max(k, 0)), dtype=np.float32)
    _check(_L().mlxvs_pairwise_knn(
        _ptr(b), n, _ptr(q), nq, b.shape[1], k, code, float(metric_arg),
        None if words is None else _ptr(words), kind, _ptr(ids), _ptr(dist), st))
    return ids, dist


def hamming_knn(rows, queries, k, *, stream=None):
    """Exact k-NN of bit-packed uint8 rows by Hamming distance.

    Mirrors reference python/bindings.cpp:681-709 (src/ivf.cpp:1343-1403):
    ``rows`` uint8 [n, bytes] (as numpy.packbits), ``queries`` uint8
    [nq, bytes], k <= 256.  Returns ``(ids int32, distances float32)``
    [nq, k], nearest first, lowest id first among equal distances.
    ``stream``: as for brute_force_knn.
    """
    op = "mlxvs::hamming_knn"
    st = _host_stream(stream, op)
    r = np.asarray(rows)
    q = np.asarray(queries)
    if r.ndim != 2 or r.dtype != np.uint8 or q.ndim != 2 or q.dtype != np.uint8:
        raise ValueError(f"[{op}] rows must be bit-packed uint8 [n, bytes].")
    if r.shape[1] != q.shape[1]:
        raise ValueError(f"[{op}] queries must have the rows' bytes.")
    r = np.ascontiguousarray(r)
    q = np.ascontiguousarray(q)
    k = int(k)
    nq = q.shape[0]
    ids = np.empty((nq, max(k, 0)), dtype=np.int32)
    dist = np.empty((nq, max(k, 0)), dtype=np.float32)
    if st is None:
        _check(_L().mlxvs_hamming_knn(_ptr(r), r.shape[0], _ptr(q), nq, r.shape[1], k,
                                      _ptr(ids), _ptr(dist)))
    else:
        _check(_L().mlxvs_hamming_knn_on_stream(_ptr(r), r.shape[0], _ptr(q), nq, r.shape[1],
                                                k, _ptr(ids), _ptr(dist), st))
    return ids, dist


def all_neighbors(rows, k, metric=Metric.l2, *, algo="brute_force", n_clusters=1, **kwargs):
    """The k-NN graph of ``rows`` against themselves, each row's own id dropped.

    The single-cluster brute-force route of reference mlxvs.all_neighbors
    (python/mlxvs/__init__.py:224-230, src/all_neighbors.cpp:250-263,
    56-95): ``algo="brute_force"`` with one cluster only.  float16 rows are
    multiplied on the fp16 MFMA units.  Returns ``(ids int32 [n, k],
    distances float32 [n, k])``.
    """
    op = "mlxvs::all_neighbors"
    if algo not in ("brute_force",) or n_clusters not in (0, 1):
        raise ValueError(f"[{op}] only algo='brute_force' with one cluster is supported")
    x = _rows(rows, "rows", op)
    m = _metric(metric)
    if x.dtype == np.float16:
        x = np.ascontiguousarray(x)
        f16 = 1
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
        f16 = 0
    k = int(k)
    n = x.shape[0]
    ids = np.empty((n, max(k, 0)), dtype=np.int32)
    dist = np.empty((n, max(k, 0)), dtype=np.float32)
    _check(_L().mlxvs_knn_self_graph(_ptr(x), n, x.shape[1], f16, k, int(m), _ptr(ids),
                                     _ptr(dist)))
    return ids, dist


def kmeans_predict(x, centroids, m=1, *, tile_rows=65536, stream=None):
    """The ``m`` nearest centroids of every row, nearest first.

    Mirrors reference python/bindings.cpp:111-139 (src/kmeans.cpp:136-169):
    ``x`` [n, d] and ``centroids`` [c, d] of any real dtype (float16 when
    both are, else float32), ``1 <= m <= clusters`` (at most 256 here).
    Squared L2 with the lowest centroid index first among equal distances
    (the reference's argmin for m = 1).  Returns int32 ``[n, m]``.
    ``stream``: as for brute_force_knn.
    """
    op = "mlxvs::kmeans_predict"
    st = _host_stream(stream, op)
    xa = _rows(x, "x", op)
    ca = _rows(centroids, "centroids", op)
    if xa.shape[1] != ca.shape[1]:
        raise ValueError(f"[{op}] x and centroids must have the same number of columns.")
    m = int(m)
    if xa.dtype == np.float16 and ca.dtype == np.float16:
        xa, ca, f16 = np.ascontiguousarray(xa), np.ascontiguousarray(ca), 1
    else:
        xa = np.ascontiguousarray(xa, dtype=np.float32)
        ca = np.ascontiguousarray(ca, dtype=np.float32)
        f16 = 0
    labels = np.empty((xa.shape[0], max(m, 0)), dtype=np.int32)
    if st is None:
        _check(_L().mlxvs_kmeans_predict(_ptr(xa), xa.shape[0], _ptr(ca), ca.shape[0],
                                         xa.shape[1], f16, m, _ptr(labels)))
    else:
        _check(_L().mlxvs_kmeans_predict_on_stream(_ptr(xa), xa.shape[0], _ptr(ca), ca.shape[0],
                                                   xa.shape[1], f16, m, _ptr(labels), st))
    return labels


def topk_merge(scores, ids, best, id_offset, first, k, *, stream=None):
    """One merge step of the exact k-NN: ``(ids int32 [nq, k], scores float32
    [nq, k])``, the best k of every row of ``scores`` (float32 [nq, t]; the id
    of column c is ``id_offset + c``) together with the running lists ``ids``
    / ``best`` ([nq, k]) unless ``first``.

    Best first: score descending (-0.0 equal to +0.0), then id ascending;
    among equal scores the lowest ids are kept; -1 / -inf past
    ``min(k, t + (0 if first else k))`` entries.  Mirrors the C++ entry
    reference include/mlxvs/mlxvs.h:892-905 (src/knn.cpp:37-69), which the
    reference does not bind to Python.  ``stream``: as for brute_force_knn.
    """
    op = "mlxvs::topk_merge"
    st = _host_stream(stream, op)
    s = np.asarray(scores)
    if s.ndim != 2 or s.dtype != np.float32:
        raise ValueError(f"[{op}] scores must be float32 [nq, t]")
    s = np.ascontiguousarray(s)
    k = int(k)
    nq, t = s.shape
    first = bool(first)
    ip = bp = None
    if not first:
        pi = np.ascontiguousarray(np.asarray(ids), dtype=np.int32)
        pb = np.ascontiguousarray(np.asarray(best), dtype=np.float32)
        if pi.shape != (nq, k) or pb.shape != (nq, k):
            raise ValueError(f"[{op}] ids and best must be [nq, k] = [{nq}, {k}]")
        ip, bp = _ptr(pi), _ptr(pb)
    out_ids = np.empty((nq, max(k, 0)), dtype=np.int32)
    out_s = np.empty((nq, max(k, 0)), dtype=np.float32)
    if st is None:
        _check(_L().mlxvs_topk_merge(_ptr(s), nq, t, ip, bp, int(id_offset), int(first), k,
                                     _ptr(out_ids), _ptr(out_s)))
    else:
        _check(_L().mlxvs_topk_merge_on_stream(_ptr(s), nq, t, ip, bp, int(id_offset),
                                               int(first), k, _ptr(out_ids), _ptr(out_s), st))
    return out_ids, out_s


def topk_merge_device(scores_ptr, nq, t, ids_ptr, best_ptr, id_offset, first, k, out_ids_ptr,
                      out_scores_ptr, *, stream=None):
    """mlxvs_topk_merge_device on device pointers (ints); enqueues only."""
    _check(_L().mlxvs_topk_merge_device(scores_ptr, nq, t, ids_ptr, best_ptr, int(id_offset),
                                        int(bool(first)), int(k), out_ids_ptr, out_scores_ptr,
                                        stream))


def brute_force_knn_device(base_ptr, n, queries_ptr, nq, d, k, metric, ids_ptr,
                           dist_ptr, *, f16=False, stream=None):
    """mlxvs_brute_force_knn_device on device pointers (ints); enqueues only."""
    _check(_L().mlxvs_brute_force_knn_device(
        base_ptr, n, queries_ptr, nq, d, int(bool(f16)), int(k), int(_metric(metric)),
        ids_ptr, dist_ptr, stream))


def brute_force_knn_filtered_device(base_ptr, n, queries_ptr, nq, d, k, metric, filter_ptr,
                                    filter_kind, ids_ptr, dist_ptr, *, f16=False, stream=None):
    """mlxvs_brute_force_knn_filtered_device on device pointers (ints):
    enqueued on ``stream`` (a hipStream_t handle), returns at once."""
    _check(_L().mlxvs_brute_force_knn_filtered_device(
        base_ptr, n, queries_ptr, nq, d, int(bool(f16)), int(k), int(_metric(metric)), filter_ptr,
        int(filter_kind), ids_ptr, dist_ptr, stream))


def hamming_knn_device(rows_ptr, n, queries_ptr, nq, nbytes, k, ids_ptr, dist_ptr, *,
                       stream=None):
    """mlxvs_hamming_knn_device on device pointers (ints)."""
    _check(_L().mlxvs_hamming_knn_device(rows_ptr, n, queries_ptr, nq, nbytes, int(k),
                                         ids_ptr, dist_ptr, stream))


def knn_self_graph_device(rows_ptr, n, d, k, metric, ids_ptr, dist_ptr, *, f16=False,
                          stream=None):
    """mlxvs_knn_self_graph_device on device pointers (ints)."""
    _check(_L().mlxvs_knn_self_graph_device(rows_ptr, n, d, int(bool(f16)), int(k),
                                            int(_metric(metric)), ids_ptr, dist_ptr, stream))


def profile(enable: bool = True) -> None:
    """Enable (or disable) per-stage kernel timing with HIP events."""
    _check(_L().mlxvs_profile(int(bool(enable))))


def profile_report() -> dict:
    """{stage: (launches, total_ms)} since the last report (waits for the events)."""
    buf = ctypes.create_string_buffer(1 << 16)
    _check(_L().mlxvs_profile_report(buf, len(buf)))
    out = {}
    for line in buf.value.decode().splitlines():
        name, cnt, ms = line.split()
        out[name] = (int(cnt), float(ms))
    return out


def release_workspace() -> None:
    _check(_L().mlxvs_release_workspace())


def version() -> str:
    return _L().mlxvs_version().decode()


from mlxvs_amd.neighbors import NearestNeighbors  # noqa: E402  (uses the functions above)
from mlxvs_amd.ivf import (  # noqa: E402
    IvfFlatIndex, ivf_flat_build, ivf_flat_extend, ivf_flat_search)


def ivf_flat_search_device(centers_ptr, lists, data_ptr, n, indices_ptr, offsets_ptr, d, metric,
                           queries_ptr, nq, k, ids_ptr, dist_ptr, *, n_probes=20, stream=None):
    """mlxvs_ivf_flat_search_device on device pointers (ints)."""
    _check(_L().mlxvs_ivf_flat_search_device(
        centers_ptr, lists, data_ptr, n, indices_ptr, offsets_ptr, d, int(_metric(metric)),
        queries_ptr, nq, int(k), int(n_probes), ids_ptr, dist_ptr, stream))
