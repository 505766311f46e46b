"""Python access to the CPU restatement (oracle/knn_oracle.c) and float64 helpers.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the engine (mlxvs_amd/).

Two layers:
  * restated(...) functions call liboracle.so, the float32 restatement of the
    reference's semantics (see the header of knn_oracle.c for file:line
    citations).  They are bit-exact against the reference on integer-valued
    inputs and follow its tie rule (lowest id) everywhere.
  * exact_*(...) functions are independent float64 NumPy brute force with an
    np.lexsort tie-break, used to pin the restatement and to compute recall.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_lib = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        L.oracle_knn_f32.argtypes = [vp, i64, vp, i64, ci, ci, ci, ci, vp, vp]
        L.oracle_knn_filtered_f32.argtypes = [vp, i64, vp, i64, ci, ci, ci, ci, vp, ci, vp, vp]
        L.oracle_self_graph_f32.argtypes = [vp, i64, ci, ci, ci, ci, vp, vp]
        L.oracle_self_graph_rows.argtypes = [vp, i64, ci, ci, ci, ci, i64, vp, vp]
        L.oracle_hamming.argtypes = [vp, i64, vp, i64, ci, ci, ci, vp, vp]
        L.oracle_f16_to_f32.argtypes = [vp, i64, vp]
        L.oracle_pack_words.argtypes = [vp, i64, ci, vp]
        L.oracle_key.argtypes = [ctypes.c_float]
        L.oracle_ivf_flat.argtypes = [vp, ci, vp, vp, vp, ci, ci, vp, i64, ci, ci, ci, vp, vp]
        L.oracle_topk_merge.argtypes = [vp, i64, i64, vp, vp, ctypes.c_int32, ci, ci, vp, vp]
        L.oracle_key.restype = ctypes.c_uint32
        for f in ("oracle_knn_f32", "oracle_knn_filtered_f32", "oracle_self_graph_f32", "oracle_self_graph_rows",
                  "oracle_hamming", "oracle_topk_merge",
                  "oracle_f16_to_f32", "oracle_pack_words"):
            getattr(L, f).restype = ci
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def threads() -> int:
    return int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 1))


METRICS = {"inner_product": 0, "l2": 1, "cosine": 2}


def _m(metric) -> int:
    return METRICS[metric] if isinstance(metric, str) else int(metric)


# ---- the restatement ----------------------------------------------------------

def knn(base, queries, k, metric="l2", nthreads=None):
    """float32 restatement of brute_force_knn (src/knn.cpp:71-142)."""
    b = np.ascontiguousarray(base, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    nq = q.shape[0]
    ids = np.empty((nq, k), np.int32)
    dist = np.empty((nq, k), np.float32)
    rc = lib().oracle_knn_f32(_p(b), b.shape[0], _p(q), nq, b.shape[1], k, _m(metric),
                              nthreads or threads(), _p(ids), _p(dist))
    if rc:
        raise ValueError(f"oracle_knn_f32 rejected the arguments ({rc})")
    return ids, dist


def filter_words(mask):
    """A bool mask as filter words, as cuVS's filters.from_bitset /
    from_bitmap pack it (python/mlxvs/cuvs/neighbors/filters.py:31-37): the
    flattened bits little-endian, padded to whole uint32 words."""
    m = np.asarray(mask, dtype=np.bool_).ravel()
    b = np.packbits(m, bitorder="little")
    return np.pad(b, (0, -len(b) % 4)).view(np.uint32).copy()


def knn_filtered(base, queries, k, metric="l2", bitset=None, bitmap=None, nthreads=None):
    """Restated prefiltered brute-force search (python/mlxvs/cuvs/neighbors/
    brute_force.py:97-136): brute_force_knn over the rows a bool bitset
    [n] or bitmap [nq, n] allows (at most one of them)."""
    b = np.ascontiguousarray(base, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    nq = q.shape[0]
    kind, words = 0, None
    if bitset is not None:
        kind, words = 1, filter_words(bitset)
    elif bitmap is not None:
        kind, words = 2, filter_words(bitmap)
    ids = np.empty((nq, k), np.int32)
    dist = np.empty((nq, k), np.float32)
    rc = lib().oracle_knn_filtered_f32(_p(b), b.shape[0], _p(q), nq, b.shape[1], k, _m(metric),
                                       nthreads or threads(), None if words is None else _p(words),
                                       kind, _p(ids), _p(dist))
    if rc:
        raise ValueError(f"oracle_knn_filtered_f32 rejected the arguments ({rc})")
    return ids, dist


def topk_merge(scores, ids, best, id_offset, first, k):
    """Restated topk_merge (src/knn.cpp:37-69, src/kernels.h:37-229): the
    merged (ids int32 [nq, k], scores float32 [nq, k]), best first."""
    s = np.ascontiguousarray(scores, dtype=np.float32)
    nq, t = s.shape
    pi = pb = None
    if not first:
        pi = np.ascontiguousarray(ids, dtype=np.int32)
        pb = np.ascontiguousarray(best, dtype=np.float32)
    out_i = np.empty((nq, k), np.int32)
    out_s = np.empty((nq, k), np.float32)
    rc = lib().oracle_topk_merge(_p(s), nq, t, None if first else _p(pi),
                                 None if first else _p(pb), int(id_offset), int(bool(first)), k,
                                 _p(out_i), _p(out_s))
    if rc:
        raise ValueError(f"oracle_topk_merge rejected the arguments ({rc})")
    return out_i, out_s


def ivf_flat(centers, data, indices, offsets, queries, k, n_probes, metric="l2",
             nthreads=None):
    """Restated ivf_flat_search (src/ivf.cpp:164-221, 327-416) over a given
    index: centers [lists, d], data [n, d] grouped by list (unit rows for
    cosine), indices [n], offsets [lists + 1]."""
    c = np.ascontiguousarray(centers, dtype=np.float32)
    x = np.ascontiguousarray(data, dtype=np.float32)
    ix = np.ascontiguousarray(indices, dtype=np.int32)
    off = np.ascontiguousarray(offsets, dtype=np.int32)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    nq = q.shape[0]
    ids = np.empty((nq, k), np.int32)
    dist = np.empty((nq, k), np.float32)
    rc = lib().oracle_ivf_flat(_p(c), c.shape[0], _p(x), _p(ix), _p(off), c.shape[1],
                               _m(metric), _p(q), nq, k, n_probes, nthreads or threads(),
                               _p(ids), _p(dist))
    if rc:
        raise ValueError(f"oracle_ivf_flat rejected the arguments ({rc})")
    return ids, dist


def self_graph(rows, k, metric="l2", nthreads=None):
    """Restated single-cluster all_neighbors (src/all_neighbors.cpp:250-263, 56-95)."""
    x = np.ascontiguousarray(rows, dtype=np.float32)
    n = x.shape[0]
    ids = np.empty((n, k), np.int32)
    dist = np.empty((n, k), np.float32)
    rc = lib().oracle_self_graph_f32(_p(x), n, x.shape[1], k, _m(metric),
                                     nthreads or threads(), _p(ids), _p(dist))
    if rc:
        raise ValueError(f"oracle_self_graph_f32 rejected the arguments ({rc})")
    return ids, dist


def self_graph_rows(rows, k, first, metric="l2", nthreads=None):
    """self_graph for the first `first` rows only (all rows are candidates)."""
    x = np.ascontiguousarray(rows, dtype=np.float32)
    ids = np.empty((first, k), np.int32)
    dist = np.empty((first, k), np.float32)
    rc = lib().oracle_self_graph_rows(_p(x), x.shape[0], x.shape[1], k, _m(metric),
                                      nthreads or threads(), first, _p(ids), _p(dist))
    if rc:
        raise ValueError(f"oracle_self_graph_rows rejected the arguments ({rc})")
    return ids, dist


def hamming(rows, queries, k, nthreads=None):
    """Restated hamming_knn (src/ivf.cpp:1343-1403)."""
    r = np.ascontiguousarray(rows, dtype=np.uint8)
    q = np.ascontiguousarray(queries, dtype=np.uint8)
    nq = q.shape[0]
    ids = np.empty((nq, k), np.int32)
    dist = np.empty((nq, k), np.float32)
    rc = lib().oracle_hamming(_p(r), r.shape[0], _p(q), nq, r.shape[1], k,
                              nthreads or threads(), _p(ids), _p(dist))
    if rc:
        raise ValueError(f"oracle_hamming rejected the arguments ({rc})")
    return ids, dist


def f16_to_f32(x):
    h = np.ascontiguousarray(x, dtype=np.float16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32(_p(h.view(np.uint16)), h.size, _p(out))
    return out


def pack_words(rows):
    r = np.ascontiguousarray(rows, dtype=np.uint8)
    w = (r.shape[1] + 3) // 4
    out = np.empty((r.shape[0], w), np.uint32)
    lib().oracle_pack_words(_p(r), r.shape[0], r.shape[1], _p(out))
    return out


def key(v: float) -> int:
    return int(lib().oracle_key(ctypes.c_float(v)))


# ---- independent float64 brute force -------------------------------------------

def exact_scores(queries, base, metric="l2"):
    """float64 scores, larger is closer (-squared distance for L2), as
    python/tests/test_mlxvs.py:13-20 and tests/test_knn.cpp:35-52."""
    q = np.asarray(queries, dtype=np.float64)
    b = np.asarray(base, dtype=np.float64)
    m = _m(metric)
    if m == 1:
        qq = (q * q).sum(1)[:, None]
        bb = (b * b).sum(1)[None, :]
        return -(qq + bb - 2.0 * (q @ b.T))
    if m == 2:
        q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-300)
        b = b / np.maximum(np.linalg.norm(b, axis=1, keepdims=True), 1e-300)
    return q @ b.T


def exact_topk(scores, k):
    """ids of the k best per row by (score desc, id asc), -1 padded."""
    nq, n = scores.shape
    keff = min(k, n)
    ids = np.full((nq, k), -1, np.int64)
    col = np.arange(n)
    for i in range(nq):
        order = np.lexsort((col, -scores[i]))[:keff]
        ids[i, :keff] = order
    return ids


def hamming_distances(queries, rows):
    """popcount(q ^ r) for every pair (python/tests/test_cuvs.py:772-773)."""
    q = np.asarray(queries, dtype=np.uint8)
    r = np.asarray(rows, dtype=np.uint8)
    lut = np.array([bin(i).count("1") for i in range(256)], dtype=np.int32)
    out = np.empty((q.shape[0], r.shape[0]), dtype=np.int32)
    for i in range(q.shape[0]):
        out[i] = lut[q[i][None, :] ^ r].sum(1)
    return out


def recall(ids, scores, k, tol=1e-4):
    """Tie-tolerant recall@k (tests/test_knn.cpp:54-56, 85): an id counts when
    its exact score reaches the exact k-th minus tol * max(1, |kth|)."""
    n = scores.shape[1]
    keff = min(k, n)
    kth = -np.partition(-scores, keff - 1, axis=1)[:, keff - 1: keff]
    ok = ids[:, :keff] >= 0
    got = np.take_along_axis(scores, np.maximum(ids[:, :keff], 0), axis=1)
    hit = (got >= kth - tol * np.maximum(1.0, np.abs(kth))) & ok
    return hit.sum() / (ids.shape[0] * keff)


# ---- cuVS's other distances (test infrastructure: float64 restatement) -------------
#
# The reference's brute_force.search computes these through
# python/mlxvs/cuvs/distance.py:_pairwise (lines 154-168), with the
# expanded forms of _dot_metric (lines 90-118) and the element-wise ones of
# _elementwise (lines 121-151); a = the query, b = the row.  Restated here
# in float64, one query at a time; pinned in tests/test_oracle.py against
# scipy.spatial.distance.cdist, scipy.special.rel_entr and identities that
# a different formula gives.

PAIRWISE_CODES = {"cityblock": 3, "l1": 3, "chebyshev": 7, "canberra": 8, "minkowski": 9,
                  "lp": 9, "correlation": 10, "hellinger": 12, "braycurtis": 14,
                  "jensenshannon": 15, "hamming": 16, "kl_divergence": 17, "russellrao": 18}


def pairwise_distances(queries, rows, metric, p=2.0):
    """float64 [nq, n] distances of the reference's definitions."""
    t = PAIRWISE_CODES[metric] if isinstance(metric, str) else int(metric)
    x = np.asarray(queries, dtype=np.float64)
    y = np.asarray(rows, dtype=np.float64)
    d = x.shape[1]
    if t == 10:  # distance.py:105-111
        sx, sy = x.sum(1)[:, None], y.sum(1)[None]
        sx2, sy2 = (x * x).sum(1)[:, None], (y * y).sum(1)[None]
        numer = d * (x @ y.T) - sx * sy
        return 1 - numer / np.sqrt((d * sx2 - sx * sx) * (d * sy2 - sy * sy))
    if t == 12:  # distance.py:112-114
        return np.sqrt(np.maximum(1 - np.sqrt(x) @ np.sqrt(y).T, 0))
    if t == 18:  # distance.py:115-116
        return (d - x @ y.T) / d
    out = np.empty((x.shape[0], y.shape[0]))
    with np.errstate(divide="ignore", invalid="ignore"):
        for i, a in enumerate(x):
            a = a[None, :]
            if t == 3:
                out[i] = np.abs(a - y).sum(1)
            elif t == 7:
                out[i] = np.abs(a - y).max(1)
            elif t == 8:
                add = np.abs(a) + np.abs(y)
                out[i] = np.where(add != 0, np.abs(a - y) / np.where(add == 0, 1, add), 0).sum(1)
            elif t == 9:
                out[i] = (np.abs(a - y) ** p).sum(1) ** (1.0 / p)
            elif t == 14:
                out[i] = np.abs(a - y).sum(1) / np.abs(a + y).sum(1)
            elif t == 15:
                m = 0.5 * (a + y)
                lm = np.where(m == 0, 0, np.log(np.where(m == 0, 1, m)))
                la = np.log(np.where(a == 0, 1, a))
                lb = np.log(np.where(y == 0, 1, y))
                out[i] = np.sqrt(0.5 * (-a * (lm - la) - y * (lm - lb)).sum(1))
            elif t == 16:
                out[i] = (a != y).mean(1)
            elif t == 17:
                la = np.log(np.where(a == 0, 1, a))
                lb = np.where(y == 0, 0, np.log(np.where(y == 0, 1, y)))
                out[i] = 0.5 * (a * (la - lb)).sum(1)
            else:
                raise ValueError(f"distance type {t} is not one of the pairwise ones")
    return out


def pairwise_knn(queries, rows, k, metric, p=2.0, allowed=None):
    """(ids int64 [nq, k], distances float64 [nq, k]): the k smallest
    distances, lowest id first among equal ones, rows outside ``allowed`` (a
    bool [n] or [nq, n] mask) left out, -1 / +inf past the rows there are."""
    dist = pairwise_distances(queries, rows, metric, p)
    nq, n = dist.shape
    if allowed is not None:
        dist = np.where(np.broadcast_to(np.asarray(allowed, bool), dist.shape), dist, np.inf)
    ids = np.full((nq, k), -1, np.int64)
    out = np.full((nq, k), np.inf)
    col = np.arange(n)
    for i in range(nq):
        order = np.lexsort((col, dist[i]))[:k]
        order = order[~np.isinf(dist[i, order])]  # left out (or infinitely far): -1
        ids[i, :len(order)] = order
        out[i, :len(order)] = dist[i, order]
    return ids, out
