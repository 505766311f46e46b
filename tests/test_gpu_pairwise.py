"""GPU parity of pairwise_knn (cuVS's other distances) with the oracle.

The reference's cuvs.neighbors.brute_force.search computes these distances
in Python (python/mlxvs/cuvs/distance.py:85-168) and selects with
argpartition (python/mlxvs/cuvs/neighbors/_common.py:68-81); here one
kernel scores each query's rows and selects exactly (mlxvs_pairwise_knn).
Bars:
  * integer-valued rows under L1, Linf, Hamming and Russell-Rao: every
    distance is exact in float32, so ids (lowest id among equal distances)
    and distances equal the float64 restatement (oracle.pairwise_knn) bit
    for bit;
  * float rows under every metric: tie-tolerant recall 1.0 against the
    float64 restatement and distances within 1e-4 relative (Lp, Jensen-
    Shannon and KL: 2e-4 -- powf / logf in float32), the tolerance family of
    the reference's tests (tests/test_knn.cpp:54-56, 85-94);
  * prefilters (bitset, bitmap) as the reference's masked selection gives
    them (brute_force.py:124-136), and more queries than the grid.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

METRICS = ["cityblock", "chebyshev", "canberra", "minkowski", "correlation", "hellinger",
           "braycurtis", "jensenshannon", "hamming", "kl_divergence", "russellrao"]


def data_for(metric, n, nq, d, seed):
    rng = np.random.default_rng(seed)
    b = rng.random((n, d), dtype=np.float32)
    q = rng.random((nq, d), dtype=np.float32)
    if metric in ("jensenshannon", "kl_divergence", "hellinger"):
        # distributions, some zero entries
        b[rng.random(b.shape) < 0.1] = 0
        q[rng.random(q.shape) < 0.1] = 0
        b /= np.maximum(b.sum(1, keepdims=True), 1e-30)
        q /= np.maximum(q.sum(1, keepdims=True), 1e-30)
    if metric in ("russellrao", "hamming"):
        b = (b < 0.5).astype(np.float32)
        q = (q < 0.5).astype(np.float32)
    return b, q


def recall_check(oracle, ids, dist, b, q, k, metric, p=2.0, tol=1e-4, allowed=None):
    full = oracle.pairwise_distances(q, b, metric, p)
    if allowed is not None:
        full = np.where(allowed, full, np.inf)
    scores = -full
    assert oracle.recall(ids, scores, k, tol) == 1.0
    exact = np.take_along_axis(full, np.maximum(ids, 0), 1)
    real = ids >= 0
    err = np.abs(exact - dist) / np.maximum(1.0, np.abs(exact))
    assert err[real].max(initial=0.0) < tol, metric
    assert (np.diff(np.where(real, dist, np.inf), axis=1) >= -tol).all()


@pytest.mark.parametrize("metric", METRICS)
def test_pairwise_float_rows(engine, oracle, metric):
    # 10,007 rows: three chunks of the select; k = 10 and 100
    b, q = data_for(metric, 10_007, 37, 24, 5)
    p = 3.0 if metric == "minkowski" else 2.0
    tol = 2e-4 if metric in ("minkowski", "jensenshannon", "kl_divergence") else 1e-4
    for k in (10, 100):
        ids, dist = engine.pairwise_knn(b, q, k, metric, p)
        assert ids.shape == (37, k) and (ids >= 0).all()
        recall_check(oracle, ids, dist, b, q, k, metric, p, tol)


@pytest.mark.parametrize("metric", ["cityblock", "chebyshev", "hamming", "russellrao"])
@pytest.mark.parametrize("k", [1, 17, 256])
def test_pairwise_integer_rows_bit_exact(engine, oracle, metric, k):
    rng = np.random.default_rng(7 + k)
    hi = 2 if metric == "russellrao" else 4
    b = rng.integers(0, hi, (6_001, 12)).astype(np.float32)
    q = rng.integers(0, hi, (50, 12)).astype(np.float32)
    ids, dist = engine.pairwise_knn(b, q, k, metric)
    oid, odist = oracle.pairwise_knn(q, b, k, metric)
    assert np.array_equal(ids, oid)
    assert np.array_equal(dist, odist.astype(np.float32))


def test_pairwise_prefilters_and_padding(engine, oracle):
    b, q = data_for("cityblock", 3_000, 40, 16, 9)
    rng = np.random.default_rng(10)
    keep = rng.random(3_000) < 0.2
    ids, dist = engine.pairwise_knn(b, q, 20, "canberra", bitset=keep)
    assert keep[ids].all()
    recall_check(oracle, ids, dist, b, q, 20, "canberra", allowed=keep[None, :])
    bm = rng.random((40, 3_000)) < 0.05
    bm[3] = False
    bm[4] = False
    bm[4, [7, 2_999]] = True
    ids, dist = engine.pairwise_knn(b, q, 20, "chebyshev", bitmap=bm)
    assert (ids[3] == -1).all() and np.isinf(dist[3]).all()
    assert sorted(ids[4, :2].tolist()) == [7, 2_999] and (ids[4, 2:] == -1).all()
    ok = [i for i in range(40) if i not in (3, 4)]
    recall_check(oracle, ids[ok], dist[ok], b, q[ok], 20, "chebyshev",
                 allowed=bm[ok])
    # fewer rows than k: -1 / +inf past them
    ids, dist = engine.pairwise_knn(b[:5], q, 8, "braycurtis")
    assert (ids[:, 5:] == -1).all() and np.isinf(dist[:, 5:]).all()
    assert (np.sort(ids[:, :5], 1) == np.arange(5)).all()


def test_pairwise_many_queries(engine, oracle):
    # more queries than workgroups (the grid walks them) and the Lp exponent
    b, q = data_for("minkowski", 2_000, 2_500, 8, 11)
    ids, dist = engine.pairwise_knn(b, q, 5, "minkowski", 1.5)
    recall_check(oracle, ids, dist, b, q, 5, "minkowski", 1.5, 2e-4)


@pytest.mark.parametrize("d", [5, 32, 64, 100, 128, 129, 200])
@pytest.mark.parametrize("metric", ["cityblock", "chebyshev", "hamming"])
def test_pairwise_widths_integer_bit_exact(engine, oracle, d, metric):
    # rows of at most 128 columns take the split-parallel scan (zero-padded
    # to 32, 64 or 128 columns unless already a multiple), wider rows a query
    # per workgroup: both bit-exact on integer rows
    rng = np.random.default_rng(d)
    b = rng.integers(0, 3, (9_000, d)).astype(np.float32)
    q = rng.integers(0, 3, (30, d)).astype(np.float32)
    q[0] = b[4_321]
    ids, dist = engine.pairwise_knn(b, q, 33, metric)
    oid, odist = oracle.pairwise_knn(q, b, 33, metric)
    assert np.array_equal(ids, oid)
    assert np.array_equal(dist, odist.astype(np.float32))
    # the query's own row (or an identical one with a lower id) at distance 0
    assert dist[0, 0] == 0.0 and ids[0, 0] <= 4_321 and (b[ids[0, 0]] == q[0]).all()


@pytest.mark.parametrize("metric", METRICS)
def test_pairwise_wide_rows_float(engine, oracle, metric):
    # 160 columns: the per-query kernel, every metric
    b, q = data_for(metric, 4_000, 20, 160, 13)
    p = 3.0 if metric == "minkowski" else 2.0
    tol = 2e-4 if metric in ("minkowski", "jensenshannon", "kl_divergence") else 1e-4
    ids, dist = engine.pairwise_knn(b, q, 10, metric, p)
    recall_check(oracle, ids, dist, b, q, 10, metric, p, tol)
