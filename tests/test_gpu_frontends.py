"""GPU parity of the front ends around the k-NN path: kmeans_predict,
NearestNeighbors, the cuVS brute-force index and the .ivecs ground truth.

Oracles: float64 NumPy / SciPy distances (tie-tolerant), and the CPU
restatement where the data are integer-valued (bit-exact).
"""

import numpy as np
import pytest
from scipy import spatial

import mlxvs_amd
from mlxvs_amd import formats
from mlxvs_amd.cuvs.neighbors import brute_force

pytestmark = pytest.mark.gpu


def rows(n, d, seed):
    return np.random.default_rng(seed).standard_normal((n, d), dtype=np.float32)


# ---- kmeans_predict (reference src/kmeans.cpp:136-169) ---------------------------------

@pytest.mark.parametrize("m", [1, 2, 5, 16])
def test_kmeans_predict_integer_exact(oracle, m):
    # integer-valued rows and centroids: exact distances, ties to the lowest
    # centroid index (the reference's argmin for m = 1)
    rng = np.random.default_rng(3)
    x = rng.integers(0, 8, (5000, 24)).astype(np.float32)
    c = rng.integers(0, 8, (300, 24)).astype(np.float32)
    labels = mlxvs_amd.kmeans_predict(x, c, m)
    want, _ = oracle.knn(c, x, m, "l2")
    assert labels.dtype == np.int32 and labels.shape == (5000, m)
    assert np.array_equal(labels, want)
    if m == 1:
        d = ((x[:, None, :].astype(np.float64) - c[None]) ** 2).sum(-1)
        assert np.array_equal(labels[:, 0], d.argmin(1))


def test_kmeans_predict_separates_blobs():
    # reference python/tests/test_mlxvs.py:90-101, with the true centres as
    # the centroids (kmeans_fit is outside this engine)
    rng = np.random.default_rng(7)
    centers = 20 * rng.standard_normal((6, 16), dtype=np.float32)
    truth = np.arange(6000) % 6
    x = centers[truth] + rng.standard_normal((6000, 16), dtype=np.float32)
    labels = mlxvs_amd.kmeans_predict(x, centers, 2)
    assert labels.shape == (6000, 2)
    assert (labels[:, 0] == truth).all()
    assert (labels[:, 0] != labels[:, 1]).all()


def test_kmeans_predict_float16_and_mixed():
    c = rows(40, 32, 1)
    x = rows(700, 32, 2)
    d = spatial.distance.cdist(x.astype(np.float64), c.astype(np.float64), "sqeuclidean")
    want = d.argmin(1)
    assert (mlxvs_amd.kmeans_predict(x, c)[:, 0] == want).mean() > 0.999
    lab16 = mlxvs_amd.kmeans_predict(x.astype(np.float16), c.astype(np.float16))[:, 0]
    d16 = spatial.distance.cdist(x.astype(np.float16).astype(np.float64),
                                 c.astype(np.float16).astype(np.float64), "sqeuclidean")
    assert (lab16 == d16.argmin(1)).mean() > 0.999
    # mixed dtypes are computed in float32
    assert np.array_equal(mlxvs_amd.kmeans_predict(x.astype(np.float64), c),
                          mlxvs_amd.kmeans_predict(x, c))


# ---- NearestNeighbors (reference python/mlxvs/_neighbors.py) ---------------------------

@pytest.mark.parametrize("metric", ["euclidean", "sqeuclidean", "l2", "cosine"])
def test_nearest_neighbors_queries(metric):
    x, q = rows(3000, 48, 4), rows(200, 48, 5)
    nn = mlxvs_amd.NearestNeighbors(n_neighbors=7, metric=metric).fit(x)
    dist, ind = nn.kneighbors(q)
    assert ind.dtype == np.int64 and dist.dtype == np.float32 and ind.shape == (200, 7)
    sm = {"euclidean": "euclidean", "sqeuclidean": "sqeuclidean", "l2": "sqeuclidean",
          "cosine": "cosine"}[metric]
    full = spatial.distance.cdist(q.astype(np.float64), x.astype(np.float64), sm)
    want = np.sort(full, 1)[:, :7]
    np.testing.assert_allclose(dist, want, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(np.take_along_axis(full, ind, 1), want, rtol=1e-4, atol=1e-4)
    only = nn.kneighbors(q, return_distance=False)
    assert np.array_equal(only, ind)


def test_nearest_neighbors_self():
    x = rows(2000, 16, 6)
    nn = mlxvs_amd.NearestNeighbors(n_neighbors=5).fit(x)
    dist, ind = nn.kneighbors()
    assert (ind != np.arange(2000)[:, None]).all()
    full = spatial.distance.cdist(x.astype(np.float64), x.astype(np.float64))
    np.fill_diagonal(full, np.inf)
    np.testing.assert_allclose(dist, np.sort(full, 1)[:, :5], rtol=1e-4, atol=1e-4)


# ---- cuVS brute force (reference python/tests/test_cuvs.py:147-193, 777-794) -----------

@pytest.mark.parametrize("metric", ["euclidean", "cityblock", "chebyshev", "canberra",
                                    "correlation", "russellrao", "cosine", "sqeuclidean",
                                    "inner_product"])
@pytest.mark.parametrize("inplace", [True, False])
@pytest.mark.parametrize("serialize", [True, False])
def test_cuvs_brute_force(tmp_path, metric, inplace, serialize):
    rng = np.random.default_rng(3)
    index = rng.random((100, 40)).astype(np.float32)
    queries = rng.random((32, 40)).astype(np.float32)
    if metric == "russellrao":
        index, queries = (index >= 0.5).astype(np.float32), (queries >= 0.5).astype(np.float32)
    k = 5
    neighbors = np.zeros((32, k), np.int64)
    distances = np.zeros((32, k), np.float32)
    bf = brute_force.build(index, metric)
    if serialize:
        path = str(tmp_path / "bf.bin")
        brute_force.save(path, bf)
        bf = brute_force.load(path)
    rd, ri = brute_force.search(bf, queries, k, neighbors=neighbors if inplace else None,
                                distances=distances if inplace else None)
    got = distances if inplace else rd
    ids = neighbors if inplace else ri
    assert ids.dtype == np.int64
    if metric == "inner_product":
        full = queries.astype(np.float64) @ index.astype(np.float64).T
        want = -np.sort(-full, 1)[:, :k]
    else:
        full = spatial.distance.cdist(queries, index, metric=metric)
        want = np.sort(full, 1)[:, :k]
    got = got.copy()
    got[np.abs(got) <= 1e-5] = 0.0
    np.testing.assert_allclose(want, got, atol=1e-3, rtol=1e-3)
    np.testing.assert_allclose(np.take_along_axis(full, ids, 1), want, atol=1e-3, rtol=1e-3)


def _hamming(a, b):
    return np.unpackbits(a[:, None] ^ b[None], axis=2).sum(2)


@pytest.mark.parametrize("nbytes", [3, 16, 128])
def test_cuvs_bitwise_hamming(tmp_path, nbytes):
    rng = np.random.default_rng(11)
    data = rng.integers(0, 256, (700, nbytes), dtype=np.uint8)
    queries = rng.integers(0, 256, (40, nbytes), dtype=np.uint8)
    index = brute_force.build(data, metric="bitwise_hamming")
    path = str(tmp_path / "h.bin")
    brute_force.save(path, index)
    d, i = brute_force.search(brute_force.load(path), queries, 7)
    want = np.sort(_hamming(queries, data), axis=1)[:, :7]
    np.testing.assert_array_equal(d, want)
    np.testing.assert_array_equal(np.take_along_axis(_hamming(queries, data), i, 1), want)


def test_cuvs_k_exceeding_rows():
    # the reference selects min(k, n) per query (brute_force.py:113-136 with
    # _common.py:70-71): three rows, k = 5 -> three columns, for the fused
    # and the pairwise metrics alike
    x = rows(3, 8, 1)
    for metric in ("euclidean", "chebyshev"):
        d, i = brute_force.search(brute_force.build(x, metric), rows(2, 8, 2), 5)
        assert d.shape == (2, 3) and i.shape == (2, 3)
        assert sorted(i[0].tolist()) == [0, 1, 2] and np.isfinite(d).all()


# ---- .ivecs ground truth (reference examples/ground_truth.py) --------------------------

def test_ground_truth_files(tmp_path, oracle):
    rng = np.random.default_rng(9)
    base = rng.integers(0, 16, (4000, 32)).astype(np.float32)
    q = rng.integers(0, 16, (50, 32)).astype(np.float32)
    formats.write_fvecs(tmp_path / "b.fvecs", base)
    formats.write_fvecs(tmp_path / "q.fvecs", q)
    ids = formats.ground_truth(tmp_path / "b.fvecs", tmp_path / "q.fvecs", tmp_path / "gt.ivecs",
                               k=20, metric="l2")
    back = formats.read_ivecs(tmp_path / "gt.ivecs")
    want, _ = oracle.knn(base, q, 20, "l2")
    assert np.array_equal(back, ids) and np.array_equal(back, want)


def test_host_entries_on_a_created_stream(engine, oracle):
    # reference python/bindings.cpp:55, 125: the host-array entries take a
    # stream; the copies and kernels run on it and the call waits for it.
    # The answers are the ones of the null stream, bit for bit.
    from mlxvs_amd import _hip

    st = _hip.Stream()
    rng = np.random.default_rng(77)
    base = rng.integers(0, 9, (40_000, 48)).astype(np.float32)
    q = rng.integers(0, 9, (300, 48)).astype(np.float32)
    for s in (st, st.handle, st.handle.value):
        for metric in ("l2", "inner_product", "cosine"):
            a = engine.brute_force_knn(base, q, 20, metric)
            b = engine.brute_force_knn(base, q, 20, metric, stream=s)
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    oid, odist = oracle.knn(base, q, 20, "l2")
    ids, dist = engine.brute_force_knn(base, q, 20, "l2", stream=st)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)
    # float16 rows
    bh, qh = base.astype(np.float16), q.astype(np.float16)
    a = engine.brute_force_knn(bh, qh, 70, "l2")
    b = engine.brute_force_knn(bh, qh, 70, "l2", stream=st)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    # Hamming (the MFMA route and the few-query scan)
    codes = rng.integers(0, 256, (30_000, 64), dtype=np.uint8)
    for nq in (3, 200):
        qc = codes[:nq] ^ rng.integers(0, 2, (nq, 64), dtype=np.uint8)
        a = engine.hamming_knn(codes, qc, 100)
        b = engine.hamming_knn(codes, qc, 100, stream=st)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        oi, od = oracle.hamming(codes, qc, 100)
        assert np.array_equal(b[0], oi) and np.array_equal(b[1], od)
    # kmeans_predict
    cen = base[:500]
    assert np.array_equal(engine.kmeans_predict(base, cen, 3),
                          engine.kmeans_predict(base, cen, 3, stream=st))
    # topk_merge, first and with running lists
    S = rng.standard_normal((64, 20_000), dtype=np.float32)
    a = engine.topk_merge(S, None, None, 5, True, 40)
    b = engine.topk_merge(S, None, None, 5, True, 40, stream=st)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    a2 = engine.topk_merge(S, a[0], a[1], 100, False, 40)
    b2 = engine.topk_merge(S, b[0], b[1], 100, False, 40, stream=st.handle.value)
    assert np.array_equal(a2[0], b2[0]) and np.array_equal(a2[1], b2[1])
