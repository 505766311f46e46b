"""GPU parity of the prefiltered exact search with the oracle.

The reference's prefiltered search is cuvs.neighbors.brute_force.search
with filters.from_bitset / from_bitmap (python/mlxvs/cuvs/neighbors/
brute_force.py:97-136, filters.py:39-50; tested at python/tests/
test_cuvs.py:196-211).  Here the filter is applied inside the fused select
(mlxvs_brute_force_knn_filtered).  Bars:
  * integer-valued rows: ids and distances bit-exact against the oracle's
    restatement (oracle.knn_filtered, pinned in tests/test_oracle.py) for
    both filter kinds, on every route the engine takes -- the fused fp32 and
    fp16 kernels (lists of 10 and of 16 with the on-device redo for k > 16),
    the deep kernel (query-split and row-split), few queries (which a filter
    keeps off the stream kernel) and the exhaustive scores + select path;
  * the reference's own prefilter case through brute_force.search, as sets
    against scipy's cdist.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def int_rows(n, d, seed, hi=16):
    return np.random.default_rng(seed).integers(0, hi, (n, d)).astype(np.float32)


def make_filter(kind, nq, n, p, seed):
    rng = np.random.default_rng(seed)
    if kind == "bitmap":
        m = rng.random((nq, n)) < p
        if nq > 2:
            m[1] = False           # a query with nothing allowed
            m[2] = False
            m[2, [3, n - 1]] = True  # and one with two rows
        return {"bitmap": m}
    return {"bitset": rng.random(n) < p}


def assert_same(got, want):
    gi, gd = got
    wi, wd = want
    bad = np.flatnonzero((gi != wi).any(1) | (gd != wd).any(1))
    assert bad.size == 0, (f"{bad.size} queries differ, first {bad[:5].tolist()}: "
                           f"got {gi[bad[0]].tolist()} want {wi[bad[0]].tolist()}")


# (n, nq, d, k, dtype, metric, p): the route each takes is in the comment
CASES = [
    (20_011, 300, 128, 10, np.float32, "l2", 0.3),        # fused fp32, lists of 10
    (20_011, 300, 128, 10, np.float32, "inner_product", 0.05),
    (9_000, 260, 200, 7, np.float32, "l2", 0.5),          # fused fp32, one row block a tile
    (12_345, 200, 64, 65, np.float16, "l2", 0.2),         # fused fp16, lists of 16 + redo
    (12_345, 200, 64, 10, np.float16, "inner_product", 0.02),
    (5_003, 150, 384, 10, np.float32, "l2", 0.3),         # deep fp32, query-split
    (5_003, 20, 512, 33, np.float32, "l2", 0.1),          # deep fp32, row-split, redo
    (30_000, 7, 96, 10, np.float32, "l2", 0.01),          # few queries: fused, not stream
    (1_000, 40, 32, 200, np.float32, "l2", 0.5),          # k > what the split plan holds:
                                                          # exhaustive scores + select
]


@pytest.mark.parametrize("kind", ["bitset", "bitmap"])
@pytest.mark.parametrize("n,nq,d,k,dt,metric,p", CASES)
def test_filtered_bit_exact(engine, oracle, kind, n, nq, d, k, dt, metric, p):
    base = int_rows(n, d, 31)
    q = int_rows(nq, d, 32)
    f = make_filter(kind, nq, n, p, 33)
    got = engine.brute_force_knn_filtered(base.astype(dt), q.astype(dt), k, metric, **f)
    want = oracle.knn_filtered(base, q, k, metric, **f)
    assert_same(got, want)
    if kind == "bitmap" and nq > 2:
        assert (got[0][1] == -1).all()
        assert sorted(got[0][2, :2].tolist()) == [3, n - 1] and (got[0][2, 2:] == -1).all()


def test_filtered_all_rows_is_unfiltered(engine):
    base = int_rows(8_000, 64, 41)
    q = int_rows(100, 64, 42)
    full = engine.brute_force_knn_filtered(base, q, 12, "l2", bitset=np.ones(8_000, bool))
    plain = engine.brute_force_knn(base, q, 12, "l2")
    assert_same(full, plain)
    none = engine.brute_force_knn_filtered(base, q, 12, "cosine", bitset=np.zeros(8_000, bool))
    assert (none[0] == -1).all() and (none[1] == -np.inf).all()


def test_filtered_cosine_float(engine, oracle):
    rng = np.random.default_rng(51)
    base = rng.standard_normal((6_000, 48), dtype=np.float32)
    q = rng.standard_normal((64, 48), dtype=np.float32)
    keep = rng.random(6_000) < 0.25
    ids, dist = engine.brute_force_knn_filtered(base, q, 10, "cosine", bitset=keep)
    s = np.where(keep[None, :], oracle.exact_scores(q, base, "cosine"), -np.inf)
    assert keep[ids].all()
    assert oracle.recall(ids, s, 10, 1e-4) == 1.0
    exact = np.take_along_axis(s, ids, 1)
    assert np.abs(exact - dist).max() < 1e-4


def test_filtered_words_and_device_entry(engine, oracle):
    base = int_rows(10_000, 128, 61)
    q = int_rows(50, 128, 62)
    bm = np.random.default_rng(63).random((50, 10_000)) < 0.1
    want = oracle.knn_filtered(base, q, 16, "l2", bitmap=bm)
    # uint32 words instead of a bool mask
    words = oracle.filter_words(bm)
    assert_same(engine.brute_force_knn_filtered(base, q, 16, "l2", bitmap=words), want)
    # device pointers, enqueued on a stream
    from mlxvs_amd import _hip

    db, dq = _hip.DeviceBuffer.from_array(base), _hip.DeviceBuffer.from_array(q)
    dw = _hip.DeviceBuffer.from_array(words)
    di, dd = _hip.DeviceBuffer(50 * 16 * 4), _hip.DeviceBuffer(50 * 16 * 4)
    st = _hip.Stream()
    engine.brute_force_knn_filtered_device(db.value, 10_000, dq.value, 50, 128, 16, "l2",
                                           dw.value, engine.FILTER_BITMAP, di.value, dd.value,
                                           stream=st.handle)
    st.synchronize()
    assert_same((di.download((50, 16), np.int32), dd.download((50, 16), np.float32)), want)


@pytest.mark.parametrize("kind", ["bitset", "bitmap"])
def test_cuvs_search_prefilter_reference_case(kind):
    # python/tests/test_cuvs.py:196-211
    from scipy.spatial.distance import cdist

    from mlxvs_amd.cuvs.neighbors import brute_force, filters

    rng = np.random.default_rng(4)
    index = rng.random((300, 16)).astype(np.float32)
    queries = rng.random((20, 16)).astype(np.float32)
    if kind == "bitset":
        keep = rng.random(300) < 0.3
        pre = filters.from_bitset(keep)
        allowed = np.broadcast_to(keep, (20, 300))
    else:
        allowed = rng.random((20, 300)) < 0.3
        pre = filters.from_bitmap(allowed)
    _, i = brute_force.search(brute_force.build(index), queries, 7, prefilter=pre)
    pw = np.where(allowed, cdist(queries, index, "sqeuclidean"), np.inf)
    np.testing.assert_array_equal(np.sort(i, 1), np.sort(np.argsort(pw, 1)[:, :7], 1))


def test_cuvs_search_prefilter_hamming_and_units(oracle):
    from mlxvs_amd.cuvs.neighbors import brute_force, filters

    rng = np.random.default_rng(71)
    codes = rng.integers(0, 256, (2_000, 16), dtype=np.uint8)
    qc = rng.integers(0, 256, (30, 16), dtype=np.uint8)
    allowed = rng.random((30, 2_000)) < 0.2
    d, i = brute_force.search(brute_force.build(codes, "bitwise_hamming"), qc, 9,
                              prefilter=filters.from_bitmap(allowed))
    h = oracle.hamming_distances(qc, codes).astype(np.float64)
    h = np.where(allowed, h, np.inf)
    for r in range(30):
        order = np.lexsort((np.arange(2_000), h[r]))[:9]
        assert i[r].tolist() == order.tolist()
        assert d[r].tolist() == h[r, order].tolist()
    # euclidean units and the padding of a query with fewer allowed rows than k
    x = rng.random((100, 8)).astype(np.float32)
    keep = np.zeros(100, bool)
    keep[[4, 50, 99]] = True
    d, i = brute_force.search(brute_force.build(x, "euclidean"), x[:5], 5,
                              prefilter=filters.from_bitset(keep))
    assert (np.sort(i[:, :3], 1) == [4, 50, 99]).all() and (i[:, 3:] == -1).all()
    assert np.isinf(d[:, 3:]).all() and np.isfinite(d[:, :3]).all()
    assert i.dtype == np.int64
