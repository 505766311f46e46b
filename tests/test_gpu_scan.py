"""GPU parity of the few-query float scan (scan_float_kernel) with the oracle.

At most four queries with rows of 128 to 1,024 bytes take the VALU scan:
each (split, query) workgroup selects its split's exact best k, and the
query's last workgroup merges the splits' lists (a counter per query in
device memory that this workgroup resets).  Bars as the other float tests:
integer-valued rows bit-exact against the CPU restatement (ids and
distances), float rows to the tolerance of the reference's tests
(tests/test_knn.cpp:54-56, 85-94).  Calls in a row with different shapes
check that the counters start from zero at every call.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def int_rows(n, d, seed, hi=6):
    return np.random.default_rng(seed).integers(0, hi, (n, d)).astype(np.float32)


@pytest.mark.parametrize("nq", [1, 2, 4])
@pytest.mark.parametrize("d,dt", [(32, np.float32), (64, np.float32), (128, np.float32),
                                  (256, np.float32), (64, np.float16), (128, np.float16),
                                  (256, np.float16), (512, np.float16)])
@pytest.mark.parametrize("k", [1, 10, 17, 32])
def test_scan_integer_bit_exact(engine, oracle, nq, d, dt, k):
    # 100,003 rows: a partial chunk in the last split
    base = int_rows(100_003, d, nq * 100 + d + k)
    q = int_rows(nq, d, nq * 100 + d + k + 1)
    for metric in ("l2", "inner_product"):
        ids, dist = engine.brute_force_knn(base.astype(dt), q.astype(dt), k, metric)
        oid, odist = oracle.knn(base, q, k, metric)
        assert np.array_equal(ids, oid), metric
        assert np.array_equal(dist, odist), metric


@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_scan_float_rows(engine, oracle, metric):
    rng = np.random.default_rng(7)
    base = rng.standard_normal((400_000, 128), dtype=np.float32)
    q = rng.standard_normal((3, 128), dtype=np.float32)
    ids, dist = engine.brute_force_knn(base, q, 10, metric)
    s = oracle.exact_scores(q, base, metric)
    assert oracle.recall(ids, s, 10, 1e-4) == 1.0
    exact = np.take_along_axis(s, ids, 1)
    exact = -exact if metric == "l2" else exact
    assert (np.abs(exact - dist) / np.maximum(1.0, np.abs(exact))).max() < 1e-4


def test_scan_ties_and_small_n(engine, oracle):
    # every row equal: the k lowest ids, from the lists of many splits
    x = np.ones((60_000, 64), np.float32)
    ids, dist = engine.brute_force_knn(x, np.ones((2, 64), np.float32), 32, "l2")
    assert (ids == np.arange(32)).all() and (dist == 0).all()
    # fewer rows than k, and fewer rows than a split
    for n in (1, 5, 255, 256, 257, 4097):
        base = int_rows(n, 32, n)
        q = int_rows(3, 32, n + 1)
        ids, dist = engine.brute_force_knn(base, q, 20, "l2")
        oid, odist = oracle.knn(base, q, 20, "l2")
        assert np.array_equal(ids, oid) and np.array_equal(dist, odist), n


def test_scan_calls_in_a_row(engine, oracle):
    # the per-query counters are reset by each search's last workgroups:
    # searches of different split counts and query counts back to back
    shapes = [(200_000, 1), (9_000, 4), (300_000, 2), (700, 1), (50_000, 3), (200_000, 1)]
    for i, (n, nq) in enumerate(shapes):
        base = int_rows(n, 128, 50 + i)
        q = int_rows(nq, 128, 60 + i)
        ids, dist = engine.brute_force_knn(base, q, 10, "l2")
        oid, odist = oracle.knn(base, q, 10, "l2")
        assert np.array_equal(ids, oid) and np.array_equal(dist, odist), (n, nq)


# ---- the Hamming few-query scan (scan_bits_kernel + rank merges) ------------

@pytest.mark.parametrize("nbytes", [32, 64, 128])
@pytest.mark.parametrize("nq,k", [(1, 1), (1, 100), (3, 37), (4, 256)])
def test_hamming_scan_bit_exact(engine, oracle, nbytes, nq, k):
    rng = np.random.default_rng(nbytes + nq * 10 + k)
    rows = rng.integers(0, 256, (150_001, nbytes), dtype=np.uint8)
    q = rng.integers(0, 256, (nq, nbytes), dtype=np.uint8)
    q[0] = rows[77_777]          # an exact match: distance 0 (a -0 score)
    ids, dist = engine.hamming_knn(rows, q, k)
    oid, odist = oracle.hamming(rows, q, k)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)
    assert ids[0, 0] == 77_777 and dist[0, 0] == 0.0 and not np.signbit(dist[0, 0])


def test_hamming_scan_ties_and_calls_in_a_row(engine, oracle):
    # every row equal: all distances tie, the k lowest ids win
    rows = np.full((80_000, 64), 0x5A, np.uint8)
    ids, dist = engine.hamming_knn(rows, np.full((2, 64), 0x5B, np.uint8), 200)
    assert (ids == np.arange(200)).all() and (dist == 64.0).all()
    # searches of different split and query counts back to back
    rng = np.random.default_rng(5)
    for i, (n, nq, k) in enumerate([(300_000, 1, 100), (5_000, 4, 10), (40_000, 2, 256),
                                    (300, 1, 100), (300_000, 1, 100)]):
        r = rng.integers(0, 256, (n, 128), dtype=np.uint8)
        q = rng.integers(0, 256, (nq, 128), dtype=np.uint8)
        ids, dist = engine.hamming_knn(r, q, k)
        oid, odist = oracle.hamming(r, q, k)
        assert np.array_equal(ids, oid) and np.array_equal(dist, odist), (n, nq, k)
