"""GPU parity of the exact Hamming path (hamming_knn) with the oracle.

Bar: ids and distances bit-exact, lowest id first among equal distances
Cases follow the reference's
python/tests/test_cuvs.py:772-793, 840-848 and tests/test_ivf.cpp:252-311.
"""

from pathlib import Path

import numpy as np
import pytest

from mlxvs_amd import synth

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_tiny_kat(engine):
    # python/tests/test_cuvs.py:840-848
    codes = np.array([[0b1111, 0], [0b1, 0]], dtype=np.uint8)
    ids, dist = engine.hamming_knn(codes, codes[:1], 2)
    assert ids[0].tolist() == [0, 1] and dist[0].tolist() == [0.0, 3.0]


@pytest.mark.parametrize("nbytes", [1, 3, 4, 5, 16, 100, 128, 256, 300])
def test_random_codes_exact(engine, oracle, nbytes):
    # python/tests/test_cuvs.py:772-793 (700 rows, 40 queries, k = 7), plus
    # more byte widths (instances and the exhaustive path above 256 bytes)
    rng = np.random.default_rng(11)
    data = rng.integers(0, 256, (700, nbytes), dtype=np.uint8)
    q = rng.integers(0, 256, (40, nbytes), dtype=np.uint8)
    ids, dist = engine.hamming_knn(data, q, 7)
    h = oracle.hamming_distances(q, data)
    want = np.sort(h, axis=1)[:, :7]
    assert np.array_equal(dist, want.astype(np.float32))
    assert np.array_equal(np.take_along_axis(h, ids, 1), want)
    oid, odist = oracle.hamming(data, q, 7)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)


def test_clustered_codes(engine, oracle):
    # tests/test_ivf.cpp:252-285: 20,000 x 32-byte codes around 40 centres
    # with 10% of bits flipped, 300 queries, k = 10
    rng = np.random.default_rng(7)
    centers = rng.integers(0, 256, (40, 32), dtype=np.uint8)
    which = rng.integers(0, 40, 20_300)
    flips = np.packbits(rng.random((20_300, 256)) < 0.1, axis=1)
    allr = centers[which] ^ flips
    x, q = allr[:20_000], allr[20_000:]
    ids, dist = engine.hamming_knn(x, q, 10)
    oid, odist = oracle.hamming(x, q, 10)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)


@pytest.mark.parametrize("k", [1, 4, 8, 16, 17, 100, 256])
def test_ties_and_k(engine, oracle, k):
    # 8-byte codes over 200k rows: many equal distances at the k-th place
    rng = np.random.default_rng(3)
    x = rng.integers(0, 256, (200_000, 8), dtype=np.uint8)
    q = rng.integers(0, 256, (64, 8), dtype=np.uint8)
    ids, dist = engine.hamming_knn(x, q, k)
    oid, odist = oracle.hamming(x, q, k)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)


@pytest.mark.parametrize("nq,k", [(1, 10), (64, 16), (64, 17), (3000, 10)])
def test_zero_codes_keep_sign(engine, oracle, nq, k):
    # zero rows against zero queries: distance +0 (an empty row's popcount
    # must not reach the scores as -0), the zero rows in id order
    rng = np.random.default_rng(nq + k)
    x = rng.integers(0, 256, (30_000, 16), dtype=np.uint8)
    x[rng.choice(30_000, 200, replace=False)] = 0
    q = rng.integers(0, 256, (nq, 16), dtype=np.uint8)
    q[::2] = 0
    ids, dist = engine.hamming_knn(x, q, k)
    oid, odist = oracle.hamming(x, q, k)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)
    assert not np.signbit(dist).any()


def test_all_equal_rows(engine):
    x = np.zeros((50_000, 16), np.uint8)
    ids, dist = engine.hamming_knn(x, x[:3], 100)
    assert (ids == np.arange(100)[None, :]).all() and (dist == 0).all()


def test_fewer_rows_than_k_and_empty(engine):
    x = np.arange(24, dtype=np.uint8).reshape(6, 4)
    ids, dist = engine.hamming_knn(x, x[:2], 10)
    assert (ids[:, 6:] == -1).all() and (dist[:, 6:] == np.inf).all()
    assert (ids[:, :6] >= 0).all()
    ids, dist = engine.hamming_knn(np.zeros((0, 4), np.uint8), x[:2], 3)
    assert (ids == -1).all() and (dist == np.inf).all()


@pytest.fixture(scope="module")
def c4_data():
    gen = lambda lo, hi: synth.c4_codes(1, lo, hi)  # noqa: E731
    base = synth.chunked(gen, 1_000_000)
    q, src = synth.c4_queries(gen, 1_000_000, 2, 0, 10_000)
    return base, q, src


def test_c4_full(engine, oracle, c4_data):
    base, q, src = c4_data
    ids, dist = engine.hamming_knn(base, q, 100)
    g = np.load(GOLDEN / "c4_subset.npz")
    assert np.array_equal(ids[:32], g["ids"])
    assert np.array_equal(dist[:32], g["dist"].astype(np.float32))
    # each query's source code is its nearest, at exactly 51 flipped bits
    assert (ids[:, 0] == src).all() and (dist[:, 0] == 51).all()
    assert (np.diff(dist, axis=1) >= 0).all()
    sel = np.arange(0, 10_000, 331)
    oid, odist = oracle.hamming(base, q[sel], 100)
    assert np.array_equal(ids[sel], oid) and np.array_equal(dist[sel], odist)


def test_c4_device_api(engine, c4_data):
    from mlxvs_amd import _hip

    base, q, _ = c4_data
    q = q[:1000]
    db, dq = _hip.DeviceBuffer.from_array(base), _hip.DeviceBuffer.from_array(q)
    di, dd = _hip.DeviceBuffer(q.shape[0] * 100 * 4), _hip.DeviceBuffer(q.shape[0] * 100 * 4)
    engine.hamming_knn_device(db.value, base.shape[0], dq.value, q.shape[0], 128, 100,
                              di.value, dd.value)
    _hip.synchronize()
    hid, hdist = engine.hamming_knn(base, q, 100)
    assert np.array_equal(di.download(hid.shape, np.int32), hid)
    assert np.array_equal(dd.download(hdist.shape, np.float32), hdist)


@pytest.mark.parametrize("nq", [1, 7])
@pytest.mark.parametrize("k", [10, 100, 256])
@pytest.mark.parametrize("nbytes", [16, 128])
def test_small_batches_exact(engine, oracle, nq, k, nbytes):
    # a handful of queries: hundreds of splits, lists reduced in two levels
    # (groups keep k; for k > 16 the final merge flags overflowing lists)
    rng = np.random.default_rng(nq * 100 + k + nbytes)
    x = rng.integers(0, 256, (150_000, nbytes), dtype=np.uint8)
    q = rng.integers(0, 256, (nq, nbytes), dtype=np.uint8)
    ids, dist = engine.hamming_knn(x, q, k)
    oid, odist = oracle.hamming(x, q, k)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)


def test_unaligned_rows_are_packed(engine, oracle):
    # device rows at an address that is not 16-byte aligned take the packing
    # copy; aligned whole-chunk rows are used in place: the same answers
    from mlxvs_amd import _hip

    rng = np.random.default_rng(5)
    x = rng.integers(0, 256, (20_000, 32), dtype=np.uint8)
    q = rng.integers(0, 256, (50, 32), dtype=np.uint8)
    oid, odist = oracle.hamming(x, q, 12)
    shifted = _hip.DeviceBuffer.from_array(np.concatenate([np.zeros(1, np.uint8), x.ravel()]))
    aligned = _hip.DeviceBuffer.from_array(x)
    dq = _hip.DeviceBuffer.from_array(q)
    for ptr in (shifted.value + 1, aligned.value):
        di, dd = _hip.DeviceBuffer(50 * 12 * 4), _hip.DeviceBuffer(50 * 12 * 4)
        engine.hamming_knn_device(ptr, 20_000, dq.value, 50, 32, 12, di.value, dd.value)
        _hip.synchronize()
        assert np.array_equal(di.download((50, 12), np.int32), oid)
        assert np.array_equal(dd.download((50, 12), np.float32), odist)


@pytest.mark.parametrize("nq", [1, 2, 3, 4])
@pytest.mark.parametrize("nbytes,n", [(32, 300_000), (64, 70_000), (128, 1_000), (20, 9_000)])
@pytest.mark.parametrize("k", [1, 37, 256])
def test_few_queries_scan(engine, oracle, nq, nbytes, n, k):
    # at most four queries: one workgroup per (split, query) scores its rows
    # with VALU popcounts, and the splits' lists of k merge (row widths of
    # 2, 4 and 8 vectors; 20-byte codes are packed to 32; 1,000 rows: some
    # splits are empty)
    rng = np.random.default_rng(nq * 1000 + nbytes + k)
    x = rng.integers(0, 256, (n, nbytes), dtype=np.uint8)
    # a few exact copies and near copies of the queries: ties at distance 0
    q = rng.integers(0, 256, (nq, nbytes), dtype=np.uint8)
    x[rng.choice(n, 5, replace=False)] = q[0]
    ids, dist = engine.hamming_knn(x, q, k)
    oid, odist = oracle.hamming(x, q, k)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)
    assert not np.signbit(dist).any()


@pytest.mark.parametrize("k", [10, 100])
def test_few_queries_scan_all_ties(engine, k):
    # every distance 0 through the scan path (64-byte codes, three queries):
    # at k = 10 the slots' bound leaves the first ten splits' lists, 100
    # ranks of one key, chosen by id in the survivors' select; at k = 100
    # there are fewer splits than slots, no bound, and all the splits'
    # ranks (more than the select's buffer holds) go to the fallback
    x = np.zeros((200_000, 64), np.uint8)
    ids, dist = engine.hamming_knn(x, x[:3], k)
    assert (ids == np.arange(k)[None, :]).all() and (dist == 0).all()


@pytest.mark.parametrize("k", [10, 100])
def test_few_queries_scan_bound_slots_reset(engine, oracle, k):
    # the scan's bound slots (the best rank of each class of splits) persist
    # on the device between searches and are reset by the search's merge: a
    # search whose rows hold exact copies of its queries (every slot at the
    # best rank there is) followed by searches of rows far from theirs, whose
    # results a leftover bound would drop
    rng = np.random.default_rng(k)
    x = rng.integers(0, 256, (100_000, 64), dtype=np.uint8)
    q = rng.integers(0, 256, (3, 64), dtype=np.uint8)
    x[::50] = q[0]
    ids, dist = engine.hamming_knn(x, q, k)
    oid, odist = oracle.hamming(x, q, k)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)
    assert (dist[0] == 0).all()
    for seed in range(2):
        y = rng.integers(0, 256, (50_000, 64), dtype=np.uint8)
        p = (~y[:2]).copy()  # queries at distance 512 from rows 0 and 1
        ids, dist = engine.hamming_knn(y, p, k)
        oid, odist = oracle.hamming(y, p, k)
        assert np.array_equal(ids, oid) and np.array_equal(dist, odist)


@pytest.mark.parametrize("n", [1, 21, 255])
@pytest.mark.parametrize("k", [44, 256])
def test_few_queries_scan_under_k_rows(engine, oracle, n, k):
    # fewer rows than k at four queries (the scan path): the splits' lists
    # hold n ranks between them, and the rest of the k slots come out empty
    # (-1 / +inf), not as whatever the merge's buffer held before
    rng = np.random.default_rng(n + k)
    x = rng.integers(0, 256, (n, 71), dtype=np.uint8)
    q = rng.integers(0, 256, (4, 71), dtype=np.uint8)
    ids, dist = engine.hamming_knn(x, q, k)
    oid, odist = oracle.hamming(x, q, k)
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)
    assert (ids[:, n:] == -1).all() and (dist[:, n:] == np.inf).all()
