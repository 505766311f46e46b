"""GPU parity of the float exact k-NN path (brute_force_knn) with the oracle.

Bars:
  * integer-valued inputs (configurations c1, c2): ids and distances
    bit-exact against the CPU restatement and the float64 golden fixtures;
  * float inputs: recall@k = 1.0 against float64 (tie-tolerant as the
    reference's tests/test_knn.cpp:54-56, 85), distances within
    1e-4 * max(1, |exact|) (fp32) or 2e-3 (fp16), rows sorted nearest first.
Cases follow the reference's tests/test_knn.cpp:156-207 and
python/tests/test_mlxvs.py:30-87, 206-245.
"""

from pathlib import Path

import numpy as np
import pytest

from mlxvs_amd import synth

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def rows(n, d, seed):
    return np.random.default_rng(seed).standard_normal((n, d), dtype=np.float32)


def check_float(oracle, ids, dist, base, q, k, metric, tol=1e-4):
    """recall 1.0 vs float64 (tie-tolerant), distances within tol, sorted,
    -1 / +-inf padding."""
    n = base.shape[0]
    keff = min(k, n)
    s = oracle.exact_scores(q, base, metric)
    assert ids.shape == (q.shape[0], k) and dist.shape == (q.shape[0], k)
    assert (ids[:, keff:] == -1).all()
    if keff < k:
        pad = np.inf if metric == "l2" else -np.inf
        assert (dist[:, keff:] == pad).all()
    assert (ids[:, :keff] >= 0).all() and (ids[:, :keff] < n).all()
    assert oracle.recall(ids, s, k, tol) == 1.0
    exact = np.take_along_axis(s, ids[:, :keff], 1)
    exact = -exact if metric == "l2" else exact
    err = np.abs(exact - dist[:, :keff]) / np.maximum(1.0, np.abs(exact))
    assert err.max() < tol, err.max()
    step = np.diff(dist[:, :keff], axis=1)
    if metric == "l2":
        assert (step >= -1e-5 * np.maximum(1, np.abs(dist[:, 1:keff]))).all()
    else:
        assert (step <= 1e-5 * np.maximum(1, np.abs(dist[:, 1:keff]))).all()
    # distinct ids per row
    for r in ids[:, :keff]:
        assert len(set(r.tolist())) == keff


# ---- integer-valued configurations: bit-exact -----------------------------------

def test_c1_bit_exact(engine, oracle):
    base = synth.c1_rows(1, 0, 10_000)
    q = synth.c1_rows(2, 0, 100)
    ids, dist = engine.brute_force_knn(base, q, 10, "l2")
    oid, odist = oracle.knn(base, q, 10, "l2")
    assert np.array_equal(ids, oid)
    assert np.array_equal(dist, odist)
    g = np.load(GOLDEN / "c1_full.npz")
    assert np.array_equal(ids, g["ids"])
    assert np.array_equal(dist, g["dist"].astype(np.float32))


@pytest.fixture(scope="module")
def c2_data():
    cen = synth.c2_centres()
    base = synth.chunked(lambda lo, hi: synth.c2_rows(1, lo, hi, centres=cen), 1_000_000)
    q = synth.chunked(lambda lo, hi: synth.c2_rows(2, lo, hi, centres=cen), 10_000)
    return base, q


def test_c2_full_bit_exact(engine, oracle, c2_data):
    base, q = c2_data
    ids, dist = engine.brute_force_knn(base, q, 10, "l2")
    g = np.load(GOLDEN / "c2_subset.npz")
    assert np.array_equal(ids[:64], g["ids"])
    assert np.array_equal(dist[:64], g["dist"].astype(np.float32))
    # every query against the CPU restatement (about 10 s on 16 cores)
    oid, odist = oracle.knn(base, q, 10, "l2")
    bad = np.flatnonzero((ids != oid).any(1) | (dist != odist).any(1))
    assert bad.size == 0, f"{bad.size} of 10,000 queries differ, first {bad[:5]}"
    # every returned distance is the exact integer squared distance
    diff = base[ids.astype(np.int64)] - q[:, None, :]
    assert np.array_equal(dist, (diff.astype(np.float64) ** 2).sum(-1).astype(np.float32))
    assert (np.diff(dist, axis=1) >= 0).all()


def test_c2_device_api_matches_host_api(engine, c2_data):
    from mlxvs_amd import _hip

    base, q = c2_data
    q = q[:2000]
    db, dq = _hip.DeviceBuffer.from_array(base), _hip.DeviceBuffer.from_array(q)
    di, dd = _hip.DeviceBuffer(q.shape[0] * 10 * 4), _hip.DeviceBuffer(q.shape[0] * 10 * 4)
    engine.brute_force_knn_device(db.value, base.shape[0], dq.value, q.shape[0], 128, 10,
                                  "l2", di.value, dd.value)
    _hip.synchronize()
    ids = di.download((q.shape[0], 10), np.int32)
    dist = dd.download((q.shape[0], 10), np.float32)
    hid, hdist = engine.brute_force_knn(base, q, 10, "l2")
    assert np.array_equal(ids, hid) and np.array_equal(dist, hdist)


# ---- reference test cases (float data) ------------------------------------------

CASES = [  # tests/test_knn.cpp:197-207 (metric, name, n, nq, d, k)
    ("inner_product", 5000, 64, 64, 10),
    ("inner_product", 5000, 64, 64, 100),
    ("cosine", 5000, 64, 96, 96),
    ("l2", 5000, 64, 128, 32),
    ("l2", 3000, 16, 32, 256),
    ("inner_product", 50, 8, 16, 100),
    ("cosine", 4000, 32, 64, 1),
    ("l2", 5000, 61, 64, 16),
    ("cosine", 3000, 29, 32, 10),
]


@pytest.mark.parametrize("metric,n,nq,d,k", CASES)
def test_reference_cases(engine, oracle, metric, n, nq, d, k):
    base, q = rows(n, d, 1), rows(nq, d, 2)
    ids, dist = engine.brute_force_knn(base, q, k, metric)
    check_float(oracle, ids, dist, base, q, k, metric)


@pytest.mark.parametrize("metric", ["inner_product", "l2", "cosine"])
@pytest.mark.parametrize("k", [10, 100, 256])
def test_python_grid(engine, oracle, metric, k):
    # python/tests/test_mlxvs.py:30-48
    base, q = rows(3000, 48, 1), rows(32, 48, 2)
    ids, dist = engine.brute_force_knn(base, q, k, metric)
    check_float(oracle, ids, dist, base, q, k, metric)


@pytest.mark.parametrize("d", [1, 3, 7, 8, 13, 31, 64, 100, 129, 200, 256, 257, 300])
@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_dimensions(engine, oracle, d, metric):
    base, q = rows(20_000, d, 3), rows(300, d, 4)
    ids, dist = engine.brute_force_knn(base, q, 10, metric)
    check_float(oracle, ids, dist, base, q, 10, metric)


@pytest.mark.parametrize("k", [1, 4, 5, 8, 9, 10, 11, 16, 17, 32, 64, 65, 128, 256])
def test_k_values_large_n(engine, oracle, k):
    # exercises every list length and the k > T check of the merge
    base, q = rows(200_000, 32, 5), rows(200, 32, 6)
    ids, dist = engine.brute_force_knn(base, q, k, "l2")
    check_float(oracle, ids, dist, base, q, k, "l2")


def test_float_data_vs_restatement(engine, oracle):
    # ids equal to the float32 restatement wherever its k-th and (k+1)-th
    # scores are not within rounding of each other
    base, q = rows(50_000, 64, 7), rows(128, 64, 8)
    ids, dist = engine.brute_force_knn(base, q, 10, "l2")
    oid, odist = oracle.knn(base, q, 10, "l2")
    np.testing.assert_allclose(dist, odist, rtol=1e-4, atol=1e-4)
    same = (ids == oid).all(1).mean()
    assert same > 0.95


def test_ties_keep_lowest_ids(engine):
    # tests/test_knn.cpp:156-192
    g = np.load(GOLDEN / "kat_ties.npz")
    first, _ = engine.brute_force_knn(g["base"], g["queries"], 10, "l2")
    for _ in range(20):
        again, _ = engine.brute_force_knn(g["base"], g["queries"], 10, "l2")
        assert np.array_equal(again, first)
    assert np.array_equal(first, g["ids"])


@pytest.mark.parametrize("d,dtype", [(3, np.float32), (3, np.float16), (300, np.float32)])
def test_tie_pushed_down_keeps_lower_id(engine, d, dtype):
    # One lane's stream (rows 0-3, 8-11, ... share a lane): rows 0 and 1 tie at
    # distance 10, rows 2 and 3 are nearer, then row 8 (distance 1) pushes the
    # list down one slot.  With k = 4 the tie is at the edge: row 0 (the
    # lower id) must stay and row 1 go.  (A carried entry once lost an
    # equal-key comparison against the newer entry below it.)
    x = np.zeros((64, d), np.float32)
    x[:, 0] = 10.0                      # distance 100 for the other rows
    x[0, :3] = (1, 3, 0)                # 10
    x[1, :3] = (3, 1, 0)                # 10
    x[2, :3] = (1, 2, 0)                # 5
    x[3, :3] = (1, 1, 2)                # 6
    x[8, :3] = (1, 0, 0)                # 1
    q = np.zeros((1, d), np.float32)
    ids, dist = engine.brute_force_knn(x.astype(dtype), q.astype(dtype), 4, "l2")
    assert ids.tolist() == [[8, 2, 3, 0]]
    assert dist.tolist() == [[1.0, 5.0, 6.0, 10.0]]


def test_tie_pushed_down_hamming(engine):
    # the same pattern on Hamming codes (int8 MFMA route): distances 3, 3, 1,
    # 2, then 0 for rows 0, 1, 2, 3, 8
    codes = np.full((64, 16), 0xFF, np.uint8)  # distance 128 for the others
    q = np.zeros((1, 16), np.uint8)
    codes[0] = 0; codes[0, 0] = 0b0111
    codes[1] = 0; codes[1, 1] = 0b0111
    codes[2] = 0; codes[2, 0] = 0b1
    codes[3] = 0; codes[3, 0] = 0b11
    codes[8] = 0
    ids, dist = engine.hamming_knn(codes, q, 4)
    assert ids.tolist() == [[8, 2, 3, 0]]
    assert dist.tolist() == [[0.0, 1.0, 2.0, 3.0]]


def test_massive_ties_large_k(engine):
    # every row at the same distance: the k lowest ids, for k above the
    # register list length (the merge's check sends these to the
    # exhaustive select)
    x = np.ones((100_000, 16), np.float32)
    ids, dist = engine.brute_force_knn(x, x[:5], 100, "l2")
    assert (ids == np.arange(100)[None, :]).all()
    assert (dist == 0).all()


def test_sorted_data_forces_exhaustive_check(engine, oracle):
    # consecutive ids are nearest: one segment holds the whole answer
    x = np.arange(300_000, dtype=np.float32)[:, None] * 0.5
    q = np.array([[1000.3], [77777.1], [149999.0]], np.float32)
    for k in (50, 256):
        ids, dist = engine.brute_force_knn(x, q, k, "l2")
        oid, odist = oracle.knn(x, q, k, "l2")
        assert np.array_equal(ids, oid) and np.array_equal(dist, odist)


def test_fewer_rows_than_k(engine):
    # python/tests/test_mlxvs.py:63-69
    b, q = rows(5, 8, 3), rows(4, 8, 4)
    ids, dist = engine.brute_force_knn(b, q, 8, "l2")
    assert (ids[:, :5] >= 0).all() and (ids[:, 5:] == -1).all()
    assert np.isinf(dist[:, 5:]).all() and (dist[:, 5:] > 0).all()
    assert sorted(ids[0, :5].tolist()) == list(range(5))
    ids, dist = engine.brute_force_knn(b, q, 8, "inner_product")
    assert (ids[:, 5:] == -1).all() and (dist[:, 5:] == -np.inf).all()


def test_tiny_shapes(engine, oracle):
    # python/tests/test_mlxvs.py:51-60
    b, q = rows(100, 8, 21), rows(2, 8, 22)
    ids, _ = engine.brute_force_knn(b, q, 3, "cosine")
    s = oracle.exact_scores(q, b, "cosine")
    assert oracle.recall(ids, s, 3) == 1.0
    ids, _ = engine.brute_force_knn(b, q, 1, "l2", tile_rows=7)
    assert ids.shape == (2, 1)


def test_empty_inputs(engine):
    ids, dist = engine.brute_force_knn(np.zeros((0, 4), np.float32), rows(3, 4, 1), 5, "l2")
    assert (ids == -1).all() and (dist == np.inf).all()
    ids, dist = engine.brute_force_knn(np.zeros((0, 4), np.float32), rows(3, 4, 1), 5, "cosine")
    assert (ids == -1).all() and (dist == -np.inf).all()
    ids, dist = engine.brute_force_knn(rows(10, 4, 1), np.zeros((0, 4), np.float32), 5, "l2")
    assert ids.shape == (0, 5)


def test_non_contiguous_input(engine):
    # python/tests/test_mlxvs.py:81-87
    b = rows(500, 64, 5)
    bt = np.ascontiguousarray(b.T).T
    q = rows(8, 64, 6)
    a1, _ = engine.brute_force_knn(bt, q, 10, "l2")
    a2, _ = engine.brute_force_knn(b, q, 10, "l2")
    assert np.array_equal(a1, a2)


@pytest.mark.parametrize("convert", [
    lambda x: x, lambda x: x.astype(np.float64), lambda x: x.tolist(),
    lambda x: x.astype(np.float16)], ids=["numpy", "float64", "list", "float16"])
def test_array_likes_and_dtypes(engine, convert):
    # python/tests/test_mlxvs.py:206-226
    x = rows(500, 16, 15)
    want, _ = engine.brute_force_knn(x, x, 5, "l2")
    got, _ = engine.brute_force_knn(convert(x), convert(x), 5, "l2")
    assert (got[:, 0] == np.arange(500)).all()
    assert (got == want).mean() > 0.9


def test_metric_names(engine):
    # python/tests/test_mlxvs.py:228-237
    x = rows(300, 8, 16)
    for name in ["l2", "cosine", "inner_product"]:
        a, _ = engine.brute_force_knn(x, x, 3, name)
        b, _ = engine.brute_force_knn(x, x, 3, getattr(engine.Metric, name))
        assert (a == b).all()


@pytest.mark.parametrize("metric", ["l2", "inner_product"])
@pytest.mark.parametrize("d", [64, 128, 200, 256])
def test_fp16_path(engine, oracle, metric, d):
    # binary16 storage, fp16 MFMA with fp32 accumulation: the products are
    # exact, so the result is the float32 computation on upcast rows
    b = rows(30_000, d, 9).astype(np.float16)
    q = rows(100, d, 10).astype(np.float16)
    ids, dist = engine.brute_force_knn(b, q, 16, metric)
    check_float(oracle, ids, dist, oracle.f16_to_f32(b), oracle.f16_to_f32(q), 16, metric,
                tol=2e-3)


# ---- deep rows (d > 256): the K-looped kernel --------------------------------------

@pytest.mark.parametrize("d", [288, 512, 1000, 1536, 2048])
@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_deep_dimensions(engine, oracle, d, metric):
    base, q = rows(6_000, d, 21), rows(300, d, 22)
    ids, dist = engine.brute_force_knn(base, q, 10, metric)
    check_float(oracle, ids, dist, base, q, 10, metric)


@pytest.mark.parametrize("k", [1, 4, 10, 16, 17, 32, 100, 256])
def test_deep_integer_bit_exact(engine, oracle, k):
    # integer values in [0, 16): every score is an integer below 2^24, exact
    # in any summation order, so ids (ties to the lowest id) and distances
    # equal the CPU restatement's bit for bit; n and nq leave partial tiles
    # and a query block with one query
    rng = np.random.default_rng(31)
    base = rng.integers(0, 16, (20_000, 768)).astype(np.float32)
    q = rng.integers(0, 16, (257, 768)).astype(np.float32)
    for metric in ("l2", "inner_product"):
        ids, dist = engine.brute_force_knn(base, q, k, metric)
        oid, odist = oracle.knn(base, q, k, metric)
        assert np.array_equal(ids, oid), metric
        assert np.array_equal(dist, odist), metric


@pytest.mark.parametrize("n", [1, 9, 127, 128, 129, 1_000])
def test_deep_small_n(engine, oracle, n):
    base, q = rows(n, 320, 23), rows(40, 320, 24)
    for k in (1, 10, 64):
        ids, dist = engine.brute_force_knn(base, q, k, "l2")
        check_float(oracle, ids, dist, base, q, k, "l2")


def test_deep_device_api_matches_host_api(engine):
    from mlxvs_amd import _hip

    base, q = rows(30_000, 640, 25), rows(130, 640, 26)
    ids, dist = engine.brute_force_knn(base, q, 10, "l2")
    db, dq = _hip.DeviceBuffer.from_array(base), _hip.DeviceBuffer.from_array(q)
    di, dd = _hip.DeviceBuffer(130 * 10 * 4), _hip.DeviceBuffer(130 * 10 * 4)
    engine.brute_force_knn_device(db.value, 30_000, dq.value, 130, 640, 10, "l2", di.value,
                                  dd.value)
    _hip.synchronize()
    assert np.array_equal(di.download((130, 10), np.int32), ids)
    assert np.array_equal(dd.download((130, 10), np.float32), dist)


@pytest.mark.parametrize("k", [10, 17, 65, 128])
def test_fp16_integer_bit_exact(engine, oracle, k):
    # binary16 integers in [0, 16), d = 256: scores are exact in fp32, so the
    # fp16 MFMA path must equal the restatement bit for bit, also for k > 16
    # where the lists share multi-slot bounds
    rng = np.random.default_rng(41)
    base = rng.integers(0, 16, (50_000, 256)).astype(np.float16)
    q = rng.integers(0, 16, (300, 256)).astype(np.float16)
    ids, dist = engine.brute_force_knn(base, q, k, "l2")
    oid, odist = oracle.knn(oracle.f16_to_f32(base), oracle.f16_to_f32(q), k, "l2")
    assert np.array_equal(ids, oid)
    assert np.array_equal(dist, odist)


@pytest.mark.parametrize("nq", [16, 256])
def test_c3_subset(engine, oracle, nq):
    # c3's mixture on its first 100,000 rows: 16 queries take the row-split
    # deep kernel, 256 the query-split one that the full c3 runs
    cen = synth.c3_centres()
    base = synth.chunked(lambda lo, hi: synth.c3_rows(1, lo, hi, centres=cen), 100_000,
                         chunk=5_000)
    q = synth.c3_rows(2, 0, nq, centres=cen)
    g = np.load(GOLDEN / "c3_subset.npz")
    for metric, key in (("inner_product", "ip"), ("cosine", "cos")):
        ids, dist = engine.brute_force_knn(base, q, 10, metric)
        s = oracle.exact_scores(q, base, metric)
        assert oracle.recall(ids, s, 10) == 1.0
        exact = np.take_along_axis(s, ids, 1)
        assert np.abs(exact - dist).max() < 1e-4
        np.testing.assert_allclose(dist, g["score_" + key][:nq], atol=1e-4)
        assert (ids == g["ids_" + key][:nq]).mean() > 0.95


@pytest.fixture(scope="module")
def c3_full():
    cen = synth.c3_centres()
    base = synth.chunked(lambda lo, hi: synth.c3_rows(1, lo, hi, centres=cen), 1_000_000,
                         chunk=5_000)
    # 64 of the configuration's 10,000 queries, strided (the generator is
    # counter-based: query i is the same row whichever others are made)
    sel = np.arange(0, 10_000, 157)[:64]
    q = np.concatenate([synth.c3_rows(2, int(i), int(i) + 1, centres=cen) for i in sel])
    return base, q


def exact_scores_chunked(oracle, q, base, metric, chunk=100_000):
    return np.concatenate([oracle.exact_scores(q, base[c:c + chunk], metric)
                           for c in range(0, base.shape[0], chunk)], axis=1)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("metric", ["inner_product", "cosine"])
def test_c3_full_size(engine, oracle, c3_full, metric):
    # configuration c3 at its full size (1,000,000 x 1,536 fp32): 64 queries
    # take the query-split deep kernel that the 10,000-query run uses;
    # recall 1.0 against float64 (tie-tolerant) and distances within 1e-4
    base, q = c3_full
    ids, dist = engine.brute_force_knn(base, q, 10, metric)
    s = exact_scores_chunked(oracle, q, base, metric)
    assert oracle.recall(ids, s, 10) == 1.0
    exact = np.take_along_axis(s, ids, 1)
    assert (np.abs(exact - dist) / np.maximum(1.0, np.abs(exact))).max() < 1e-4
    assert (np.diff(dist, axis=1) <= 1e-6).all()
    assert all(len(set(r.tolist())) == 10 for r in ids)


# ---- small batches (<= 32 queries, fp32, d <= 128, k <= 16: the streamed scan) ---------

@pytest.mark.parametrize("nq", [1, 7, 32])
@pytest.mark.parametrize("d", [4, 20, 32, 48, 64, 100, 128])
@pytest.mark.parametrize("k", [1, 4, 10, 16])
def test_small_batch_integer_bit_exact(engine, oracle, nq, d, k):
    # n leaves a partial tile in the last split; d below 2 x the half width
    # exercises the masked dims (values there belong to the next row)
    rng = np.random.default_rng(nq * 1000 + d * 10 + k)
    base = rng.integers(0, 6, (70_001, d)).astype(np.float32)
    q = rng.integers(0, 6, (nq, d)).astype(np.float32)
    for metric in ("l2", "inner_product"):
        ids, dist = engine.brute_force_knn(base, q, k, metric)
        oid, odist = oracle.knn(base, q, k, metric)
        assert np.array_equal(ids, oid), metric
        assert np.array_equal(dist, odist), metric


@pytest.mark.parametrize("nq", [1, 32])
@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_small_batch_float(engine, oracle, nq, metric):
    base, q = rows(300_000, 128, 31), rows(nq, 128, 32)
    ids, dist = engine.brute_force_knn(base, q, 10, metric)
    check_float(oracle, ids, dist, base, q, 10, metric)


@pytest.mark.parametrize("n", [1, 31, 127, 128, 129, 5_000])
def test_small_batch_small_n(engine, oracle, n):
    rng = np.random.default_rng(n)
    base = rng.integers(0, 5, (n, 24)).astype(np.float32)
    q = rng.integers(0, 5, (3, 24)).astype(np.float32)
    ids, dist = engine.brute_force_knn(base, q, 10, "l2")
    oid, odist = oracle.knn(base, q, 10, "l2")
    assert np.array_equal(ids, oid) and np.array_equal(dist, odist)


def test_small_batch_next_row_values_stay_out():
    # d = 20 reads 32-dim halves: dims 20-31 of a row's fetch are the next
    # row's first values (here inf); they must not reach any score
    x = np.zeros((4096, 20), np.float32)
    x[:, 0] = np.arange(4096, dtype=np.float32)
    x[1::2, 0] = np.inf
    import mlxvs_amd
    ids, dist = mlxvs_amd.brute_force_knn(x, np.zeros((1, 20), np.float32), 3, "l2")
    assert ids.tolist() == [[0, 2, 4]]
    assert dist.tolist() == [[0.0, 4.0, 16.0]]


def test_small_batch_ties_keep_lowest_ids(engine):
    # every row equal: the k lowest ids, from segments of many splits
    x = np.ones((50_000, 16), np.float32)
    ids, dist = engine.brute_force_knn(x, np.ones((2, 16), np.float32), 16, "l2")
    assert (ids == np.arange(16)).all() and (dist == 0).all()


@pytest.mark.parametrize("nq", [1, 64, 3000])
@pytest.mark.parametrize("k", [4, 16, 17])
@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_zero_scores_tie_and_keep_sign(engine, oracle, nq, k, metric):
    # zero rows (scores of exactly 0 from -0 products too) among rows whose
    # scores are worse: the best answers are the zero rows in id order, and
    # zero distances come out as the reference's +0
    rng = np.random.default_rng(nq + k)
    base = -rng.integers(1, 4, (40_000, 32)).astype(np.float32)
    base[rng.choice(40_000, 300, replace=False)] = 0.0
    base[5::997] = -0.0
    q = rng.integers(0, 3, (nq, 32)).astype(np.float32)
    q[::3] = 0.0
    q[1::7, :8] = -0.0
    ids, dist = engine.brute_force_knn(base, q, k, metric)
    oid, odist = oracle.knn(base, q, k, metric)
    assert np.array_equal(ids, oid)
    assert np.array_equal(dist, odist)
    assert np.array_equal(np.signbit(dist), np.signbit(odist))


@pytest.mark.parametrize("nq", [1, 5, 32])
@pytest.mark.parametrize("k", [17, 64, 100, 256])
def test_small_batch_large_k_bit_exact(engine, oracle, nq, k):
    # k > T on the streamed scan: thousands of 16-long lists reduced in two
    # levels (groups keep k, the final merge flags a query when a full list's
    # last entry made the k; flagged queries go exhaustive)
    rng = np.random.default_rng(nq * 7 + k)
    base = rng.integers(0, 6, (120_000, 64)).astype(np.float32)
    q = rng.integers(0, 6, (nq, 64)).astype(np.float32)
    for metric in ("l2", "inner_product"):
        ids, dist = engine.brute_force_knn(base, q, k, metric)
        oid, odist = oracle.knn(base, q, k, metric)
        assert np.array_equal(ids, oid), metric
        assert np.array_equal(dist, odist), metric


def test_small_batch_large_k_clustered_ids():
    # the k best in a contiguous id range: few lists hold all of them, so
    # the lists overflow and the flagged query is answered exhaustively
    x = np.full((200_000, 8), 100.0, np.float32)
    x[5000:5300] = 1.0
    x[5000:5300, 0] = np.arange(300, dtype=np.float32) / 1000.0
    import mlxvs_amd
    ids, dist = mlxvs_amd.brute_force_knn(x, np.ones((1, 8), np.float32), 200, "l2")
    want = np.argsort(((x.astype(np.float64) - 1.0) ** 2).sum(1), kind="stable")[:200]
    assert np.array_equal(ids[0], want)


# ---- fp16 deep rows (d > 256): the K-looped kernel on the fp16 MFMA ----------------

@pytest.mark.parametrize("d", [288, 300, 512, 768, 1536])
@pytest.mark.parametrize("k", [10, 16, 64])
def test_fp16_deep_integer_bit_exact(engine, oracle, d, k):
    # binary16 integers in [0, 8): exact products and sums, so the answers
    # equal the restatement's bit for bit (d = 300: zero-padded to 320)
    rng = np.random.default_rng(d + k)
    base = rng.integers(0, 8, (20_000, d)).astype(np.float16)
    q = rng.integers(0, 8, (150, d)).astype(np.float16)
    for metric in ("l2", "inner_product"):
        ids, dist = engine.brute_force_knn(base, q, k, metric)
        oid, odist = oracle.knn(oracle.f16_to_f32(base), oracle.f16_to_f32(q), k, metric)
        assert np.array_equal(ids, oid), metric
        assert np.array_equal(dist, odist), metric


@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_fp16_deep_float(engine, oracle, metric):
    b = rows(30_000, 768, 11).astype(np.float16)
    q = rows(100, 768, 12).astype(np.float16)
    ids, dist = engine.brute_force_knn(b, q, 10, metric)
    check_float(oracle, ids, dist, oracle.f16_to_f32(b), oracle.f16_to_f32(q), 10, metric,
                tol=2e-3)


# ---- deep rows, small batches (<= 32 queries): the row-split deep kernel ------------

@pytest.mark.parametrize("nq", [1, 7, 32])
@pytest.mark.parametrize("d", [288, 512, 1536])
@pytest.mark.parametrize("k", [1, 10, 16, 64, 256])
def test_deep_small_batch_integer_bit_exact(engine, oracle, nq, d, k):
    # the four wavefronts take a tile's four row blocks against the same
    # queries (eight lists per split); n leaves a partial last tile
    rng = np.random.default_rng(nq * 100 + d + k)
    base = rng.integers(0, 16, (50_001, d)).astype(np.float32)
    q = rng.integers(0, 16, (nq, d)).astype(np.float32)
    for metric in ("l2", "inner_product"):
        ids, dist = engine.brute_force_knn(base, q, k, metric)
        oid, odist = oracle.knn(base, q, k, metric)
        assert np.array_equal(ids, oid), metric
        assert np.array_equal(dist, odist), metric


@pytest.mark.parametrize("nq", [1, 32])
@pytest.mark.parametrize("d", [320, 1536])
def test_deep_small_batch_fp16_integer_bit_exact(engine, oracle, nq, d):
    rng = np.random.default_rng(nq + d)
    base = rng.integers(0, 8, (40_000, d)).astype(np.float16)
    q = rng.integers(0, 8, (nq, d)).astype(np.float16)
    for k in (10, 64):
        ids, dist = engine.brute_force_knn(base, q, k, "l2")
        oid, odist = oracle.knn(oracle.f16_to_f32(base), oracle.f16_to_f32(q), k, "l2")
        assert np.array_equal(ids, oid)
        assert np.array_equal(dist, odist)


@pytest.mark.parametrize("nq", [1, 32])
@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_deep_small_batch_float(engine, oracle, nq, metric):
    base, q = rows(60_000, 768, 41), rows(nq, 768, 42)
    ids, dist = engine.brute_force_knn(base, q, 10, metric)
    check_float(oracle, ids, dist, base, q, 10, metric)


@pytest.mark.parametrize("n", [1, 31, 127, 128, 129, 1_000])
def test_deep_small_batch_small_n(engine, oracle, n):
    base, q = rows(n, 384, 43), rows(3, 384, 44)
    for k in (1, 10, 64):
        ids, dist = engine.brute_force_knn(base, q, k, "l2")
        check_float(oracle, ids, dist, base, q, k, "l2")


def test_deep_small_batch_ties_keep_lowest_ids(engine):
    # every row equal: the k lowest ids, spread over the four row blocks of
    # the first tile
    x = np.ones((20_000, 512), np.float32)
    ids, dist = engine.brute_force_knn(x, np.ones((2, 512), np.float32), 100, "l2")
    assert (ids == np.arange(100)).all() and (dist == 0).all()


# ---- many queries, k > T, heavy ties ---------------------------------------------

@pytest.mark.parametrize("k", [17, 64, 100])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_many_queries_large_k_integer_bit_exact(engine, oracle, k, dtype):
    # 40,000 queries (313 query blocks) and lists of 16 < k over few rows of
    # small integers: the shared bounds, the list overflow checks and the
    # lowest-id tie-break all see many equal scores
    rng = np.random.default_rng(k + (dtype == np.float16))
    base = rng.integers(0, 8, (6000, 24)).astype(dtype)
    q = rng.integers(0, 8, (40_000, 24)).astype(dtype)
    b32, q32 = base.astype(np.float32), q.astype(np.float32)
    for metric in ("l2", "inner_product"):
        ids, dist = engine.brute_force_knn(base, q, k, metric)
        oid, odist = oracle.knn(b32, q32, k, metric)
        assert np.array_equal(ids, oid), metric
        assert np.array_equal(dist, odist), metric


# ---- the device redo of flagged queries over many 4,096-row chunks -------------------

@pytest.mark.parametrize("nq", [5, 40])
@pytest.mark.parametrize("k", [100, 256])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_redo_skewed_rows_many_chunks(engine, oracle, nq, k, dtype):
    # scores that rise with the row id (rows ever closer to the queries, in
    # runs of equal distance): the k best lie in one split, so its lists
    # overflow and the query is flagged; the redo's exact select then sees
    # every chunk's rows at or above its bound, so its candidate count
    # crosses half the LDS buffer and the buffer itself within a chunk
    n = 61_000
    rng = np.random.default_rng(k + nq)
    base = np.zeros((n, 8), np.float32)
    base[:, 0] = (n - np.arange(n)) // 3          # runs of three equal rows
    base[:, 1] = rng.integers(0, 2, n)
    base = base.astype(dtype)
    q = rng.integers(0, 2, (nq, 8)).astype(dtype)
    b32, q32 = base.astype(np.float32), q.astype(np.float32)
    for metric in ("l2", "inner_product"):
        ids, dist = engine.brute_force_knn(base, q, k, metric)
        oid, odist = oracle.knn(b32, q32, k, metric)
        assert np.array_equal(ids, oid), metric
        assert np.array_equal(dist, odist), metric


def test_redo_skewed_hamming_many_chunks(engine, oracle):
    # Hamming: distance falls with the row id (runs of equal codes), k = 256
    n, nb = 50_000, 64
    bits = np.zeros((n, nb * 8), np.uint8)
    ones = (np.arange(n)[::-1] * (nb * 8) // n)
    bits[np.arange(nb * 8)[None, :] < ones[:, None]] = 1
    rows_ = np.packbits(bits, axis=1)
    q = np.zeros((40, nb), np.uint8)
    q[1::2, 0] = 1
    for k in (100, 256):
        ids, dist = engine.hamming_knn(rows_, q, k)
        oid, odist = oracle.hamming(rows_, q, k)
        assert np.array_equal(ids, oid)
        assert np.array_equal(dist, odist)
