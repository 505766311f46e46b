"""GPU parity of the IVF-Flat list scan (mlxvs_ivf_flat_search) with the CPU
restatement (oracle.ivf_flat, itself pinned by tests/test_oracle.py against
a float64 restatement of src/ivf.cpp:164-221, 327-416).

Bars: integer-valued data bit-exact (ids, tie order, distances, padding);
float data recall 1.0 against the restatement's scores within 1e-4; the
reference's own IVF-Flat tests (tests/test_ivf.cpp:62-115,
python/tests/test_mlxvs.py:610-634) as recall / self-match checks.
"""

import numpy as np
import pytest

import mlxvs_amd
from mlxvs_amd import _hip

pytestmark = pytest.mark.gpu


def int_rows(n, d, seed, hi=8):
    return np.random.default_rng(seed).integers(0, hi, (n, d)).astype(np.float32)


def ivf_index(x, lists):
    c = x[:: max(1, x.shape[0] // lists)][:lists].astype(np.float32)
    d2 = ((x[:, None, :].astype(np.float64) - c[None].astype(np.float64)) ** 2).sum(-1)
    lab = d2.argmin(1)
    order = np.argsort(lab, kind="stable")
    off = np.concatenate([[0], np.cumsum(np.bincount(lab, minlength=lists))]).astype(np.int32)
    return c, x[order].astype(np.float32), order.astype(np.int32), off


@pytest.mark.parametrize("metric", ["l2", "inner_product"])
@pytest.mark.parametrize("d", [16, 48, 300])
@pytest.mark.parametrize("n_probes,k", [(1, 4), (5, 10), (5, 16), (12, 40), (64, 128)])
def test_ivf_integer_exact(oracle, metric, d, n_probes, k):
    # k <= 16 and d <= 256: fused scan; otherwise candidate buffers + radix
    # select (d = 300: the VALU scan).  nq leaves a partial item.
    x = int_rows(6000, d, 1)
    q = int_rows(333, d, 2)
    c, data, ind, off = ivf_index(x, 64)
    ids, dist = mlxvs_amd.ivf_flat_search(c, data, ind, off, metric, q, k, n_probes=n_probes)
    wi, wd = oracle.ivf_flat(c, data, ind, off, q, k, n_probes, metric)
    assert np.array_equal(ids, wi)
    assert np.array_equal(dist, wd)


@pytest.mark.parametrize("metric", ["l2", "inner_product"])
@pytest.mark.parametrize("nq", [1, 3, 40])
@pytest.mark.parametrize("n_probes,k", [(1, 10), (7, 16), (20, 4), (64, 10)])
def test_ivf_small_batch_row_parts(oracle, metric, nq, n_probes, k):
    # few (query, probe) pairs: each list's rows are cut into parts scanned by
    # workgroups of their own (columns offset by the part's first row)
    x = int_rows(20_000, 32, 11)
    q = int_rows(nq, 32, 12)
    c, data, ind, off = ivf_index(x, 64)
    ids, dist = mlxvs_amd.ivf_flat_search(c, data, ind, off, metric, q, k, n_probes=n_probes)
    wi, wd = oracle.ivf_flat(c, data, ind, off, q, k, n_probes, metric)
    assert np.array_equal(ids, wi) and np.array_equal(dist, wd)


@pytest.mark.parametrize("lists,n_probes,nq", [(500, 100, 2000), (10_000, 80, 500)])
def test_ivf_device_plan_many_pairs(oracle, lists, n_probes, nq):
    # the work items planned on the device: many chunks of (query, probe)
    # pairs, more than 64 probes per query, and (10,000 lists) more lists
    # than the LDS bins hold
    rng = np.random.default_rng(lists)
    n, d = 30_000, 16
    lab = rng.integers(0, lists, n)
    order = np.argsort(lab, kind="stable")
    x = int_rows(n, d, 5)[order]
    off = np.concatenate([[0], np.cumsum(np.bincount(lab, minlength=lists))]).astype(np.int32)
    c = int_rows(lists, d, 6)
    q = int_rows(nq, d, 7)
    ids, dist = mlxvs_amd.ivf_flat_search(c, x, order.astype(np.int32), off, "l2", q, 10,
                                          n_probes=n_probes)
    wi, wd = oracle.ivf_flat(c, x, order.astype(np.int32), off, q, 10, n_probes, "l2")
    assert np.array_equal(ids, wi) and np.array_equal(dist, wd)


def test_ivf_short_lists_padding(oracle):
    x = int_rows(500, 8, 3)
    c, data, ind, off = ivf_index(x, 50)
    q = int_rows(20, 8, 4)
    for k in (10, 200):
        ids, dist = mlxvs_amd.ivf_flat_search(c, data, ind, off, "l2", q, k, n_probes=2)
        wi, wd = oracle.ivf_flat(c, data, ind, off, q, k, 2, "l2")
        assert np.array_equal(ids, wi) and np.array_equal(dist, wd)
    assert (ids[:, -1] == -1).all() and np.isinf(dist[:, -1]).all()


@pytest.mark.parametrize("k", [10, 50])
def test_ivf_cosine_float(oracle, k):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((8000, 64), dtype=np.float32)
    q = rng.standard_normal((200, 64), dtype=np.float32)
    u = (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)
    c, data, ind, off = ivf_index(u, 40)
    ids, dist = mlxvs_amd.ivf_flat_search(c, data, ind, off, "cosine", q, k, n_probes=6)
    wi, wd = oracle.ivf_flat(c, data, ind, off, q, k, 6, "cosine")
    np.testing.assert_allclose(dist, wd, atol=1e-5)
    # the same neighbours wherever the k-th and (k+1)-th scores are apart
    assert (ids == wi).mean() > 0.99


def test_ivf_device_api_matches_host_api():
    x = int_rows(5000, 32, 6)
    q = int_rows(150, 32, 7)
    c, data, ind, off = ivf_index(x, 32)
    ids, dist = mlxvs_amd.ivf_flat_search(c, data, ind, off, "l2", q, 10, n_probes=4)
    bufs = [_hip.DeviceBuffer.from_array(a) for a in (c, data, ind, off, q)]
    di, dd = _hip.DeviceBuffer(150 * 10 * 4), _hip.DeviceBuffer(150 * 10 * 4)
    mlxvs_amd.ivf_flat_search_device(bufs[0].value, 32, bufs[1].value, 5000, bufs[2].value,
                                     bufs[3].value, 32, "l2", bufs[4].value, 150, 10, di.value,
                                     dd.value, n_probes=4)
    _hip.synchronize()
    assert np.array_equal(di.download((150, 10), np.int32), ids)
    assert np.array_equal(dd.download((150, 10), np.float32), dist)


@pytest.mark.parametrize("metric", ["l2", "inner_product"])
@pytest.mark.parametrize("d,n_probes,k", [
    (32, 4, 10),     # fused scan, k <= 16
    (32, 6, 40),     # fused scan, k > 16: flagged queries searched again on the device
    (32, 3, 256),    # k > 16 with short lists: padding
    (300, 4, 10),    # rows longer than the fused scan takes: the exhaustive device route
    (300, 5, 64),
    (16, 200, 20),   # more probes than the fused merge holds: the exhaustive device route
])
def test_ivf_device_entry_routes(oracle, metric, d, n_probes, k):
    # the device entry plans from the device offsets alone (no host copy of
    # offsets or probes); every route matches the restatement bit for bit on
    # integer rows, and the host-array entry
    x = int_rows(6000, d, 21)
    q = int_rows(257, d, 22)
    c, data, ind, off = ivf_index(x, 250 if n_probes > 64 else 48)
    lists = c.shape[0]
    wi, wd = oracle.ivf_flat(c, data, ind, off, q, k, n_probes, metric)
    bufs = [_hip.DeviceBuffer.from_array(a) for a in (c, data, ind, off, q)]
    di, dd = _hip.DeviceBuffer(257 * k * 4), _hip.DeviceBuffer(257 * k * 4)
    mlxvs_amd.ivf_flat_search_device(bufs[0].value, lists, bufs[1].value, 6000, bufs[2].value,
                                     bufs[3].value, d, metric, bufs[4].value, 257, k, di.value,
                                     dd.value, n_probes=n_probes)
    _hip.synchronize()
    ids, dist = di.download((257, k), np.int32), dd.download((257, k), np.float32)
    assert np.array_equal(ids, wi) and np.array_equal(dist, wd)
    hi, hd = mlxvs_amd.ivf_flat_search(c, data, ind, off, metric, q, k, n_probes=n_probes)
    assert np.array_equal(hi, ids) and np.array_equal(hd, dist)


def test_ivf_argument_errors():
    x = int_rows(100, 4, 8)
    c, data, ind, off = ivf_index(x, 4)
    with pytest.raises(ValueError, match="columns"):
        mlxvs_amd.ivf_flat_search(c, data, ind, off, "l2", np.zeros((2, 5), np.float32), 3)
    with pytest.raises(ValueError, match="k must be"):
        mlxvs_amd.ivf_flat_search(c, data, ind, off, "l2", x[:2], 0)
    bad = off.copy()
    bad[1], bad[2] = bad[2], bad[1] - 1
    with pytest.raises(ValueError, match="offsets"):
        mlxvs_amd.ivf_flat_search(c, data, ind, bad, "l2", x[:2], 3)
    # n_probes is clamped to [1, lists]
    a, _ = mlxvs_amd.ivf_flat_search(c, data, ind, off, "l2", x[:5], 3, n_probes=0)
    b, _ = mlxvs_amd.ivf_flat_search(c, data, ind, off, "l2", x[:5], 3, n_probes=1)
    assert np.array_equal(a, b)


# ---- the reference's IVF-Flat tests ---------------------------------------------------

def low_rank(n, d, r, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, r)) @ rng.standard_normal((r, d))
            + 0.1 * rng.standard_normal((n, d))).astype(np.float32)


def recall(ids, exact):
    return np.mean([len(set(a) & set(b)) / len(b) for a, b in zip(ids.tolist(), exact.tolist())])


@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_ivf_build_search_recall(metric):
    # tests/test_ivf.cpp:62-90: 20000 x 48, 128 lists, recall@10 >= 0.9 at 16
    # probes and >= 0.999 with every list
    all_ = low_rank(20500, 48, 12, 51)
    x, q = all_[:20000], all_[20000:]
    index = mlxvs_amd.IvfFlatIndex.build(x, n_lists=128, metric=metric)
    exact, _ = mlxvs_amd.brute_force_knn(x, q, 10, metric)
    ids, dist = index.search(q, 10, n_probes=128)
    assert recall(ids, exact) >= 0.999
    ids, dist = index.search(q, 10, n_probes=16)
    assert recall(ids, exact) >= 0.9
    assert (ids >= 0).all()
    step = np.diff(dist, axis=1)
    assert (step >= -1e-4).all() if metric == "l2" else (step <= 1e-4).all()


def test_ivf_extend_and_save_load(tmp_path):
    # tests/test_ivf.cpp:92-115 and python/tests/test_mlxvs.py:610-634
    x = low_rank(12000, 32, 8, 61)
    index = mlxvs_amd.IvfFlatIndex.build(x[:10000], n_lists=64)
    index.extend(x[10000:])
    assert len(index) == 12000 and index.n_lists == 64
    ids, _ = index.search(x[10000:], 5, n_probes=64)
    assert (ids[:, 0] == np.arange(10000, 12000)).all()
    path = tmp_path / "ivf.safetensors"
    index.save(path)
    loaded = mlxvs_amd.IvfFlatIndex.load(path)
    a, _ = index.search(x[:300], 10, n_probes=16)
    b, _ = loaded.search(x[:300], 10, n_probes=16)
    assert np.array_equal(a, b) and loaded.metric == "l2"
    with pytest.raises(ValueError):
        index.extend(x[:5, :10])


def test_lists_of_16_repeated_calls(oracle):
    # k > 16 through lists of 16 with the rows of long lists cut into parts:
    # items of fewer than 128 pairs leave wavefronts without queries, so the
    # scanning wavefronts often reach the tile barrier last and read their
    # accumulators right after it.  Read too soon after the last MFMA, the
    # last accumulator registers held stale values now and then (a list lost
    # a candidate); every call of several must be exact.
    x = int_rows(6000, 16, 1)
    q = int_rows(333, 16, 2)
    c, data, ind, off = ivf_index(x, 64)
    for k in (17, 24, 40, 64):
        wi, wd = oracle.ivf_flat(c, data, ind, off, q, k, 12, "l2")
        for rep in range(4):
            ids, dist = mlxvs_amd.ivf_flat_search(c, data, ind, off, "l2", q, k, n_probes=12)
            assert np.array_equal(ids, wi), (k, rep)
            assert np.array_equal(dist, wd), (k, rep)
