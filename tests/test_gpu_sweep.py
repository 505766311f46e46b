"""A seeded sweep over shapes, list lengths and metrics: the HIP engine
against the CPU restatement, bit for bit (exact k-NN over fp32 and fp16
rows, Hamming codes, IVF-Flat, the self k-NN graph and topk_merge).

Every case draws its sizes from a fixed generator (log-uniform row and
query counts, dimensions, code widths and k up to 256), so the sweep
reaches the plan's corners -- one split or hundreds, k below, at and
above the list lengths, merges of one level or several, partial tiles --
that the named cases cover only in part.  Inputs are small integers, so
every score is exact in fp32 (and in the fp16 path's fp32 accumulation)
and the results must equal the restatement's exactly; Hamming codes are
random bytes.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

WORK = 1.5e9  # rows x queries x dims per case (bounds the restatement's time)


def log_int(rng, lo, hi):
    return int(np.exp(rng.uniform(np.log(lo), np.log(hi + 1))))


def float_case(seed):
    rng = np.random.default_rng(1000 + seed)
    f16 = seed % 4 == 3
    n = log_int(rng, 1, 60_000)
    d = log_int(rng, 1, 256 if f16 else 400)
    k = log_int(rng, 1, 256)
    nq = max(1, min(log_int(rng, 1, 400), int(WORK / max(1, n * d))))
    metric = "l2" if seed % 2 == 0 else "inner_product"
    return rng, f16, n, nq, d, k, metric


@pytest.mark.parametrize("seed", range(64))
def test_float_sweep(engine, oracle, seed):
    rng, f16, n, nq, d, k, metric = float_case(seed)
    dt = np.float16 if f16 else np.float32
    base = rng.integers(-4, 5, (n, d)).astype(dt)
    q = rng.integers(-4, 5, (nq, d)).astype(dt)
    ids, dist = engine.brute_force_knn(base, q, k, metric)
    ob = oracle.f16_to_f32(base) if f16 else base
    oq = oracle.f16_to_f32(q) if f16 else q
    oid, odist = oracle.knn(ob, oq, k, metric)
    case = f"n={n} nq={nq} d={d} k={k} {metric} {'fp16' if f16 else 'fp32'}"
    assert np.array_equal(ids, oid), case
    assert np.array_equal(dist, odist), case


@pytest.mark.parametrize("seed", range(40))
def test_hamming_sweep(engine, oracle, seed):
    rng = np.random.default_rng(2000 + seed)
    nbytes = log_int(rng, 1, 300)
    n = log_int(rng, 1, 200_000)
    k = log_int(rng, 1, 256)
    nq = max(1, min(log_int(rng, 1, 600), int(WORK / max(1, n * nbytes))))
    x = rng.integers(0, 256, (n, nbytes), dtype=np.uint8)
    q = rng.integers(0, 256, (nq, nbytes), dtype=np.uint8)
    ids, dist = engine.hamming_knn(x, q, k)
    oid, odist = oracle.hamming(x, q, k)
    case = f"n={n} nq={nq} bytes={nbytes} k={k}"
    assert np.array_equal(ids, oid), case
    assert np.array_equal(dist, odist), case


def ivf_index(x, lists):
    c = x[:: max(1, x.shape[0] // lists)][:lists].astype(np.float32)
    d2 = ((x[:, None, :].astype(np.float64) - c[None].astype(np.float64)) ** 2).sum(-1)
    lab = d2.argmin(1)
    order = np.argsort(lab, kind="stable")
    off = np.concatenate([[0], np.cumsum(np.bincount(lab, minlength=c.shape[0]))]).astype(np.int32)
    return c, x[order].astype(np.float32), order.astype(np.int32), off


@pytest.mark.parametrize("seed", range(32))
def test_ivf_sweep(oracle, seed):
    import mlxvs_amd

    rng = np.random.default_rng(3000 + seed)
    n = log_int(rng, 1, 20_000)
    d = log_int(rng, 1, 300)
    lists = max(1, min(n, log_int(rng, 1, 256)))
    nq = log_int(rng, 1, 500)
    n_probes = max(1, min(lists, log_int(rng, 1, 64)))
    k = log_int(rng, 1, 256)
    metric = "l2" if seed % 2 == 0 else "inner_product"
    x = rng.integers(-4, 5, (n, d)).astype(np.float32)
    q = rng.integers(-4, 5, (nq, d)).astype(np.float32)
    c, data, ind, off = ivf_index(x, lists)
    ids, dist = mlxvs_amd.ivf_flat_search(c, data, ind, off, metric, q, k, n_probes=n_probes)
    wi, wd = oracle.ivf_flat(c, data, ind, off, q, k, n_probes, metric)
    case = f"n={n} d={d} lists={c.shape[0]} nq={nq} probes={n_probes} k={k} {metric}"
    assert np.array_equal(ids, wi), case
    assert np.array_equal(dist, wd), case


@pytest.mark.parametrize("seed", range(24))
def test_self_graph_sweep(engine, oracle, seed):
    rng = np.random.default_rng(4000 + seed)
    f16 = seed % 3 == 2
    n = max(2, log_int(rng, 1, 20_000))  # the route needs two rows
    d = log_int(rng, 1, 256)
    k = log_int(rng, 1, 128)
    metric = "l2" if seed % 2 == 0 else "inner_product"
    x = rng.integers(-4, 5, (n, d)).astype(np.float16 if f16 else np.float32)
    ids, dist = engine.all_neighbors(x, k, metric)
    oid, odist = oracle.self_graph(oracle.f16_to_f32(x) if f16 else x, k, metric)
    case = f"n={n} d={d} k={k} {metric} {'fp16' if f16 else 'fp32'}"
    assert np.array_equal(ids, oid), case
    assert np.array_equal(dist, odist), case


@pytest.mark.parametrize("seed", range(24))
def test_topk_merge_sweep(engine, oracle, seed):
    rng = np.random.default_rng(5000 + seed)
    nq = log_int(rng, 1, 300)
    t = log_int(rng, 1, 70_000)
    k = log_int(rng, 1, 256)
    first = seed % 3 != 0
    off = int(rng.integers(-(1 << 20), 1 << 20))
    s = rng.integers(-30, 30, (nq, t)).astype(np.float32)
    if first:
        pi = pb = None
    else:
        pb = np.sort(rng.integers(-30, 30, (nq, k)).astype(np.float32), axis=1)[:, ::-1].copy()
        pi = rng.integers(0, 1 << 20, (nq, k)).astype(np.int32)
    gi, gs = engine.topk_merge(s, pi, pb, off, first, k)
    oi, os_ = oracle.topk_merge(s, pi, pb, off, first, k)
    case = f"nq={nq} t={t} k={k} first={first} off={off}"
    assert np.array_equal(gi, oi), case
    assert np.array_equal(np.asarray(gs, np.float32).view(np.uint32),
                          np.asarray(os_, np.float32).view(np.uint32)), case


def test_device_calls_queued_on_two_streams(engine, oracle):
    # 24 device calls of mixed shapes and routes (float fp32 / fp16, Hamming,
    # self graph) queued back to back on two streams with no wait between
    # them: each call's workspace is reused by the next, so every result must
    # still equal the restatement's once both streams drain
    from mlxvs_amd import _hip

    streams = [_hip.Stream(), _hip.Stream()]
    keep, checks = [], []
    rng = np.random.default_rng(6000)
    for i in range(24):
        st = streams[i % 2].handle.value
        kind = ("float", "f16", "hamming", "self")[i % 4]
        n, k = log_int(rng, 2, 30_000), log_int(rng, 1, 200)
        if kind == "hamming":
            nbytes, nq = log_int(rng, 1, 128), log_int(rng, 1, 300)
            x = rng.integers(0, 256, (n, nbytes), dtype=np.uint8)
            q = rng.integers(0, 256, (nq, nbytes), dtype=np.uint8)
            dx, dq = _hip.DeviceBuffer.from_array(x), _hip.DeviceBuffer.from_array(q)
            di, dd = _hip.DeviceBuffer(nq * k * 4), _hip.DeviceBuffer(nq * k * 4)
            engine.hamming_knn_device(dx.value, n, dq.value, nq, nbytes, k, di.value, dd.value,
                                      stream=st)
            want = lambda x=x, q=q, k=k: oracle.hamming(x, q, k)
        elif kind == "self":
            d = log_int(rng, 1, 128)
            x = rng.integers(-4, 5, (n, d)).astype(np.float32)
            nq = n
            dx = _hip.DeviceBuffer.from_array(x)
            dq = None
            di, dd = _hip.DeviceBuffer(n * k * 4), _hip.DeviceBuffer(n * k * 4)
            engine.knn_self_graph_device(dx.value, n, d, k, "l2", di.value, dd.value, stream=st)
            want = lambda x=x, k=k: oracle.self_graph(x, k, "l2")
        else:
            f16 = kind == "f16"
            d, nq = log_int(rng, 1, 256), log_int(rng, 1, 500)
            metric = "l2" if i % 3 else "inner_product"
            dt = np.float16 if f16 else np.float32
            x = rng.integers(-4, 5, (n, d)).astype(dt)
            q = rng.integers(-4, 5, (nq, d)).astype(dt)
            dx, dq = _hip.DeviceBuffer.from_array(x), _hip.DeviceBuffer.from_array(q)
            di, dd = _hip.DeviceBuffer(nq * k * 4), _hip.DeviceBuffer(nq * k * 4)
            engine.brute_force_knn_device(dx.value, n, dq.value, nq, d, k, metric, di.value,
                                          dd.value, f16=f16, stream=st)
            ox = oracle.f16_to_f32(x) if f16 else x
            oq = oracle.f16_to_f32(q) if f16 else q
            want = lambda ox=ox, oq=oq, k=k, metric=metric: oracle.knn(ox, oq, k, metric)
        keep.append((dx, dq, di, dd))
        checks.append((f"call {i} {kind} n={n} nq={nq} k={k}", di, dd, nq, k, want))
    for s in streams:
        s.synchronize()
    for case, di, dd, nq, k, want in checks:
        ids = di.download((nq, k), np.int32)
        dist = dd.download((nq, k), np.float32)
        oid, odist = want()
        assert np.array_equal(ids, oid), case
        assert np.array_equal(dist, odist), case
