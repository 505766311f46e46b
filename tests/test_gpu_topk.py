"""GPU parity of topk_merge (reference src/knn.cpp:37-69, src/kernels.h:37-229)
with the CPU restatement (oracle_topk_merge, pinned in tests/test_oracle.py).

The selection and output order are integer work on the scores' bits (keys,
unsigned ids), so the bar is bit-exact: ids and scores, including the sign of
zero scores and the -1 / -inf padding.  Cases: first and running lists, id
offsets (negative ones wrap as int32), k in {1, 10, 100, 256}, fewer
candidates than k, all-equal and +-0 scores, row lengths around the kernel's
chunk boundaries (16,384 scores per chunk) and up to 70,000, unaligned rows,
the host and device entries, a stream, and outputs written over the running
lists in place.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def same(a, b):
    """Bit-equal float32 arrays (so -0.0 differs from +0.0)."""
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def check(engine, oracle, S, k, off=0, prev=None):
    first = prev is None
    pi, pb = (None, None) if first else prev
    gi, gs = engine.topk_merge(S, pi, pb, off, first, k)
    oi, os_ = oracle.topk_merge(S, pi, pb, off, first, k)
    bad = np.flatnonzero((gi != oi).any(1))
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5]}: {gi[bad[0]]} vs {oi[bad[0]]}"
    assert same(gs, os_)


def scores(nq, t, seed, kind="normal"):
    g = np.random.default_rng(seed)
    if kind == "normal":
        return g.standard_normal((nq, t), dtype=np.float32)
    if kind == "int":  # heavy ties
        return g.integers(-20, 20, (nq, t)).astype(np.float32)
    if kind == "equal":
        return np.full((nq, t), 1.5, np.float32)
    if kind == "zeros":  # +0 and -0 only
        return np.where(g.random((nq, t)) < 0.5, np.float32(-0.0), np.float32(0.0))
    raise ValueError(kind)


@pytest.mark.parametrize("k", [1, 10, 100, 256])
@pytest.mark.parametrize("t", [1, 7, 100, 1024, 1025, 4096, 4097, 16384, 16385, 65536, 70001])
def test_first(engine, oracle, t, k):
    nq = 48 if t <= 16385 else 12
    check(engine, oracle, scores(nq, t, t * 7 + k), k)


@pytest.mark.parametrize("kind", ["int", "equal", "zeros"])
@pytest.mark.parametrize("t,k", [(300, 10), (5000, 100), (20000, 256), (40000, 7)])
def test_ties(engine, oracle, kind, t, k):
    check(engine, oracle, scores(6, t, t + k, kind), k)


@pytest.mark.parametrize("off", [0, 1_000_000, -5, -70_000, 2**31 - 100])
def test_id_offsets(engine, oracle, off):
    check(engine, oracle, scores(8, 20000, 4, "int"), 50, off)
    check(engine, oracle, scores(8, 20000, 5, "equal"), 50, off)


@pytest.mark.parametrize("t,k", [(0, 10), (3, 10), (100, 10), (9000, 64), (16384, 256),
                                 (33000, 256)])
@pytest.mark.parametrize("kind", ["normal", "int"])
def test_running_lists(engine, oracle, t, k, kind):
    nq = 16
    g = np.random.default_rng(t + k)
    if kind == "normal":
        pb = g.standard_normal((nq, k), dtype=np.float32) + 1.0
    else:
        pb = g.integers(-20, 20, (nq, k)).astype(np.float32)
    pi = g.integers(0, 100_000, (nq, k)).astype(np.int32)
    check(engine, oracle, scores(nq, t, t, kind), k, 500, (pi, pb))


def test_running_lists_initial_padding(engine, oracle):
    # the reference's initial lists (-1 / -inf) passed with first = false:
    # they are candidates, so a short row keeps copies of them
    k = 20
    pi = np.full((5, k), -1, np.int32)
    pb = np.full((5, k), -np.inf, np.float32)
    check(engine, oracle, scores(5, 7, 1), k, 0, (pi, pb))
    check(engine, oracle, scores(5, 70, 2), k, 0, (pi, pb))


def test_tiles_chained_like_brute_force(engine, oracle):
    # src/knn.cpp:104-121: one merge per 65,536-score tile with the running
    # lists; the chained result equals one merge of the whole row
    S = scores(16, 3 * 65536 + 1000, 9)
    k = 10
    ids = best = None
    for t0 in range(0, S.shape[1], 65536):
        ids, best = engine.topk_merge(np.ascontiguousarray(S[:, t0:t0 + 65536]), ids, best, t0,
                                      t0 == 0, k)
    oi, os_ = oracle.topk_merge(S, None, None, 0, True, k)
    assert np.array_equal(ids, oi) and same(best, os_)


def test_unaligned_rows(engine, oracle):
    # t % 4 != 0 and a base that is not 16-byte aligned take the scalar loads
    S = scores(10, 5003, 3)
    check(engine, oracle, S, 30)
    buf = np.empty(10 * 5000 + 1, np.float32)
    view = buf[1:].reshape(10, 5000)
    view[...] = scores(10, 5000, 4)
    assert view.ctypes.data % 16 != 0
    check(engine, oracle, view, 30)


def test_many_rows(engine, oracle):
    check(engine, oracle, scores(5000, 200, 8, "int"), 16)


def test_device_in_place_on_a_stream(engine, oracle):
    from mlxvs_amd import _hip

    nq, t, k = 64, 30000, 32
    S = scores(nq, t, 12)
    g = np.random.default_rng(13)
    pb = (g.standard_normal((nq, k), dtype=np.float32) + 2.5)
    pi = g.integers(0, 10**6, (nq, k)).astype(np.int32)
    oi, os_ = oracle.topk_merge(S, pi, pb, 7, False, k)
    ds = _hip.DeviceBuffer.from_array(S)
    di = _hip.DeviceBuffer.from_array(pi)
    db = _hip.DeviceBuffer.from_array(pb)
    st = _hip.Stream()
    # outputs written over the running lists
    engine.topk_merge_device(ds.value, nq, t, di.value, db.value, 7, False, k, di.value,
                             db.value, stream=st.handle.value)
    st.synchronize()
    assert np.array_equal(di.download((nq, k), np.int32), oi)
    assert same(db.download((nq, k), np.float32), os_)
    # first: the running lists are not read (null), scores output optional
    out = _hip.DeviceBuffer(nq * k * 4)
    engine.topk_merge_device(ds.value, nq, t, None, None, 0, True, k, out.value, None)
    _hip.synchronize()
    oi2, _ = oracle.topk_merge(S, None, None, 0, True, k)
    assert np.array_equal(out.download((nq, k), np.int32), oi2)


# Rows whose candidate count crosses half of the kernel's 4,096-rank buffer
# (and the whole of it) while a chunk is being appended: every wavefront
# must take the same compaction / overflow decision on that count (a
# wavefront that read it after another had appended took the other branch,
# whose barriers the rest skipped).  Ascending rows put every element of a
# chunk above the bound; the stepped rows put about 2,500 per chunk there;
# the sawtooth mixes both.
def patterned(nq, t, kind, seed):
    g = np.random.default_rng(seed)
    c = np.arange(t, dtype=np.float64)
    if kind == "ascending":
        s = np.broadcast_to(c, (nq, t)) + g.integers(0, 3, (nq, t))
    elif kind == "stepped":
        # per chunk of 8,192: 2,500 elements above everything before
        blk = (c // 8192)
        hi = (c % 8192) < 2500
        s = np.broadcast_to(np.where(hi, 1000.0 * blk + (c % 8192) % 97, -1e6 + c % 13),
                            (nq, t)) + g.integers(0, 2, (nq, t))
    else:  # sawtooth
        s = np.broadcast_to((c % 6000) + (c // 6000) * 10.0, (nq, t)) + g.integers(0, 2, (nq, t))
    return np.ascontiguousarray(s, dtype=np.float32)


@pytest.mark.parametrize("kind", ["ascending", "stepped", "sawtooth"])
@pytest.mark.parametrize("t,k", [(4 * 8192 + 77, 256), (12 * 8192, 256), (5 * 4096, 100),
                                 (3000, 256)])
def test_count_crossing_within_a_chunk(engine, oracle, kind, t, k):
    check(engine, oracle, patterned(24, t, kind, t + k), k)


@pytest.mark.parametrize("kind", ["ascending", "stepped"])
def test_count_crossing_with_running_lists(engine, oracle, kind):
    nq, t, k = 16, 6 * 8192, 256
    g = np.random.default_rng(3)
    pb = g.integers(0, 60_000, (nq, k)).astype(np.float32)
    pi = g.integers(0, 100_000, (nq, k)).astype(np.int32)
    check(engine, oracle, patterned(nq, t, kind, 5), k, 11, (pi, pb))
