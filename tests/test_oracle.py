"""Pins the CPU restatement (oracle/) before it is trusted as the checker.

Each check is independent of the restatement's own arithmetic: float64 NumPy
brute force with an np.lexsort (score desc, id asc) tie-break, scipy's cdist,
an 8-bit popcount table, the committed float64 golden fixtures
(tests/golden/make_golden.py) and the reference's known-answer tests.  Each
is chosen so that a plausible mistake (a flipped sign in the L2 epilogue, a
dropped |b|^2 term, highest-id instead of lowest-id ties, a transposed
operand, an off-by-one in padding) fails at least one of them.
"""

from pathlib import Path

import numpy as np
import pytest

from mlxvs_amd import synth

GOLDEN = Path(__file__).resolve().parent / "golden"


def int_rows(n, d, seed, hi=16):
    return np.random.default_rng(seed).integers(0, hi, (n, d)).astype(np.float32)


def rows(n, d, seed):
    return np.random.default_rng(seed).standard_normal((n, d), dtype=np.float32)


# ---- ordering key (src/kernels.h:16-19) ---------------------------------------

def test_key_orders_floats(oracle):
    vals = [-np.inf, -1e30, -1.0, -1e-30, -0.0, 0.0, 1e-30, 1.0, 1e30, np.inf]
    keys = [oracle.key(v) for v in vals]
    assert keys == sorted(keys) and len(set(keys)) == len(keys)
    assert oracle.key(-0.0) + 1 == oracle.key(0.0)
    assert oracle.key(float("nan")) > oracle.key(np.inf)


# ---- exact integer data: bit-exact against float64 ---------------------------

@pytest.mark.parametrize("metric", ["l2", "inner_product"])
@pytest.mark.parametrize("n,nq,d,k", [(500, 20, 8, 10), (3000, 16, 32, 64),
                                      (50, 8, 16, 100), (1000, 5, 3, 256)])
def test_integer_data_exact(oracle, metric, n, nq, d, k):
    b, q = int_rows(n, d, 1), int_rows(nq, d, 2)  # heavy ties
    ids, dist = oracle.knn(b, q, k, metric)
    s = oracle.exact_scores(q, b, metric)
    want = oracle.exact_topk(s, k)
    assert np.array_equal(ids, want)
    keff = min(k, n)
    got = np.take_along_axis(s, want[:, :keff], 1)
    exp = -got if metric == "l2" else got
    assert np.array_equal(dist[:, :keff], exp.astype(np.float32))
    pad = np.inf if metric == "l2" else -np.inf
    assert (dist[:, keff:] == pad).all() and (ids[:, keff:] == -1).all()


def test_l2_matches_scipy_cdist(oracle):
    from scipy.spatial.distance import cdist

    b, q = int_rows(800, 24, 3, hi=256), int_rows(30, 24, 4, hi=256)
    ids, dist = oracle.knn(b, q, 15, "l2")
    full = cdist(q.astype(np.float64), b.astype(np.float64), "sqeuclidean")
    assert np.array_equal(dist, np.take_along_axis(full, ids.astype(np.int64), 1))
    assert np.array_equal(np.sort(full, 1)[:, :15], dist)


@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_float_data_recall(oracle, metric):
    b, q = rows(4000, 48, 5), rows(40, 48, 6)
    ids, dist = oracle.knn(b, q, 20, metric)
    s = oracle.exact_scores(q, b, metric)
    assert oracle.recall(ids, s, 20) == 1.0
    exact = np.take_along_axis(s, ids, 1)
    exact = -exact if metric == "l2" else exact
    assert (np.abs(exact - dist) / np.maximum(1, np.abs(exact))).max() < 1e-4


def test_cosine_zero_query_and_rows(oracle):
    # unit_rows divides by max(|x|, 1e-30): a zero row stays zero and scores 0
    b = rows(100, 8, 7)
    b[::7] = 0
    q = np.zeros((2, 8), np.float32)
    ids, dist = oracle.knn(b, q, 5, "cosine")
    assert (dist == 0).all() and (ids == np.arange(5)).all()


def test_ties_kat(oracle):
    # tests/test_knn.cpp:156-192
    g = np.load(GOLDEN / "kat_ties.npz")
    ids, dist = oracle.knn(g["base"], g["queries"], 10, "l2")
    assert np.array_equal(ids, g["ids"]) and (dist == 0).all()


def test_fewer_rows_than_k(oracle):
    # python/tests/test_mlxvs.py:63-69
    b, q = rows(5, 8, 3), rows(4, 8, 4)
    ids, dist = oracle.knn(b, q, 8, "l2")
    assert (ids[:, :5] >= 0).all() and (ids[:, 5:] == -1).all()
    assert np.isinf(dist[:, 5:]).all() and (dist[:, 5:] > 0).all()
    assert sorted(ids[0, :5].tolist()) == list(range(5))


def test_argument_checks(oracle):
    b = rows(10, 4, 1)
    with pytest.raises(ValueError):
        oracle.knn(b, b, 300, "l2")
    with pytest.raises(ValueError):
        oracle.knn(b, b, 0, "l2")
    ids, dist = oracle.knn(np.zeros((0, 4), np.float32), b[:2], 3, "l2")
    assert (ids == -1).all() and (dist == np.inf).all()


# ---- golden fixtures ---------------------------------------------------------------

def test_c1_golden(oracle):
    base = synth.c1_rows(1, 0, 10_000)
    q = synth.c1_rows(2, 0, 100)
    g = np.load(GOLDEN / "c1_full.npz")
    ids, dist = oracle.knn(base, q, 10, "l2")
    assert np.array_equal(ids, g["ids"])
    assert np.array_equal(dist, g["dist"].astype(np.float32))


def test_c2_golden(oracle):
    cen = synth.c2_centres()
    base = synth.chunked(lambda lo, hi: synth.c2_rows(1, lo, hi, centres=cen), 1_000_000)
    q = synth.c2_rows(2, 0, 64, centres=cen)
    g = np.load(GOLDEN / "c2_subset.npz")
    ids, dist = oracle.knn(base, q, 10, "l2")
    assert np.array_equal(ids, g["ids"])
    assert np.array_equal(dist, g["dist"].astype(np.float32))


def test_c3_golden(oracle):
    cen = synth.c3_centres()
    base = synth.chunked(lambda lo, hi: synth.c3_rows(1, lo, hi, centres=cen), 100_000,
                         chunk=5_000)
    q = synth.c3_rows(2, 0, 16, centres=cen)
    g = np.load(GOLDEN / "c3_subset.npz")
    for metric, key in (("inner_product", "ip"), ("cosine", "cos")):
        ids, dist = oracle.knn(base, q, 10, metric)
        np.testing.assert_allclose(dist, g["score_" + key][:16], atol=1e-4)
        s = oracle.exact_scores(q, base, metric)
        assert oracle.recall(ids, s, 10) == 1.0


def test_c4_golden(oracle):
    gen = lambda lo, hi: synth.c4_codes(1, lo, hi)  # noqa: E731
    base = synth.chunked(gen, 1_000_000)
    q, src = synth.c4_queries(gen, 1_000_000, 2, 0, 32)
    g = np.load(GOLDEN / "c4_subset.npz")
    ids, dist = oracle.hamming(base, q, 100)
    assert np.array_equal(ids, g["ids"])
    assert np.array_equal(dist, g["dist"].astype(np.float32))
    assert (ids[:, 0] == src).all() and (dist[:, 0] == 51).all()


def test_c5_golden(oracle):
    cen = synth.c5_centres()
    x = synth.chunked(lambda lo, hi: synth.c5_rows(1, lo, hi, centres=cen), 200_000)
    xf = oracle.f16_to_f32(x)
    g = np.load(GOLDEN / "c5_subset.npz")
    ids, dist = oracle.self_graph_rows(xf, 64, 32, "l2")
    assert (ids != np.arange(32)[:, None]).all()
    np.testing.assert_allclose(dist, g["dist"], rtol=1e-4)
    assert (ids == g["ids"]).mean() > 0.98


# ---- Hamming (src/ivf.cpp:1343-1403) ------------------------------------------------

def test_hamming_tiny_kat(oracle):
    # python/tests/test_cuvs.py:840-848
    codes = np.array([[0b1111, 0], [0b1, 0]], dtype=np.uint8)
    ids, dist = oracle.hamming(codes, codes[:1], 2)
    assert ids[0].tolist() == [0, 1] and dist[0].tolist() == [0.0, 3.0]


@pytest.mark.parametrize("nbytes", [1, 3, 16, 128])
def test_hamming_vs_popcount_table(oracle, nbytes):
    # python/tests/test_cuvs.py:772-793
    rng = np.random.default_rng(11)
    data = rng.integers(0, 256, (700, nbytes), dtype=np.uint8)
    q = rng.integers(0, 256, (40, nbytes), dtype=np.uint8)
    ids, dist = oracle.hamming(data, q, 7)
    h = oracle.hamming_distances(q, data)
    order = np.lexsort((np.broadcast_to(np.arange(700), h.shape), h), axis=1)[:, :7]
    assert np.array_equal(ids, order)
    assert np.array_equal(dist, np.take_along_axis(h, order, 1).astype(np.float32))


def test_hamming_padding_and_empty(oracle):
    x = np.arange(24, dtype=np.uint8).reshape(6, 4)
    ids, dist = oracle.hamming(x, x[:2], 10)
    assert (ids[:, 6:] == -1).all() and (dist[:, 6:] == np.inf).all()
    ids, dist = oracle.hamming(np.zeros((0, 4), np.uint8), x[:2], 3)
    assert (ids == -1).all() and (dist == np.inf).all()
    with pytest.raises(ValueError):
        oracle.hamming(x, x, 0)


def test_pack_words_little_endian(oracle):
    r = np.arange(1, 8, dtype=np.uint8).reshape(1, 7)
    w = oracle.pack_words(r)
    assert w.tolist() == [[0x04030201, 0x00070605]]


# ---- self graph (src/all_neighbors.cpp:56-95, 250-263) --------------------------------

@pytest.mark.parametrize("metric", ["l2", "inner_product", "cosine"])
def test_self_graph_vs_float64(oracle, metric):
    x = int_rows(400, 6, 9, hi=8)  # many ties and duplicate rows
    ids, dist = oracle.self_graph(x, 7, metric)
    s = oracle.exact_scores(x, x, metric)
    np.fill_diagonal(s, -np.inf)
    want = oracle.exact_topk(s, 7)
    if metric != "cosine":  # cosine: float32 rounding decides near-ties
        assert np.array_equal(ids, want)
    assert (ids != np.arange(400)[:, None]).all()


def test_f16_to_f32_all_patterns(oracle):
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    got = oracle.f16_to_f32(h)
    want = h.astype(np.float32)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    assert np.array_equal(np.signbit(got), np.signbit(want))


# ---- IVF-Flat search (src/ivf.cpp:164-221, 327-416; src/ivf_kernels.h:16-99) --------

def ivf_index(x, lists, seed):
    """A deterministic index: centers = every (n // lists)-th row, each row
    in the list of its nearest center (float64, lowest index on ties), rows of
    a list in input order.  Some lists may stay empty."""
    c = x[:: max(1, x.shape[0] // lists)][:lists].astype(np.float32)
    d2 = ((x[:, None, :].astype(np.float64) - c[None].astype(np.float64)) ** 2).sum(-1)
    lab = d2.argmin(1)
    order = np.argsort(lab, kind="stable")
    off = np.concatenate([[0], np.cumsum(np.bincount(lab, minlength=lists))]).astype(np.int32)
    return c, x[order].astype(np.float32), order.astype(np.int32), off


def ivf_float64(centers, data, indices, offsets, queries, k, n_probes, metric):
    """Independent float64 restatement of the reference's IVF-Flat search."""
    c, x, q = (a.astype(np.float64) for a in (centers, data, queries))
    lists = c.shape[0]
    P = min(max(n_probes, 1), lists)
    if metric == "inner_product":
        ps = q @ c.T
    else:
        ps = -((q[:, None, :] - c[None]) ** 2).sum(-1)
    probes = np.array([np.lexsort((np.arange(lists), -row))[:P] for row in ps])
    sizes = np.diff(offsets)
    width = max(1, int(sizes[probes].sum(1).max()))
    kk = min(k, width)
    ids = np.full((q.shape[0], k), -1, np.int32)
    dist = np.full((q.shape[0], k), np.inf if metric == "l2" else -np.inf, np.float32)
    for i in range(q.shape[0]):
        pos = np.concatenate([np.arange(offsets[l], offsets[l + 1]) for l in probes[i]])
        if metric == "l2":
            sc = -((x[pos] - q[i]) ** 2).sum(1)
        else:
            sc = x[pos] @ q[i]
        cols = np.arange(pos.size)
        order = np.lexsort((cols, -sc))[:kk]
        ids[i, :order.size] = indices[pos[order]]
        dist[i, :order.size] = -sc[order] if metric == "l2" else sc[order]
    return ids, dist


@pytest.mark.parametrize("metric", ["l2", "inner_product"])
@pytest.mark.parametrize("n_probes,k", [(1, 5), (3, 10), (8, 40), (100, 7)])
def test_ivf_flat_vs_float64(oracle, metric, n_probes, k):
    # integer data: every score is exact in float32, so the restatement must
    # equal the float64 one bit for bit, including its tie order (probe
    # order, then row order) and the -1 padding when the lists run short
    x = int_rows(3000, 12, 21, hi=6)
    q = int_rows(70, 12, 22, hi=6)
    c, data, ind, off = ivf_index(x, 37, 0)
    ids, dist = oracle.ivf_flat(c, data, ind, off, q, k, n_probes, metric)
    wi, wd = ivf_float64(c, data, ind, off, q, k, n_probes, metric)
    assert np.array_equal(ids, wi)
    assert np.array_equal(dist, wd)


def test_ivf_flat_all_lists_is_brute_force(oracle):
    x = int_rows(2000, 8, 23, hi=8)
    q = int_rows(50, 8, 24, hi=8)
    c, data, ind, off = ivf_index(x, 20, 0)
    ids, dist = oracle.ivf_flat(c, data, ind, off, q, 10, 20, "l2")
    bid, bdist = oracle.knn(x, q, 10, "l2")
    assert np.array_equal(dist, bdist)  # same distances; ties may differ in id


def test_ivf_flat_short_lists_and_cosine(oracle):
    x = int_rows(300, 6, 25, hi=8)
    c, data, ind, off = ivf_index(x, 30, 0)
    q = int_rows(10, 6, 26, hi=8)
    ids, dist = oracle.ivf_flat(c, data, ind, off, q, 256, 2, "l2")
    wi, wd = ivf_float64(c, data, ind, off, q, 256, 2, "l2")
    assert np.array_equal(ids, wi) and np.array_equal(dist, wd)
    assert (ids[:, -1] == -1).all() and np.isinf(dist[:, -1]).all()
    # cosine: queries unit-normalised, data stored as unit rows
    u = x / np.maximum(np.linalg.norm(x, axis=1, keepdims=True), 1e-30)
    c, data, ind, off = ivf_index(u.astype(np.float32), 30, 0)
    ids, dist = oracle.ivf_flat(c, data, ind, off, q, 5, 4, "cosine")
    qn = q / np.linalg.norm(q, axis=1, keepdims=True)
    wi, wd = ivf_float64(c, data, ind, off, qn, 5, 4, "cosine")
    np.testing.assert_allclose(dist, wd, atol=1e-6)


# ---- topk_merge (src/knn.cpp:37-69, src/kernels.h:37-229) ----------------------

def _lexsort_best(S, k, id_offset=0):
    """The k best columns of every row by (score desc, id asc) in float64,
    ids id_offset + column (id_offset >= 0, so id order is column order)."""
    nq, t = S.shape
    keff = min(k, t)
    ids = np.full((nq, k), -1, np.int64)
    sc = np.full((nq, k), -np.inf, np.float64)
    col = np.arange(t)
    for i in range(nq):
        o = np.lexsort((col, -S[i].astype(np.float64)))[:keff]
        ids[i, :keff] = o + id_offset
        sc[i, :keff] = S[i, o]
    return ids, sc


@pytest.mark.parametrize("t,k,off", [(1000, 10, 0), (777, 256, 5000), (40, 100, 7),
                                     (5000, 1, 123)])
def test_topk_merge_integer_scores_lexsort(oracle, t, k, off):
    # inner products of small integers: exact in float32, many ties
    b, q = int_rows(t, 8, 11, hi=4), int_rows(12, 8, 12, hi=4)
    S = (q.astype(np.float64) @ b.T.astype(np.float64)).astype(np.float32)
    ids, sc = oracle.topk_merge(S, None, None, off, True, k)
    want_i, want_s = _lexsort_best(S, k, off)
    assert np.array_equal(ids, want_i) and np.array_equal(sc, want_s.astype(np.float32))


def test_topk_merge_tiles_equal_one_merge(oracle):
    # the reference's brute_force_knn merges tile after tile (src/knn.cpp:104-121):
    # chained merges with the running lists equal one merge over the whole row
    S = np.random.default_rng(3).integers(-50, 50, (20, 3000)).astype(np.float32)
    k = 37
    one_i, one_s = oracle.topk_merge(S, None, None, 0, True, k)
    ids = best = None
    for t0 in range(0, 3000, 700):
        ids, best = oracle.topk_merge(S[:, t0:t0 + 700], ids, best, t0, t0 == 0, k)
    assert np.array_equal(ids, one_i) and np.array_equal(best, one_s)


def test_topk_merge_matches_the_pinned_knn(oracle):
    # L2 scores 2 q.b - |b|^2 (src/knn.cpp:111-116) of integer rows merged once
    # give the ids of the brute-force restatement pinned above
    b, q = int_rows(2000, 16, 21), int_rows(30, 16, 22)
    bb = (b.astype(np.float64) ** 2).sum(1)
    S = (2.0 * (q.astype(np.float64) @ b.T.astype(np.float64)) - bb).astype(np.float32)
    ids, _ = oracle.topk_merge(S, None, None, 0, True, 16)
    kid, _ = oracle.knn(b, q, 16, "l2")
    assert np.array_equal(ids, kid)


def test_topk_merge_known_answers(oracle):
    # all scores equal: the lowest ids
    ids, sc = oracle.topk_merge(np.full((1, 50), 2.5, np.float32), None, None, 100, True, 4)
    assert ids.tolist() == [[100, 101, 102, 103]] and (sc == 2.5).all()
    # ascending scores: the last columns, best first
    ids, sc = oracle.topk_merge(np.arange(10, dtype=np.float32)[None], None, None, 0, True, 3)
    assert ids.tolist() == [[9, 8, 7]] and sc.tolist() == [[9, 8, 7]]
    # fewer candidates than k: -1 / -inf padding (src/kernels.h:224-228)
    ids, sc = oracle.topk_merge(np.array([[1, 3, 2]], np.float32), None, None, 0, True, 5)
    assert ids.tolist() == [[1, 2, 0, -1, -1]]
    assert sc[0, :3].tolist() == [3, 2, 1] and (sc[0, 3:] == -np.inf).all()
    # +0 outranks -0 when selecting (key order), but they are equal when
    # sorting (float compare), so the lower id comes first
    S = np.array([[-0.0, 0.0]], np.float32)
    ids, sc = oracle.topk_merge(S, None, None, 0, True, 1)
    assert ids.tolist() == [[1]] and not np.signbit(sc[0, 0])
    ids, sc = oracle.topk_merge(S, None, None, 0, True, 2)
    assert ids.tolist() == [[0, 1]] and np.signbit(sc[0, 0]) and not np.signbit(sc[0, 1])
    # ids compare unsigned: -2 and -1 (id_offset -2) lose to 0 and 1
    ids, _ = oracle.topk_merge(np.zeros((1, 4), np.float32), None, None, -2, True, 2)
    assert ids.tolist() == [[0, 1]]
    # running lists take part unless first; the initial -1 / -inf entries are
    # candidates too
    prev_i = np.array([[-1, -1, -1, -1]], np.int32)
    prev_s = np.full((1, 4), -np.inf, np.float32)
    ids, sc = oracle.topk_merge(np.array([[5, 4]], np.float32), prev_i, prev_s, 10, False, 4)
    assert ids.tolist() == [[10, 11, -1, -1]] and sc[0, 2:].tolist() == [-np.inf, -np.inf]
    ids, _ = oracle.topk_merge(np.array([[5, 4]], np.float32), np.array([[3, 7]], np.int32),
                               np.array([[4.5, 9]], np.float32), 10, False, 2)
    assert ids.tolist() == [[7, 10]]
    ids, _ = oracle.topk_merge(np.array([[5, 4]], np.float32), np.array([[3, 7]], np.int32),
                               np.array([[4.5, 9]], np.float32), 10, True, 2)
    assert ids.tolist() == [[10, 11]]


# ---- prefiltered search (python/mlxvs/cuvs/neighbors/brute_force.py:97-136) -------

def _masked_best(s, allowed, k):
    """ids of the k best allowed rows per query by (score desc, id asc)."""
    nq, n = s.shape
    out = np.full((nq, k), -1, np.int64)
    for i in range(nq):
        idx = np.flatnonzero(allowed[i])
        order = idx[np.lexsort((idx, -s[i, idx]))][:k]
        out[i, :len(order)] = order
    return out


def _filter(kind, nq, n, p, seed):
    rng = np.random.default_rng(seed)
    if kind == "bitmap":
        allowed = rng.random((nq, n)) < p
        return allowed, {"bitmap": allowed}
    keep = rng.random(n) < p
    return np.broadcast_to(keep, (nq, n)), {"bitset": keep}


@pytest.mark.parametrize("kind", ["bitset", "bitmap"])
@pytest.mark.parametrize("metric", ["l2", "inner_product"])
@pytest.mark.parametrize("n,nq,d,k,p", [(300, 20, 16, 7, 0.3), (1000, 9, 8, 64, 0.05),
                                        (77, 5, 3, 10, 0.5)])
def test_filtered_integer_exact(oracle, kind, metric, n, nq, d, k, p):
    # n = 77: a bitmap row starts mid-word (the bits are row-major over
    # nq * n, not padded per query), so a per-query padded reading fails
    b, q = int_rows(n, d, 11), int_rows(nq, d, 12)
    allowed, kw = _filter(kind, nq, n, p, 13)
    ids, dist = oracle.knn_filtered(b, q, k, metric, **kw)
    s = oracle.exact_scores(q, b, metric)
    want = _masked_best(s, allowed, k)
    assert np.array_equal(ids, want)
    got = np.take_along_axis(s, np.maximum(want, 0), 1)
    exp = (-got if metric == "l2" else got).astype(np.float32)
    pad = np.inf if metric == "l2" else -np.inf
    assert np.array_equal(dist, np.where(want >= 0, exp, pad).astype(np.float32))


@pytest.mark.parametrize("kind", ["bitset", "bitmap"])
def test_filtered_reference_case(oracle, kind):
    # python/tests/test_cuvs.py:196-211: the allowed rows' k nearest by
    # scipy's sqeuclidean, as sets
    from scipy.spatial.distance import cdist
    rng = np.random.default_rng(4)
    index = rng.random((300, 16)).astype(np.float32)
    queries = rng.random((20, 16)).astype(np.float32)
    if kind == "bitset":
        keep = rng.random(300) < 0.3
        allowed, kw = np.broadcast_to(keep, (20, 300)), {"bitset": keep}
    else:
        allowed = rng.random((20, 300)) < 0.3
        kw = {"bitmap": allowed}
    ids, _ = oracle.knn_filtered(index, queries, 7, "l2", **kw)
    pw = np.where(allowed, cdist(queries, index, "sqeuclidean"), np.inf)
    assert np.array_equal(np.sort(ids, 1), np.sort(np.argsort(pw, 1)[:, :7], 1))


def test_filtered_limits(oracle):
    b, q = int_rows(200, 8, 21), int_rows(6, 8, 22)
    # every row allowed: the unfiltered search
    full = oracle.knn_filtered(b, q, 12, "l2", bitset=np.ones(200, bool))
    plain = oracle.knn(b, q, 12, "l2")
    assert np.array_equal(full[0], plain[0]) and np.array_equal(full[1], plain[1])
    # no row allowed: every slot missing, +inf for L2, -inf for similarities
    ids, dist = oracle.knn_filtered(b, q, 5, "l2", bitmap=np.zeros((6, 200), bool))
    assert (ids == -1).all() and (dist == np.inf).all()
    ids, dist = oracle.knn_filtered(b, q, 5, "cosine", bitset=np.zeros(200, bool))
    assert (ids == -1).all() and (dist == -np.inf).all()
    # two allowed rows and k = 4: those two, then padding
    keep = np.zeros(200, bool)
    keep[[17, 190]] = True
    ids, dist = oracle.knn_filtered(b, q, 4, "l2", bitset=keep)
    assert (np.sort(ids[:, :2], 1) == [17, 190]).all() and (ids[:, 2:] == -1).all()
    assert np.isfinite(dist[:, :2]).all() and (dist[:, 2:] == np.inf).all()
    # the packing: bit i % 32 of word i / 32 (filters.py:39-43)
    w = oracle.filter_words(np.arange(40) % 3 == 0)
    assert w.dtype == np.uint32 and len(w) == 2
    assert w[0] == sum(1 << i for i in range(0, 32, 3))
    assert w[1] == sum(1 << (i - 32) for i in range(33, 40, 3))


# ---- cuVS's other distances (oracle.pairwise_distances / pairwise_knn) ----------------

@pytest.mark.parametrize("metric,kw", [("cityblock", {}), ("chebyshev", {}), ("canberra", {}),
                                       ("minkowski", {"p": 3.0}), ("minkowski", {"p": 1.5}),
                                       ("correlation", {}), ("braycurtis", {}),
                                       ("hamming", {})])
def test_pairwise_matches_scipy(oracle, metric, kw):
    from scipy.spatial.distance import cdist

    rng = np.random.default_rng(31)
    # small integers: equal columns (hamming) and zero pairs (canberra's 0 / 0)
    q = rng.integers(0, 4, (9, 13)).astype(np.float32)
    b = rng.integers(0, 4, (40, 13)).astype(np.float32)
    q[0] = b[5]
    if metric == "correlation":
        q += rng.random(q.shape).astype(np.float32)  # no constant rows
        b += rng.random(b.shape).astype(np.float32)
    got = oracle.pairwise_distances(q, b, metric, kw.get("p", 2.0))
    want = cdist(q.astype(np.float64), b.astype(np.float64), metric, **kw)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_pairwise_russellrao_jensenshannon_kl_hellinger(oracle):
    from scipy.spatial.distance import cdist
    from scipy.special import rel_entr

    rng = np.random.default_rng(32)
    # Russell-Rao on {0, 1} rows: scipy's boolean definition (n - c_TT) / n
    qb = (rng.random((6, 20)) < 0.5).astype(np.float32)
    bb = (rng.random((30, 20)) < 0.5).astype(np.float32)
    np.testing.assert_allclose(oracle.pairwise_distances(qb, bb, "russellrao"),
                               cdist(qb.astype(bool), bb.astype(bool), "russellrao"), rtol=1e-12)
    # distributions with zeros: Jensen-Shannon as scipy's (natural log)
    q = rng.random((5, 16))
    b = rng.random((25, 16))
    q[:, :3] = 0
    b[::2, 5:7] = 0
    q /= q.sum(1, keepdims=True)
    b /= b.sum(1, keepdims=True)
    np.testing.assert_allclose(oracle.pairwise_distances(q, b, "jensenshannon"),
                               cdist(q, b, "jensenshannon"), rtol=1e-10, atol=1e-12)
    # KL: half the relative entropy where b > 0; where b = 0 the reference
    # takes log b as 0 (a log a, not the infinite entropy)
    bp = b + 1e-3
    np.testing.assert_allclose(oracle.pairwise_distances(q, bp, "kl_divergence"),
                               0.5 * rel_entr(q[:, None, :], bp[None]).sum(2), rtol=1e-10)
    one = oracle.pairwise_distances(np.array([[0.5, 0.5]]), np.array([[1.0, 0.0]]),
                                    "kl_divergence")
    assert np.isclose(one[0, 0], 0.5 * (0.5 * np.log(0.5) + 0.5 * np.log(0.5)))
    # Hellinger of distributions: 1 - sum sqrt(a b) = sum (sqrt a - sqrt b)^2 / 2
    want = np.sqrt(0.5 * ((np.sqrt(q)[:, None, :] - np.sqrt(b)[None]) ** 2).sum(2))
    np.testing.assert_allclose(oracle.pairwise_distances(q, b, "hellinger"), want, atol=1e-7)
    assert np.allclose(np.diag(oracle.pairwise_distances(b[:5], b[:5], "hellinger")), 0,
                       atol=1e-7)


def test_pairwise_knn_selection(oracle):
    # integer rows with many equal L1 distances: smallest first, lowest id
    # among equal ones; prefilter masks; padding past the allowed rows
    rng = np.random.default_rng(33)
    b = rng.integers(0, 2, (60, 4)).astype(np.float32)
    q = rng.integers(0, 2, (7, 4)).astype(np.float32)
    ids, dist = oracle.pairwise_knn(q, b, 12, "cityblock")
    full = np.abs(q[:, None, :] - b[None]).sum(2)
    for i in range(7):
        order = sorted(range(60), key=lambda j: (full[i, j], j))[:12]
        assert ids[i].tolist() == order and dist[i].tolist() == full[i, order].tolist()
    keep = np.zeros(60, bool)
    keep[[3, 41, 59]] = True
    ids, dist = oracle.pairwise_knn(q, b, 5, "chebyshev", allowed=keep)
    assert (np.sort(ids[:, :3], 1) == [3, 41, 59]).all() and (ids[:, 3:] == -1).all()
    assert np.isinf(dist[:, 3:]).all()
    with pytest.raises(ValueError):
        oracle.pairwise_distances(q, b, 11)
