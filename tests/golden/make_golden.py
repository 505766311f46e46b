"""Writes the golden fixtures of tests/golden/ from independent float64 NumPy.

    python tests/golden/make_golden.py

Every expected answer here comes from float64 brute force with an explicit
(score descending, id ascending) np.lexsort -- the reference's selection rule
(src/kernels.h:104-147) -- or, for Hamming, from an 8-bit popcount table.
Nothing here calls the CPU restatement (oracle/) or the engine, so the
fixtures pin both.  Inputs are regenerated from mlxvs_amd.synth; each
fixture stores a digest of its inputs so that generator drift is caught.

Fixtures (all .npz, loadable with allow_pickle=False):
  c1_full.npz       configuration c1 in full: 100 queries x 10,000 rows, L2, k=10
  c2_subset.npz     configuration c2, first 64 queries x all 1,000,000 rows, L2, k=10
  c3_subset.npz     configuration c3 on its first 100,000 rows, first 256 queries,
                    inner product and cosine, k=10 (float64 ids and scores)
  c4_subset.npz     configuration c4, first 32 queries x all 1,000,000 codes, k=100
  c5_subset.npz     configuration c5 self graph, first 32 rows x all 200,000 rows,
                    L2, k=64 (self excluded; float64 ids and distances)
  kat_ties.npz      tests/test_knn.cpp:156-192 ties case (input and answer)
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from mlxvs_amd import synth  # noqa: E402


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def topk_rows(scores: np.ndarray, k: int):
    """(ids, scores) of the k best of each row by (score desc, id asc)."""
    n = scores.shape[1]
    col = np.arange(n)
    ids = np.empty((scores.shape[0], k), np.int64)
    for i in range(scores.shape[0]):
        # partition first, then an exact lexsort of a safe candidate set
        if n > 4 * k:
            thr = np.partition(-scores[i], k - 1)[k - 1]
            cand = np.nonzero(-scores[i] <= thr)[0]
        else:
            cand = col
        order = cand[np.lexsort((cand, -scores[i][cand]))][:k]
        ids[i] = order
    return ids, np.take_along_axis(scores, ids, 1)


def chunked_topk(qs: np.ndarray, gen, n: int, k: int, score_fn, chunk=125_000):
    """Best k over base rows generated in chunks: float64 scores per chunk,
    running merge by (score desc, id asc)."""
    best_s = np.full((qs.shape[0], 0), -np.inf)
    best_i = np.zeros((qs.shape[0], 0), np.int64)
    h = hashlib.sha256()
    for lo in range(0, n, chunk):
        hi = min(n, lo + chunk)
        b = gen(lo, hi)
        h.update(np.ascontiguousarray(b).tobytes())
        s = score_fn(qs, b)
        ids, sc = topk_rows(s, min(k, hi - lo))
        best_s = np.concatenate([best_s, sc], 1)
        best_i = np.concatenate([best_i, ids + lo], 1)
        rows_s, rows_i = [], []
        for r in range(qs.shape[0]):
            o = np.lexsort((best_i[r], -best_s[r]))[:k]
            rows_s.append(best_s[r][o])
            rows_i.append(best_i[r][o])
        best_s, best_i = np.array(rows_s), np.array(rows_i)
    return best_i, best_s, h.hexdigest()


def l2_scores(q, b):
    q = q.astype(np.float64)
    b = b.astype(np.float64)
    return -((q * q).sum(1)[:, None] + (b * b).sum(1)[None, :] - 2.0 * q @ b.T)


def ip_scores(q, b):
    return q.astype(np.float64) @ b.astype(np.float64).T


def cos_scores(q, b):
    q = q.astype(np.float64)
    b = b.astype(np.float64)
    q = q / np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-300)
    b = b / np.maximum(np.linalg.norm(b, axis=1, keepdims=True), 1e-300)
    return q @ b.T


def make_c1():
    base = synth.c1_rows(1, 0, 10_000)
    q = synth.c1_rows(2, 0, 100)
    ids, sc = topk_rows(l2_scores(q, base), 10)
    np.savez_compressed(HERE / "c1_full.npz", ids=ids.astype(np.int32), dist=-sc,
                        base_digest=digest(base), query_digest=digest(q))


def make_c2():
    cen = synth.c2_centres()
    q = synth.c2_rows(2, 0, 64, centres=cen)
    ids, sc, dg = chunked_topk(q, lambda lo, hi: synth.c2_rows(1, lo, hi, centres=cen),
                               1_000_000, 10, l2_scores)
    np.savez_compressed(HERE / "c2_subset.npz", ids=ids.astype(np.int32), dist=-sc,
                        base_digest=dg, query_digest=digest(q))


def make_c3():
    cen = synth.c3_centres()
    q = synth.c3_rows(2, 0, 256, centres=cen)
    gen = lambda lo, hi: synth.c3_rows(1, lo, hi, centres=cen)  # noqa: E731
    ids_ip, sc_ip, dg = chunked_topk(q, gen, 100_000, 10, ip_scores, chunk=25_000)
    ids_cos, sc_cos, _ = chunked_topk(q, gen, 100_000, 10, cos_scores, chunk=25_000)
    np.savez_compressed(HERE / "c3_subset.npz", ids_ip=ids_ip.astype(np.int32), score_ip=sc_ip,
                        ids_cos=ids_cos.astype(np.int32), score_cos=sc_cos,
                        base_digest=dg, query_digest=digest(q))


def popcount_distances(q, rows):
    lut = np.array([bin(i).count("1") for i in range(256)], dtype=np.int64)
    return np.stack([lut[qi[None, :] ^ rows].sum(1) for qi in q])


def make_c4():
    gen = lambda lo, hi: synth.c4_codes(1, lo, hi)  # noqa: E731
    q, src = synth.c4_queries(gen, 1_000_000, 2, 0, 32)
    score = lambda qq, b: -popcount_distances(qq, b).astype(np.float64)  # noqa: E731
    ids, sc, dg = chunked_topk(q, gen, 1_000_000, 100, score, chunk=100_000)
    np.savez_compressed(HERE / "c4_subset.npz", ids=ids.astype(np.int32), dist=-sc,
                        src=src, base_digest=dg, query_digest=digest(q))


def make_c5():
    cen = synth.c5_centres()
    x = synth.chunked(lambda lo, hi: synth.c5_rows(1, lo, hi, centres=cen), 200_000)
    q = x[:32]
    s = l2_scores(q, x)
    s[np.arange(32), np.arange(32)] = -np.inf  # self excluded
    ids, sc = topk_rows(s, 64)
    np.savez_compressed(HERE / "c5_subset.npz", ids=ids.astype(np.int32), dist=-sc,
                        base_digest=digest(x))


def make_ties():
    # tests/test_knn.cpp:156-192: 4000 x 8 ones, rows = 0 (mod 97) have x0 = 5;
    # queries are rows 1 and 2; k = 10 -> ids 1..10 (lowest ids among the
    # many rows at distance 0)
    x = np.ones((4000, 8), np.float32)
    x[::97, 0] = 5.0
    q = x[1:3]
    s = l2_scores(q, x)
    ids, sc = topk_rows(s, 10)
    want = []
    for _ in range(2):
        row, v = [], 1
        while len(row) < 10:
            if v % 97 != 0:
                row.append(v)
            v += 1
        want.append(row)
    assert (ids == np.array(want)).all()
    np.savez_compressed(HERE / "kat_ties.npz", base=x, queries=q,
                        ids=ids.astype(np.int32), dist=-sc)


if __name__ == "__main__":
    which = sys.argv[1:] or ["ties", "c1", "c4", "c5", "c2", "c3"]
    for w in which:
        print("making", w, flush=True)
        globals()["make_" + w]()
