"""A seeded sweep over shapes, list lengths and metrics: the HIP engine
against the CPU restatement, bit for bit.

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
