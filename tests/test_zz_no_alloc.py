"""The no-allocation entry point (mlxvs_brute_force_knn_device_noalloc),
called through the C ABI, against mlxvs_brute_force_knn_device on the same
device inputs: the same kernels, so ids and distances must be bit-identical.
Calls in a row, later ones smaller (the shared scratch keeps the earlier
calls' contents), one with k = 64 (lists shorter than k, the merge's flags
and the redo of flagged queries all in the scratch), then the rejection of a
workspace beyond the fixed scratch, with device buffers of the real size.
"""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

INVALID = 1


def run(engine, fn, db, n, dq, nq, d, k, metric, f16=False):
    from mlxvs_amd import _hip

    di = _hip.DeviceBuffer(nq * k * 4)
    dd = _hip.DeviceBuffer(nq * k * 4)
    rc = fn(db.value, n, dq.value, nq, d, int(f16), k, int(metric), di.value, dd.value, None)
    return rc, di, dd


@pytest.mark.parametrize("f16", [False, True])
def test_no_alloc_matches_the_allocating_entry(engine, f16):
    from mlxvs_amd import _hip, synth

    lib = engine._L()
    # (at 300 and 500 queries, over 1,024 candidates a query, the allocating
    # entry merges by the bounded batch merge and the no-allocation entry by
    # the merge levels, so the comparison covers both; at k = 64 the redo
    # flags as well)
    cases = [(200_000, 2_000, 128, 10, engine.Metric.l2),
             (30_000, 300, 64, 8, engine.Metric.inner_product),
             (50_000, 500, 128, 64, engine.Metric.l2)]
    for n, nq, d, k, metric in cases:
        print(f"[no_alloc] f16={f16} n={n} nq={nq} d={d} k={k} metric={int(metric)}", flush=True)
        cen = synth.c2_centres()
        base = synth.c2_rows(1, 0, n, centres=cen)[:, :d]
        q = synth.c2_rows(2, 0, nq, centres=cen)[:, :d]
        if f16:
            base, q = base.astype(np.float16), q.astype(np.float16)
        db = _hip.DeviceBuffer.from_array(np.ascontiguousarray(base))
        dq = _hip.DeviceBuffer.from_array(np.ascontiguousarray(q))
        rc, wi, wd = run(engine, lib.mlxvs_brute_force_knn_device, db, n, dq, nq, d, k, metric,
                         f16)
        assert rc == 0, lib.mlxvs_last_error()
        rc, gi, gd = run(engine, lib.mlxvs_brute_force_knn_device_noalloc, db, n, dq, nq, d, k,
                         metric, f16)
        assert rc == 0, lib.mlxvs_last_error()
        _hip.synchronize()
        want_i, want_d = wi.download((nq, k), np.int32), wd.download((nq, k), np.float32)
        got_i, got_d = gi.download((nq, k), np.int32), gd.download((nq, k), np.float32)
        assert np.array_equal(got_i, want_i)
        assert np.array_equal(got_d.view(np.uint32), want_d.view(np.uint32))


def test_no_alloc_rejects_what_it_cannot_hold(engine):
    from mlxvs_amd import _hip

    lib = engine._L()
    fn = lib.mlxvs_brute_force_knn_device_noalloc
    n, d = 1_000_000, 4
    db = _hip.DeviceBuffer.from_array(np.zeros((n, d), np.float32))
    # 100,000 queries' lists need more than the 64 MiB of scratch
    nq = 100_000
    dq = _hip.DeviceBuffer.from_array(np.zeros((nq, d), np.float32))
    rc, _, _ = run(engine, fn, db, n, dq, nq, d, 10, engine.Metric.l2)
    assert rc == INVALID and b"MiB of scratch" in lib.mlxvs_last_error()
    _hip.synchronize()
