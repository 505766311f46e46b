#!/usr/bin/env python3
"""Benchmark of the exact k-NN hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 10] [--warmup 2] [--workload c2]

Default workload (BASELINE.json metric): configuration c2, exact L2 k-NN,
k = 10, 1,000,000 x 128 float32 base rows (1,024-component mixture, integer
values in [0, 255]) and 10,000 queries.  Inputs are generated with
mlxvs_amd.synth, copied to HBM before timing, and one step is one
mlxvs_brute_force_knn_device call over all 10,000 queries (norms, fused
MFMA distance + top-k, merge).  W warm-up steps, then exactly K timed steps
between two device synchronisations; value = queries answered per second.
The same K steps then run again with the engine's HIP events around every
launch (ms_per_step_profiled): the kernel times below come from them.

The same JSON line carries:
  roofline      the dominant kernel's achieved MFMA rate, from HIP events
                recorded around each of its launches in the second K steps
                (2 nq n d flops per launch over its mean duration; for Hamming
                2 nq n bits ops on the FP4 MFMA), against MI355X's dense peak
                of that type (FP32 157.3, FP16 2516.6, FP4 10066.4 TFLOP/s),
                or, below the ridge point (small batches), the rows' bytes per
                launch against HBM's 8 TB/s;
                traffic = HBM bytes per launch from the committed rocprofv3
                counter summary when present;
  cpu_baseline  the CPU restatement of the reference path (oracle/, a port:
                the reference itself runs only on Apple GPUs) timed on this
                host's cores over a bounded query sample;
  check         the last step's answers against the CPU restatement for the
                queries it answered (bit-exact on integer-valued data; float
                data: distances within the tests' tolerance and the share of
                equal ids) and, where a fixture exists, the first queries
                against the float64 golden fixture.

Other workloads (c1, c2h, c3, c3cos, c3h, c4, c5, ivf, topk) are for measurement runs; the
driver's line is the default.  --workload copy times a 1 GiB device copy, the
reference reading for scaling HBM byte counters.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = ("queries/s, exact kNN k=10 on 1M×128 fp32 (10k queries); "
          "% of MFMA/HBM roofline")
PEAK_FP32_MFMA = 157.3   # TFLOP/s, MI355X dense FP32 matrix
PEAK_FP16_MFMA = 2516.6  # TFLOP/s, MI355X dense FP16 matrix
PEAK_FP4_MFMA = 10066.4  # TFLOP/s, MI355X dense FP4 (e2m1) matrix
PEAK_HBM = 8000.0        # GB/s
VALU_LANE_OPS = 256 * 64 * 2.4e9  # non-packed VALU lane-ops per second


def workload(name: str):
    from mlxvs_amd import synth

    if name == "c1":
        base = synth.c1_rows(1, 0, 10_000)
        q = synth.c1_rows(2, 0, 100)
        return dict(kind="float", base=base, q=q, k=10, metric="l2",
                    desc="c1: exact L2 kNN k=10, 10k x 128 fp32 (int-valued), 100 queries")
    if name in ("c2", "c2h"):
        cen = synth.c2_centres()
        base = synth.chunked(lambda lo, hi: synth.c2_rows(1, lo, hi, centres=cen), 1_000_000)
        q = synth.chunked(lambda lo, hi: synth.c2_rows(2, lo, hi, centres=cen), 10_000)
        if name == "c2h":
            # the same integers in [0, 255] stored as binary16 (exact), on the
            # fp16 MFMA path: answers identical to c2's
            return dict(kind="float", base=base.astype(np.float16), q=q.astype(np.float16),
                        k=10, metric="l2",
                        desc="c2h: c2 (1M x 128, int-valued, 10k queries) stored as fp16, "
                             "L2 k=10")
        return dict(kind="float", base=base, q=q, k=10, metric="l2",
                    desc="c2: exact L2 kNN k=10, 1M x 128 fp32 base (1024-component "
                         "mixture, int-valued in [0,255]), 10k queries")
    if name in ("c3", "c3cos", "c3h"):
        cen = synth.c3_centres()
        base = synth.chunked(lambda lo, hi: synth.c3_rows(1, lo, hi, centres=cen),
                             1_000_000, chunk=4096)
        q = synth.chunked(lambda lo, hi: synth.c3_rows(2, lo, hi, centres=cen), 10_000,
                          chunk=4096)
        if name == "c3h":
            return dict(kind="float", base=base.astype(np.float16), q=q.astype(np.float16),
                        k=10, metric="inner_product",
                        desc="c3h: c3's rows stored as fp16 (1M x 1536), inner product k=10, "
                             "10k queries")
        metric = "cosine" if name == "c3cos" else "inner_product"
        return dict(kind="float", base=base, q=q, k=10, metric=metric,
                    desc=f"c3: exact {metric} kNN k=10, 1M x 1536 unit rows, 10k queries")
    if name == "c4":
        gen = lambda lo, hi: synth.c4_codes(1, lo, hi)  # noqa: E731
        base = synth.chunked(gen, 1_000_000)
        q, _ = synth.c4_queries(gen, 1_000_000, 2, 0, 10_000)
        return dict(kind="hamming", base=base, q=q, k=100, metric="hamming",
                    desc="c4: exact Hamming kNN k=100, 1M x 1024-bit codes, 10k queries")
    if name == "ivf":
        from mlxvs_amd import ivf_flat_build

        cen = synth.c2_centres()
        base = synth.chunked(lambda lo, hi: synth.c2_rows(1, lo, hi, centres=cen), 1_000_000)
        q = synth.chunked(lambda lo, hi: synth.c2_rows(2, lo, hi, centres=cen), 10_000)
        index = ivf_flat_build(base, "l2", n_lists=1024, kmeans_n_iters=10, seed=42)
        return dict(kind="ivf", base=base, q=q, k=10, metric="l2", index=index, n_probes=20,
                    desc="ivf: IVF-Flat L2 k=10, c2 rows (1M x 128 fp32), 1024 lists, "
                         "20 probes, 10k queries")
    if name == "topk":
        # one merge step of the reference's tile loop as bench/bench_knn.cpp:73-80
        # times it: the best k of every row of a [block, tile] score matrix,
        # block = 4,096 queries and tile = 65,536 rows (src/knn.cpp:90-94),
        # k = 10, first = true; the scores are L2 scores 2 q.b - |b|^2 of
        # c2-like integer rows (synthetic normal values of that spread)
        g = np.random.default_rng(5)
        S = g.standard_normal((4096, 65536), dtype=np.float32)
        S *= 2.0e5
        S -= 2.0e6
        return dict(kind="topk", base=S, q=S[:, :0], k=10, metric="topk",
                    desc="topk: topk_merge of a 4,096 x 65,536 fp32 score matrix (one tile "
                         "step of the reference loop), k=10, first=true")
    if name == "c5":
        cen = synth.c5_centres()
        x = synth.chunked(lambda lo, hi: synth.c5_rows(1, lo, hi, centres=cen), 200_000)
        return dict(kind="self", base=x, q=x, k=64, metric="l2",
                    desc="c5: self kNN graph, 200k x 256 fp16, L2, k=64, self excluded")
    raise SystemExit(f"unknown workload {name}")


def copy_probe(steps: int) -> int:
    """A plain device-to-device copy of 1 GiB (the runtime's copy kernel),
    timed; its FETCH_SIZE / WRITE_SIZE counter readings per byte copied are
    the scale factors for the fused kernel's counter readings."""
    from mlxvs_amd import _hip

    nbytes = 1 << 30
    src, dst = _hip.DeviceBuffer(nbytes), _hip.DeviceBuffer(nbytes)
    lib = _hip.lib()
    t0 = time.perf_counter()
    for _ in range(steps):
        _hip.check(lib.hipMemcpy(dst.ptr, src.ptr, ctypes.c_size_t(nbytes), 3), "hipMemcpy D2D")
    _hip.synchronize()
    dt = time.perf_counter() - t0
    print(json.dumps({"workload": "copy", "bytes_per_copy": nbytes, "copies": steps,
                      "GB/s": round(2 * nbytes * steps / dt / 1e9, 1)}), flush=True)
    return 0


def cpu_baseline(w, sample: int):
    """The CPU restatement on the first `sample` queries, all host cores."""
    import oracle

    threads = os.cpu_count() or 1
    base, q = w["base"], w["q"][:sample]
    t0 = time.perf_counter()
    if w["kind"] == "topk":
        threads = 1  # the restatement merges rows on one core
        out = oracle.topk_merge(base[:sample], None, None, 0, True, w["k"])
    elif w["kind"] == "hamming":
        out = oracle.hamming(base, q, w["k"], nthreads=threads)
    elif w["kind"] == "self":
        x = oracle.f16_to_f32(base)
        out = oracle.knn(x, x[:sample], w["k"] + 1, w["metric"], nthreads=threads)
    elif w["kind"] == "ivf":
        c, data, ind, off = w["index"]
        out = oracle.ivf_flat(c, data, ind, off, q, w["k"], w["n_probes"], w["metric"],
                              nthreads=threads)
    elif base.dtype == np.float16:
        out = oracle.knn(oracle.f16_to_f32(base), oracle.f16_to_f32(q), w["k"], w["metric"],
                         nthreads=threads)
    else:
        out = oracle.knn(base, q, w["k"], w["metric"], nthreads=threads)
    dt = time.perf_counter() - t0
    if w["kind"] == "topk":
        what = (f"first {sample} of {base.shape[0]} score rows of {base.shape[1]} scores, "
                f"{dt:.1f} s")
    else:
        what = (f"first {sample} of {w['q'].shape[0]} queries against all {base.shape[0]} "
                f"rows, {dt:.1f} s")
    return {"value": round(sample / dt, 2), "unit": "queries/s", "cores": threads,
            "cpu": cpu_model(), "kind": "port", "sample": what}, out


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it: model name, family / model /
    stepping, clock, AVX-512 or not, and the CPUs this process may use (a
    virtualised host may report only a generic model name)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                key, val = (t.strip() for t in line.split(":", 1))
                info.setdefault(key, val)
            if not line.strip() and info:
                break
    except OSError:
        return "unknown"
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    parts = [info.get("model name", "unknown"),
             f"family {info.get('cpu family', '?')} model {info.get('model', '?')} "
             f"stepping {info.get('stepping', '?')}"]
    if "cpu MHz" in info:
        parts.append(f"{float(info['cpu MHz']):.0f} MHz")
    parts.append("avx512f" if "avx512f" in info.get("flags", "").split() else "no avx512f")
    parts.append(f"{usable} usable CPUs")
    return ", ".join(parts)


def host_api_ms(w, reps: int = 3):
    """The reference's full call as a caller sees it: the C-ABI entry on host
    arrays, copies in and out included (median of `reps` after a warm-up;
    bench/bench_knn.cpp:20-33, 83-87 time brute_force_knn the same way)."""
    import mlxvs_amd

    if w["kind"] == "float":
        fn = lambda: mlxvs_amd.brute_force_knn(w["base"], w["q"], w["k"], w["metric"])  # noqa
    elif w["kind"] == "hamming":
        fn = lambda: mlxvs_amd.hamming_knn(w["base"], w["q"], w["k"])  # noqa: E731
    elif w["kind"] == "topk":
        fn = lambda: mlxvs_amd.topk_merge(w["base"], None, None, 0, True, w["k"])  # noqa
    else:
        return None
    fn()
    t = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        t.append((time.perf_counter() - t0) * 1e3)
    return round(sorted(t)[len(t) // 2], 3)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="c2")
    ap.add_argument("--e2e", type=int, default=1,
                    help="also time the host C-ABI call with its copies (e2e_ms; 0: skip)")
    ap.add_argument("--cpu-sample", type=int, default=None,
                    help="queries timed on the CPU restatement (0: skip)")
    ap.add_argument("--nq", type=int, default=None,
                    help="use only the first NQ queries (small-batch runs; the roofline "
                         "switches to HBM bytes when 2 nq d n flops over the rows' bytes "
                         "fall below the MFMA ridge point)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        return 2

    if args.workload == "copy":
        return copy_probe(args.steps)

    import mlxvs_amd
    from mlxvs_amd import _hip

    w = workload(args.workload)
    if args.nq is not None:
        if w["kind"] == "self":
            raise SystemExit("--nq does not apply to the self graph")
        w["q"] = np.ascontiguousarray(w["q"][:args.nq])
        w["desc"] += f" (first {args.nq} queries)"
    base, q, k = w["base"], w["q"], w["k"]
    n, nq = base.shape[0], q.shape[0]
    d = base.shape[1]
    if w["kind"] == "ivf":
        c, data, ind, off = w["index"]
        dix = [_hip.DeviceBuffer.from_array(a) for a in (c, data, ind, off)]
        db = dix[1]
    else:
        db = _hip.DeviceBuffer.from_array(base)
    if w["kind"] == "topk":
        nq, n = base.shape  # score rows, scores per row
    dq = db if w["kind"] in ("self", "topk") else _hip.DeviceBuffer.from_array(q)
    di = _hip.DeviceBuffer(nq * k * 4)
    dd = _hip.DeviceBuffer(nq * k * 4)

    def step():
        if w["kind"] == "topk":
            mlxvs_amd.topk_merge_device(db.value, nq, n, None, None, 0, True, k, di.value,
                                        dd.value)
        elif w["kind"] == "float":
            mlxvs_amd.brute_force_knn_device(db.value, n, dq.value, nq, d, k, w["metric"],
                                             di.value, dd.value,
                                             f16=base.dtype == np.float16)
        elif w["kind"] == "hamming":
            mlxvs_amd.hamming_knn_device(db.value, n, dq.value, nq, d, k, di.value, dd.value)
        elif w["kind"] == "ivf":
            mlxvs_amd.ivf_flat_search_device(dix[0].value, c.shape[0], dix[1].value, n,
                                             dix[2].value, dix[3].value, d, w["metric"],
                                             dq.value, nq, k, di.value, dd.value,
                                             n_probes=w["n_probes"])
        else:
            mlxvs_amd.knn_self_graph_device(db.value, n, d, k, w["metric"], di.value,
                                            dd.value, f16=base.dtype == np.float16)

    for _ in range(args.warmup):
        step()
    _hip.synchronize()
    # the K timed steps, as a caller runs them (no instrumentation) ...
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    _hip.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    # ... then the same K steps with the engine's HIP events around every
    # launch, on its stream: the kernel times (the events add GPU work of
    # their own: a few microseconds a launch, which matters only to the
    # one-query lines)
    mlxvs_amd.profile(True)
    _hip.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    _hip.synchronize()
    ms_per_step_profiled = (time.perf_counter() - t0) * 1e3 / args.steps
    stages = mlxvs_amd.profile_report()
    mlxvs_amd.profile(False)

    ids = di.download((nq, k), np.int32)
    dist = dd.download((nq, k), np.float32)
    check = None
    if w["kind"] == "topk":
        import oracle

        m = 64
        oi, os_ = oracle.topk_merge(base[:m], None, None, 0, True, k)
        ok = np.array_equal(ids[:m], oi) and np.array_equal(dist[:m].view(np.uint32),
                                                             os_.view(np.uint32))
        check = f"first {m} rows vs the CPU restatement: {'bit-exact' if ok else 'MISMATCH'}"
    if args.workload in ("c1", "c2", "c2h", "c4"):
        fx = {"c1": "c1_full.npz", "c2": "c2_subset.npz", "c2h": "c2_subset.npz",
              "c4": "c4_subset.npz"}[args.workload]
        g = np.load(ROOT / "tests" / "golden" / fx)
        m = min(g["ids"].shape[0], nq)
        ok = np.array_equal(ids[:m], g["ids"][:m]) and np.array_equal(
            dist[:m], g["dist"][:m].astype(np.float32))
        check = f"first {m} queries vs float64 golden: {'bit-exact' if ok else 'MISMATCH'}"

    # roofline of the dominant scan kernel (the distance stage with the most
    # time; the merge, norms, packing and fills are reported in the stages):
    # its algorithmic work per launch over its mean launch duration
    scan = {s_: v for s_, v in stages.items() if s_ not in ("merge", "prep", "pack", "fill")}
    kname = max(scan or stages, key=lambda s_: stages[s_][1])
    cnt, tot = stages[kname]
    per = tot / max(cnt, 1) / 1e3  # seconds per launch
    if w["kind"] == "topk":
        # HBM: the score matrix read once, the [rows, k] ids and scores written
        tbytes = (float(nq) * n * 4 + nq * k * 8) / (cnt / args.steps)
        roof = {"bound": "hbm", "achieved": round(tbytes / per / 1e9, 1), "peak": PEAK_HBM,
                "unit": "GB/s"}
    elif w["kind"] == "ivf" and kname == "ivf_scan":
        # 2 d flops per (query, candidate row) of the probed lists
        c, data, ind, off = w["index"]
        probes = mlxvs_amd.kmeans_predict(q, c, w["n_probes"])
        cands = float(np.diff(off)[probes].sum())
        flops = 2.0 * d * cands / (cnt / args.steps)
        roof = {"bound": "mfma", "achieved": round(flops / per / 1e12, 2),
                "peak": PEAK_FP32_MFMA, "unit": "TFLOP/s", "candidates_per_query": round(cands / nq, 1)}
    elif w["kind"] == "hamming" and kname == "scan_bits":
        # a few queries: the codes read once (the queries of a split share
        # the rows in L2)
        row_bytes = float(n) * d / (cnt / args.steps)
        roof = {"bound": "hbm", "achieved": round(row_bytes / per / 1e9, 1), "peak": PEAK_HBM,
                "unit": "GB/s"}
    elif w["kind"] == "hamming" and kname in ("hamming_mfma", "stream_bits"):
        # the FP4 MFMA route: 2 ops (multiply, add) per code bit and pair
        ops = 2.0 * nq * n * 8 * d / (cnt / args.steps)  # per launch
        row_bytes = float(n) * d / (cnt / args.steps)
        if ops / row_bytes < PEAK_FP4_MFMA * 1e12 / (PEAK_HBM * 1e9):
            roof = {"bound": "hbm", "achieved": round(row_bytes / per / 1e9, 1),
                    "peak": PEAK_HBM, "unit": "GB/s"}
        else:
            roof = {"bound": "mfma", "achieved": round(ops / per / 1e12, 2),
                    "peak": PEAK_FP4_MFMA, "unit": "TFLOP/s"}
    elif w["kind"] == "hamming":
        # the popcount route: XOR + popcount-accumulate per 32-bit word
        words = (d + 3) // 4
        work = nq * n * words * 2.0 / (cnt / args.steps)  # per launch
        roof = {"bound": "valu", "achieved": round(work / per / 1e12, 3),
                "peak": round(VALU_LANE_OPS / 1e12, 2), "unit": "Tlane-op/s"}
    else:
        f16 = base.dtype == np.float16 and w["metric"] != "cosine"
        # fused kernels cover all queries in one launch; the exhaustive path
        # splits them over several score launches
        flops = 2.0 * nq * n * d / (cnt / args.steps)
        peak = PEAK_FP16_MFMA if (f16 and kname.startswith("fused")) else PEAK_FP32_MFMA
        row_bytes = float(n) * d * base.dtype.itemsize / (cnt / args.steps)
        if flops / row_bytes < peak * 1e12 / (PEAK_HBM * 1e9):
            # below the ridge point: the base rows' bytes bound the kernel
            roof = {"bound": "hbm", "achieved": round(row_bytes / per / 1e9, 1),
                    "peak": PEAK_HBM, "unit": "GB/s"}
        else:
            roof = {"bound": "mfma", "achieved": round(flops / per / 1e12, 2), "peak": peak,
                    "unit": "TFLOP/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["kernel"] = kname
    roof["kernel_ms"] = round(per * 1e3, 4)
    traffic = None
    tfile = ROOT / "profiles" / "traffic.json"
    if tfile.exists():
        key = args.workload if args.nq is None else f"{args.workload}_nq{args.nq}"
        t = json.loads(tfile.read_text()).get(key, {})
        traffic = t.get("hbm_bytes_per_launch")
    roof["traffic"] = traffic

    sample = args.cpu_sample
    if sample is None:
        sample = {"c1": 100, "c2": 10000, "c2h": 2000, "c3": 16, "c3cos": 16, "c3h": 16,
                  "c4": 256, "c5": 512, "ivf": 10000, "topk": 4096}[args.workload]
    cpu, cpu_out = cpu_baseline(w, min(sample, nq)) if sample else (None, None)
    if cpu and w["kind"] == "topk":
        cpu["unit"] = "score rows/s"
    # the whole GPU answer for the queries the CPU restatement answered
    # (bit-exact on integer-valued data; float data: ids and distances to
    # the tolerances the tests use)
    if cpu_out is not None and not args.nq:
        oi, od = cpu_out
        m = oi.shape[0]
        if w["kind"] == "topk":
            same = np.array_equal(ids[:m], oi) and np.array_equal(dist[:m].view(np.uint32),
                                                                  od.view(np.uint32))
        elif args.workload in ("c1", "c2", "c2h", "c4"):
            same = np.array_equal(ids[:m], oi) and np.array_equal(dist[:m], od)
        else:
            same = None
        if same is not None:
            full = f"{m} of {nq} rows vs the CPU restatement: {'bit-exact' if same else 'MISMATCH'}"
            check = full if check is None else f"{full}; {check}"
        elif w["kind"] in ("float", "self", "ivf"):
            # float data: the distances within the tests' tolerance, and the
            # share of equal ids (near-equal scores may swap places)
            if w["kind"] == "self":
                # the restatement's k + 1 include the row itself: drop it
                keep = oi != np.arange(m)[:, None]
                keep[keep.sum(1) > w["k"], -1] = False
                oi = oi[keep].reshape(m, w["k"])
                od = od[keep].reshape(m, w["k"])
            tol = 2e-3 if base.dtype == np.float16 else 1e-4
            close = np.allclose(dist[:m], od, rtol=tol, atol=tol)
            share = float((ids[:m] == oi).mean())
            check = (f"{m} of {nq} rows vs the CPU restatement: distances within {tol:g} "
                     f"{'yes' if close else 'NO'}, ids equal {100 * share:.2f}%")
    e2e = host_api_ms(w) if args.e2e else None

    line = {
        "metric": METRIC if args.workload == "c2" else w["desc"],
        "value": round(nq / (ms_per_step / 1e3), 1),
        "unit": "score rows/s" if w["kind"] == "topk" else "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_profiled": round(ms_per_step_profiled, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if base.dtype == np.float16 else ("e2m1" if w["kind"] == "hamming" else "f32"),
        "data": "synthetic (mlxvs_amd.synth, seeded splitmix64)",
        "config": {"workload": w["desc"], "n": n, "nq": nq, "d": d, "k": k,
                   "metric": w["metric"], "parallelism": "single GPU"},
        "roofline": roof,
        "cpu_baseline": cpu,
        "stages_ms_per_step": {s: round(v[1] / args.steps, 4) for s, v in stages.items()},
        "e2e_ms": e2e,
        "check": check,
    }
    print(json.dumps(line), flush=True)
    return 1 if (check is not None and "MISMATCH" in check) else 0


if __name__ == "__main__":
    sys.exit(main())
