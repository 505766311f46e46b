"""The C ABI surface of libmlxvs_c.so, checked without a GPU.

  * every function include/mlxvs/mlxvs_c.h declares is exported, and nothing
    but mlxvs_* C symbols and the C++ API of include/mlxvs/mlxvs.hpp is;
  * a C program (tests/c/abi_check.c) compiled against the header as C and
    linked against the library gets the reference's status codes and error
    messages for invalid arguments (reference tests/test_c_api.c:247-258);
  * the Python API raises ValueError for invalid input (reference
    python/tests/test_mlxvs.py:72-78, 240-245) and, without a GPU,
    RuntimeError for valid input -- there is no CPU fallback.
"""

import ctypes
import os
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mlxvs" / "mlxvs_c.h"


def declared_functions():
    text = HEADER.read_text()
    return re.findall(r"MLXVS_C_API\s+[\w\s\*]+?\b(mlxvs_\w+)\s*\(", text)


def lib_path():
    import mlxvs_amd

    return mlxvs_amd.library_path()


def test_header_declares_the_reference_entry_points():
    names = declared_functions()
    for n in ("mlxvs_brute_force_knn", "mlxvs_last_error", "mlxvs_version"):
        assert n in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(lib_path())
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_only_mlxvs_symbols_exported():
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path()], capture_output=True,
                         text=True, check=True).stdout
    for line in out.splitlines():
        parts = line.split()
        if len(parts) < 3 or parts[1] not in ("T", "W"):
            continue
        sym = parts[2]
        assert sym.startswith("mlxvs_") or sym.startswith("_ZN5mlxvs"), sym


def test_c_program_against_the_header(tmp_path):
    exe = tmp_path / "abi_check"
    libdir = str(Path(lib_path()).parent)
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "c" / "abi_check.c"), "-o", str(exe),
                    f"-L{libdir}", "-lmlxvs_c", f"-Wl,-rpath,{libdir}"], check=True)
    env = dict(os.environ)
    import mlxvs_amd._hip as hip

    env["MLXVS_EXPECT_GPU"] = "1" if hip.device_count() > 0 else "0"
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all tests passed" in r.stdout


def test_ivf_range_planning(tmp_path):
    # the IVF-Flat scan's row parts keep every workgroup inside one 32-bit
    # buffer range (host arithmetic, mlxvs_amd/csrc/plan.h)
    exe = tmp_path / "plan_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror",
                    f"-I{ROOT / 'mlxvs_amd' / 'csrc'}", str(ROOT / "tests" / "c" / "plan_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and "all tests passed" in r.stdout, r.stdout + r.stderr


def test_python_argument_errors(engine):
    with pytest.raises(ValueError, match="same number of columns"):
        engine.brute_force_knn(np.zeros((4, 3)), np.zeros((2, 5)), 1)
    with pytest.raises(ValueError, match=r"k must be in \[1, 256\]"):
        engine.brute_force_knn(np.zeros((4, 3)), np.zeros((2, 3)), 300)
    with pytest.raises(ValueError, match="real numbers"):
        engine.brute_force_knn(np.zeros((4, 3), bool), np.zeros((2, 3)), 1)
    with pytest.raises(ValueError, match="2-D"):
        engine.brute_force_knn(np.zeros(4), np.zeros((2, 3)), 1)
    with pytest.raises(ValueError, match="unknown Metric 'cosin'"):
        engine.brute_force_knn(np.zeros((4, 3)), np.zeros((2, 3)), 1, "cosin")
    with pytest.raises(ValueError, match="bit-packed uint8"):
        engine.hamming_knn(np.zeros((4, 3), np.int8), np.zeros((2, 3), np.uint8), 1)
    with pytest.raises(ValueError, match="k must be in"):
        engine.hamming_knn(np.zeros((4, 3), np.uint8), np.zeros((2, 3), np.uint8), 0)
    with pytest.raises(ValueError, match="1 <= k <= 255"):
        engine.all_neighbors(np.zeros((4, 3), np.float32), 300)
    # a stream must be a hipStream_t handle (checked before any GPU work)
    with pytest.raises(ValueError, match="hipStream_t handle"):
        engine.brute_force_knn(np.zeros((4, 3)), np.zeros((2, 3)), 1, stream="s")
    with pytest.raises(ValueError, match="hipStream_t handle"):
        engine.hamming_knn(np.zeros((4, 3), np.uint8), np.zeros((2, 3), np.uint8), 1, stream=-7)
    with pytest.raises(ValueError, match="hipStream_t handle"):
        engine.kmeans_predict(np.zeros((4, 3)), np.zeros((2, 3)), 1, stream=1.5)
    with pytest.raises(ValueError, match="hipStream_t handle"):
        engine.topk_merge(np.zeros((2, 3), np.float32), None, None, 0, True, 1, stream=[1])
    # topk_merge: the reference's checks and messages (src/knn.cpp:46-54)
    with pytest.raises(ValueError, match=r"scores must be float32 \[nq, t\]"):
        engine.topk_merge(np.zeros((2, 3), np.float64), None, None, 0, True, 1)
    with pytest.raises(ValueError, match=r"scores must be float32 \[nq, t\]"):
        engine.topk_merge(np.zeros(3, np.float32), None, None, 0, True, 1)
    with pytest.raises(ValueError, match=r"k must be in \[1, 256\]"):
        engine.topk_merge(np.zeros((2, 3), np.float32), None, None, 0, True, 0)
    with pytest.raises(ValueError, match=r"k must be in \[1, 256\]"):
        engine.topk_merge(np.zeros((2, 3), np.float32), None, None, 0, True, 257)
    with pytest.raises(ValueError, match=r"\[nq, k\]"):
        engine.topk_merge(np.zeros((2, 3), np.float32), np.zeros((2, 2), np.int32),
                          np.zeros((2, 2), np.float32), 0, False, 3)


def test_no_cpu_fallback_without_gpu(engine):
    import mlxvs_amd._hip as hip

    if hip.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="no HIP device"):
        engine.brute_force_knn(np.zeros((4, 3)), np.zeros((2, 3)), 1)
    with pytest.raises(RuntimeError, match="no HIP device"):
        engine.hamming_knn(np.zeros((4, 3), np.uint8), np.zeros((2, 3), np.uint8), 1)


def test_metric_enum_values(engine):
    assert int(engine.Metric.inner_product) == 0
    assert int(engine.Metric.l2) == 1
    assert int(engine.Metric.cosine) == 2
    assert engine.version() == "0.16.1"
