"""CPU checks of the front ends around the k-NN path: vector files, cuVS index
files, argument validation of NearestNeighbors / kmeans_predict / the cuVS
brute-force index.  No GPU call is made here.

The cuVS records are pinned against NumPy's own ``.npy`` format-1.0 reader
(numpy.lib.format), which parses every record this build writes, and against
the layout the reference's test checks (python/tests/test_cuvs.py:214-221).
"""

import io

import numpy as np
import numpy.lib.format as npf
import pytest

import mlxvs_amd
from mlxvs_amd import formats
from mlxvs_amd.cuvs import _serialize as ser
from mlxvs_amd.cuvs.neighbors import brute_force


# ---- .fvecs / .ivecs / .bvecs ------------------------------------------------------

@pytest.mark.parametrize("kind,dtype", [("fvecs", np.float32), ("ivecs", np.int32),
                                        ("bvecs", np.uint8)])
def test_vecs_round_trip_and_layout(tmp_path, kind, dtype):
    rng = np.random.default_rng(1)
    a = (rng.standard_normal((7, 5)) * 100).astype(dtype)
    path = tmp_path / f"x.{kind}"
    getattr(formats, f"write_{kind}")(path, a)
    raw = path.read_bytes()
    item = np.dtype(dtype).itemsize
    assert len(raw) == 7 * (4 + 5 * item)
    # every record: int32 little-endian dimension, then the components
    for r in range(7):
        rec = raw[r * (4 + 5 * item):(r + 1) * (4 + 5 * item)]
        assert int.from_bytes(rec[:4], "little") == 5
        assert rec[4:] == a[r].astype(np.dtype(dtype).newbyteorder("<")).tobytes()
    b = getattr(formats, f"read_{kind}")(path)
    assert b.dtype == dtype and np.array_equal(a, b)


def test_vecs_rejects_malformed(tmp_path):
    p = tmp_path / "bad.fvecs"
    p.write_bytes((3).to_bytes(4, "little") + b"\0" * 10)
    with pytest.raises(ValueError):
        formats.read_fvecs(p)
    p.write_bytes((2).to_bytes(4, "little") + b"\0" * 8 + (3).to_bytes(4, "little") + b"\0" * 8)
    with pytest.raises(ValueError):
        formats.read_fvecs(p)


def test_reference_ivecs_layout(tmp_path):
    # reference examples/ground_truth.py:25-30: out[:, 0] = k, out[:, 1:] = ids
    ids = np.arange(12, dtype=np.int32).reshape(3, 4)
    p = tmp_path / "gt.ivecs"
    formats.write_ivecs(p, ids)
    want = np.empty((3, 5), np.int32)
    want[:, 0] = 4
    want[:, 1:] = ids
    assert p.read_bytes() == want.astype("<i4").tobytes()


# ---- cuVS records ------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.int8, np.uint8, np.int32,
                                   np.uint32, np.int64, np.uint64, np.float64])
@pytest.mark.parametrize("shape", [(), (0,), (5,), (3, 4), (2, 3, 4), (123456, 7)])
def test_records_parse_with_numpy(dtype, shape):
    buf = io.BytesIO()
    if shape == ():
        ser.RecordWriter(buf).scalar(3, dtype)
    else:
        ser.RecordWriter(buf).array(np.zeros(shape, dtype))
    raw = buf.getvalue()
    if dtype == np.float16:
        # RAFT spells binary16 "<e2", which NumPy's reader does not know;
        # "<f2" has the same length
        assert b"'descr': '<e2'" in raw
        raw = raw.replace(b"'<e2'", b"'<f2'")
    f = io.BytesIO(raw)
    assert npf.read_magic(f) == (1, 0)
    got_shape, fortran, got_dtype = npf.read_array_header_1_0(f)
    assert got_shape == shape and not fortran and got_dtype == np.dtype(dtype)
    start = f.tell()
    assert start % 64 == 0  # magic + version + length + header: multiple of 64
    assert raw[start - 1:start] == b"\n"
    assert len(raw) - start == int(np.prod(shape)) * np.dtype(dtype).itemsize


def test_record_padding_is_1_to_64_spaces():
    # RAFT pads with 1..64 spaces: when the header would end exactly on a
    # 64-byte boundary it adds a full 64
    # (shapes of 1..130 unit dims give header texts of every length mod 64)
    seen = set()
    for dims in range(1, 131):
        h = ser.record_header(np.float32, (1,) * dims)
        body = h[10:]
        spaces = len(body) - len(body.rstrip(b" \n")) - 1
        assert 1 <= spaces <= 64 and len(h) % 64 == 0
        seen.add(spaces)
    assert seen == set(range(1, 65))


def test_record_values_round_trip():
    buf = io.BytesIO()
    a = np.random.default_rng(2).standard_normal((4, 3)).astype(np.float16)
    w = ser.RecordWriter(buf)
    w.scalar(True, np.bool_)
    w.scalar(2 ** 40 + 3, np.uint64)
    w.scalar(2.5, np.float32)
    w.array(a)
    buf.seek(0)
    r = ser.RecordReader(buf)
    assert r.scalar() == 1
    assert r.scalar() == 2 ** 40 + 3
    assert r.scalar() == 2.5
    assert np.array_equal(r.array(), a)
    # bool has no byte order and is stored as one unsigned byte
    assert b"'descr': '|u1'" in ser.record_header(np.bool_, ())
    # a truncated record is an error, not a short array
    r = ser.RecordReader(io.BytesIO(buf.getvalue()[:-3]))
    for _ in range(3):
        r.scalar()
    with pytest.raises(ValueError, match="ends inside a record"):
        r.array()


def test_dtype_prefix():
    assert ser.type_tag(np.float32, 6) == b"<f4\0"
    assert ser.type_tag(np.float16, 6) == b"<f2\0"
    assert ser.type_tag(np.float16, 5) == b"<e2\0"
    assert ser.type_tag(np.uint8, 6) == b"|u1\0"
    assert ser.read_type_tag(io.BytesIO(b"<f2\0")) == np.float16
    with pytest.raises(ValueError, match="names no cuVS type"):
        ser.read_type_tag(io.BytesIO(b"<c8\0"))


# ---- cuVS brute-force index files ---------------------------------------------------

@pytest.mark.parametrize("metric,code", [("sqeuclidean", 0), ("euclidean", 1), ("cosine", 2),
                                         ("inner_product", 6)])
def test_brute_force_file_round_trip(tmp_path, metric, code):
    x = np.random.default_rng(5).random((10, 3)).astype(np.float32)
    path = tmp_path / "bf.bin"
    brute_force.save(str(path), brute_force.build(x, metric))
    raw = path.read_bytes()
    # reference python/tests/test_cuvs.py:214-221
    assert raw[:4] == b"<f4\0"
    assert raw[4:10] == b"\x93NUMPY"
    f = io.BytesIO(raw[4:])
    r = ser.RecordReader(f)
    fields = [r.scalar() for _ in range(6)]
    assert fields == [0, 10, 3, code, pytest.approx(2.0), 1]
    assert np.array_equal(r.array(), x)
    has_norms = r.scalar()
    assert has_norms == (code in (0, 1, 2))
    if has_norms:
        norms = r.array()
        want = np.sum(x.astype(np.float32) ** 2, axis=1)
        if code == 2:
            want = np.sqrt(want)
        assert np.array_equal(norms, want.astype(np.float32))
    assert f.read() == b""
    idx = brute_force.load(str(path))
    assert idx.trained and idx.distance_type == code and np.array_equal(idx.dataset, x)
    assert len(idx) == 10


def test_brute_force_file_float16_and_hamming(tmp_path):
    x = np.random.default_rng(6).random((4, 8)).astype(np.float16)
    p = tmp_path / "h.bin"
    brute_force.save(str(p), brute_force.build(x))
    assert p.read_bytes()[:4] == b"<f2\0"
    assert brute_force.load(str(p)).dataset.dtype == np.float16
    codes = np.random.default_rng(7).integers(0, 256, (5, 16), dtype=np.uint8)
    brute_force.save(str(p), brute_force.build(codes, metric="bitwise_hamming"))
    idx = brute_force.load(str(p))
    assert idx.distance_type == 20 and np.array_equal(idx.dataset, codes)


def test_brute_force_errors(tmp_path):
    x = np.zeros((4, 3), np.float32)
    with pytest.raises(ValueError, match="not supported"):
        brute_force.build(x, "manhattan")
    # the reference builds with these names, and its search refuses them
    # (python/mlxvs/cuvs/distance.py:151)
    for name in ("jaccard", "dice"):
        with pytest.raises(ValueError, match=f"metric {name} is not supported"):
            brute_force.search(brute_force.build(x, name), x, 1)
    with pytest.raises(ValueError, match="matrix"):
        brute_force.build(np.zeros(3, np.float32))
    with pytest.raises(ValueError, match="uint8"):
        brute_force.build(x, "bitwise_hamming")
    with pytest.raises(ValueError, match="built"):
        brute_force.search(brute_force.Index(), x, 1)

    class Ranges:
        type = "ranges"

    with pytest.raises(ValueError, match="prefilter"):
        brute_force.search(brute_force.build(x), x, 1, prefilter=Ranges())
    p = tmp_path / "nodata.bin"
    brute_force.save(str(p), brute_force.build(x), include_dataset=False)
    with pytest.raises(ValueError, match="without its dataset"):
        brute_force.load(str(p))
    p.write_bytes(b"<f4\0" + b"garbage")
    with pytest.raises(ValueError):
        brute_force.load(str(p))


# ---- argument validation ------------------------------------------------------------

def test_nearest_neighbors_arguments():
    with pytest.raises(ValueError, match="unknown metric"):
        mlxvs_amd.NearestNeighbors(metric="manhattan")
    with pytest.raises(ValueError, match="nn_descent"):
        mlxvs_amd.NearestNeighbors(algorithm="nn_descent")
    with pytest.raises(ValueError, match="algorithm"):
        mlxvs_amd.NearestNeighbors(algorithm="kd_tree")
    nn = mlxvs_amd.NearestNeighbors(3)
    with pytest.raises(RuntimeError, match="fit"):
        nn.kneighbors(np.zeros((2, 2)))
    with pytest.raises(ValueError, match="2-D"):
        nn.fit(np.zeros(5))
    nn.fit(np.zeros((4, 2), np.float32))
    assert nn.n_samples_fit_ == 4 and nn.n_features_in_ == 2
    # reference python/mlxvs/_neighbors.py:71-74: k in [1, n] (n - 1 without X)
    with pytest.raises(ValueError, match="1 <= n_neighbors <= 3"):
        nn.kneighbors(n_neighbors=4)
    with pytest.raises(ValueError, match="1 <= n_neighbors <= 4"):
        nn.kneighbors(np.zeros((1, 2)), n_neighbors=5)
    with pytest.raises(ValueError):
        nn.kneighbors(np.zeros((1, 2)), n_neighbors=0)


def test_kmeans_predict_arguments():
    x = np.zeros((10, 4), np.float32)
    # reference python/tests/test_mlxvs.py:246-247, src/kmeans.cpp:143-153
    with pytest.raises(ValueError, match="same number of columns"):
        mlxvs_amd.kmeans_predict(x, np.zeros((2, 5), np.float32))
    with pytest.raises(ValueError, match="1 <= m <= clusters"):
        mlxvs_amd.kmeans_predict(x, np.zeros((2, 4), np.float32), 3)
    with pytest.raises(ValueError, match="1 <= m <= clusters"):
        mlxvs_amd.kmeans_predict(x, np.zeros((2, 4), np.float32), 0)
    with pytest.raises(ValueError, match="2-D"):
        mlxvs_amd.kmeans_predict(np.zeros(4, np.float32), np.zeros((2, 4), np.float32))


def test_filters_pack_like_cuvs():
    # cuVS's filters (reference python/mlxvs/cuvs/neighbors/filters.py:31-50):
    # bool masks packed little-endian into uint32 words; words kept as they are
    from mlxvs_amd.cuvs.neighbors import filters

    keep = np.zeros(40, bool)
    keep[[0, 5, 31, 32, 39]] = True
    f = filters.from_bitset(keep)
    assert f.type == "bitset" and f.array.dtype == np.uint32
    assert f.array.tolist() == [(1 << 0) | (1 << 5) | (1 << 31), (1 << 0) | (1 << 7)]
    assert filters.from_bitset(np.array([7, 9], np.uint32)).array.tolist() == [7, 9]
    # a bitmap is row-major over (query, row), not padded per query: 3 x 5
    # bits fill one word
    bm = np.zeros((3, 5), bool)
    bm[1, 0] = bm[2, 4] = True
    assert filters.from_bitmap(bm).array.tolist() == [(1 << 5) | (1 << 14)]
    assert filters.no_filter().type == "none"
    with pytest.raises(ValueError):
        filters.Prefilter("ranges")
    with pytest.raises(ValueError):
        filters.from_bitset(np.zeros(3, np.float32))


def test_filtered_argument_checks():
    import mlxvs_amd

    x = np.zeros((40, 4), np.float32)
    with pytest.raises(ValueError, match="not both"):
        mlxvs_amd.brute_force_knn_filtered(x, x, 1, bitset=np.ones(40, bool),
                                           bitmap=np.ones((40, 40), bool))
    with pytest.raises(ValueError, match="words"):
        mlxvs_amd.brute_force_knn_filtered(x, x, 1, bitset=np.ones(1, np.uint32))
    with pytest.raises(ValueError, match=r"\[40, 40\]"):
        mlxvs_amd.brute_force_knn_filtered(x, x, 1, bitmap=np.ones((40, 39), bool))


def test_pairwise_argument_checks():
    import mlxvs_amd

    x = np.zeros((40, 4), np.float32)
    with pytest.raises(ValueError, match="not one of"):
        mlxvs_amd.pairwise_knn(x, x, 1, "manhattan")
    with pytest.raises(ValueError, match="not both"):
        mlxvs_amd.pairwise_knn(x, x, 1, "cityblock", bitset=np.ones(40, bool),
                               bitmap=np.ones((40, 40), bool))
    with pytest.raises(ValueError, match="columns"):
        mlxvs_amd.pairwise_knn(x, np.zeros((3, 5), np.float32), 1, "chebyshev")
    # checked by the engine before any device work
    with pytest.raises(ValueError, match="distance type 11 is not supported"):
        mlxvs_amd.pairwise_knn(x, x, 1, 11)
    with pytest.raises(ValueError, match=r"k must be in \[1, 256\]"):
        mlxvs_amd.pairwise_knn(x, x, 257, "cityblock")
    # the cuVS names the search routes here
    from mlxvs_amd.cuvs.neighbors import brute_force

    for name, code in (("cityblock", 3), ("l1", 3), ("chebyshev", 7), ("canberra", 8),
                       ("minkowski", 9), ("lp", 9), ("correlation", 10), ("hellinger", 12),
                       ("braycurtis", 14), ("jensenshannon", 15), ("hamming", 16),
                       ("kl_divergence", 17), ("russellrao", 18)):
        assert brute_force.build(x, name).distance_type == code
        assert mlxvs_amd.PAIRWISE_DISTANCES[name] == code
