"""The seeded workload generators behind the benchmark and the fixtures."""

import numpy as np

from mlxvs_amd import synth


def test_stream_is_chunking_independent():
    a = synth.normal(5, 0, 1001)
    b = np.concatenate([synth.normal(5, 0, 3), synth.normal(5, 3, 500), synth.normal(5, 500, 1001)])
    assert np.array_equal(a, b)
    x = synth.chunked(lambda lo, hi: synth.c2_rows(1, lo, hi), 5000, chunk=777)
    assert np.array_equal(x, synth.c2_rows(1, 0, 5000))


def test_known_values():
    # splitmix64 of seed 0: the first outputs of the reference generator
    # (state 0 -> mix64(0x9E3779B97F4A7C15) = 0xE220A8397B1DCDAF)
    z = synth._mix64(np.array([0x9E3779B97F4A7C15], dtype=np.uint64))[0]
    assert int(z) == 0xE220A8397B1DCDAF


def test_distributions():
    u = synth.uniform(9, 0, 200_000)
    assert 0 <= u.min() and u.max() < 1 and abs(u.mean() - 0.5) < 0.01
    z = synth.normal(9, 0, 200_000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_configuration_shapes_and_ranges():
    c1 = synth.c1_rows(1, 0, 100)
    assert c1.dtype == np.float32 and c1.min() >= 0 and c1.max() <= 127
    assert (c1 == np.floor(c1)).all()
    c2 = synth.c2_rows(1, 0, 1000)
    assert c2.min() >= 0 and c2.max() <= 255 and (c2 == np.rint(c2)).all()
    assert not np.signbit(c2).any()
    c3 = synth.c3_rows(1, 0, 50, d=64, comps=4)
    assert np.allclose(np.linalg.norm(c3, axis=1), 1, atol=1e-6)
    c5 = synth.c5_rows(1, 0, 50, d=32, comps=8)
    assert c5.dtype == np.float16


def test_c4_queries_flip_exact_bits():
    gen = lambda lo, hi: synth.c4_codes(1, lo, hi)  # noqa: E731
    q, src = synth.c4_queries(gen, 10_000, 2, 0, 50)
    base = gen(0, 10_000)
    flips = np.unpackbits(q ^ base[src], axis=1).sum(1)
    assert (flips == 51).all()
