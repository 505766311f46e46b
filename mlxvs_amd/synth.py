"""Seeded synthetic workloads for the exact k-NN configurations.

Every value comes from a counter-based splitmix64 stream, so the same seed
gives the same rows on any machine and in any chunking:

    word(seed, i) = mix64(mix64(seed) + (i + 1) * 0x9E3779B97F4A7C15)

Uniforms take the top 53 bits; normals use Box-Muller on consecutive pairs.
Seeds follow the reference's tests (base 1, queries 2; tests/test_knn.cpp:58-59)
plus 3 for mixture centres.  The five configurations are the workloads of the
MI355X build:

  c1  10,000 x 128 float32 of floor(U[0, 128)); 100 queries alike; L2, k = 10
  c2  1,000,000 x 128 float32, 1,024-component mixture (centres U[0, 128],
      sigma 20), rounded and clipped to [0, 255]; 10,000 queries; L2, k = 10
  c3  1,000,000 x 1,536 unit rows of a 256-cluster mixture (centres N(0, I),
      sigma 0.3); 10,000 queries; inner product / cosine, k = 10
  c4  1,000,000 codes of 1,024 i.i.d. bits; each query is a base code with
      51 distinct bits flipped; Hamming, k = 100
  c5  200,000 x 256 float16 rows of a 512-cluster mixture (sigma 0.5);
      self k-NN graph, L2, k = 64

All generators can produce any row range [lo, hi), so large inputs are built in
chunks and subsets (the first rows, the first queries) cost only their size.
"""

from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix64(z: np.ndarray) -> np.ndarray:
    z = z.copy() if isinstance(z, np.ndarray) else np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z ^= z >> np.uint64(30)
        z *= _M1
        z ^= z >> np.uint64(27)
        z *= _M2
        z ^= z >> np.uint64(31)
    return z


def words(seed: int, lo: int, hi: int) -> np.ndarray:
    """uint64 stream values lo .. hi-1 of `seed`."""
    s0 = _mix64(np.array([seed], dtype=np.uint64))[0]
    idx = np.arange(lo, hi, dtype=np.uint64) + np.uint64(1)
    with np.errstate(over="ignore"):
        z = s0 + idx * _GOLDEN
    return _mix64(z)


def uniform(seed: int, lo: int, hi: int) -> np.ndarray:
    """float64 uniforms in [0, 1) for stream positions lo .. hi-1."""
    return (words(seed, lo, hi) >> np.uint64(11)).astype(np.float64) * (2.0**-53)


def normal(seed: int, lo: int, hi: int) -> np.ndarray:
    """float64 N(0, 1) values lo .. hi-1 (Box-Muller over position pairs)."""
    plo, phi = lo // 2, (hi + 1) // 2
    u = uniform(seed, 2 * plo, 2 * phi).reshape(-1, 2)
    r = np.sqrt(-2.0 * np.log1p(-u[:, 0]))  # 1 - u in (0, 1]
    t = 2.0 * np.pi * u[:, 1]
    z = np.empty((phi - plo, 2))
    z[:, 0] = r * np.cos(t)
    z[:, 1] = r * np.sin(t)
    z = z.reshape(-1)
    return z[lo - 2 * plo : lo - 2 * plo + (hi - lo)]


def _rows_of(fn, seed: int, lo: int, hi: int, d: int) -> np.ndarray:
    return fn(seed, lo * d, hi * d).reshape(hi - lo, d)


# ---- configuration generators ------------------------------------------------

# Each stream seed is split into disjoint sub-streams by adding a large offset,
# so that (for instance) the component choice and the noise of one row never
# share positions.
_SUB = 1 << 40


def c1_rows(seed: int, lo: int, hi: int, d: int = 128) -> np.ndarray:
    """floor(U[0, 128)) as float32 (configuration c1)."""
    return np.floor(_rows_of(uniform, seed, lo, hi, d) * 128.0).astype(np.float32)


def c2_centres(k: int = 1024, d: int = 128) -> np.ndarray:
    return _rows_of(uniform, 3, 0, k, d) * 128.0


def c2_rows(seed: int, lo: int, hi: int, d: int = 128, comps: int = 1024,
            sigma: float = 20.0, centres: np.ndarray | None = None) -> np.ndarray:
    """clip(round(c + sigma N(0, 1)), 0, 255) as float32 (configuration c2)."""
    c = c2_centres(comps, d) if centres is None else centres
    pick = (words(seed + _SUB, lo, hi) % np.uint64(comps)).astype(np.int64)
    x = c[pick] + sigma * _rows_of(normal, seed, lo, hi, d)
    # + 0.0 turns the -0.0 that rint gives for values in (-0.5, 0) into +0.0
    return (np.clip(np.rint(x), 0.0, 255.0) + 0.0).astype(np.float32)


def c3_centres(k: int = 256, d: int = 1536) -> np.ndarray:
    return _rows_of(normal, 3, 0, k, d)


def c3_rows(seed: int, lo: int, hi: int, d: int = 1536, comps: int = 256,
            sigma: float = 0.3, centres: np.ndarray | None = None) -> np.ndarray:
    """L2-normalised c + sigma N(0, I) as float32 (configuration c3)."""
    c = c3_centres(comps, d) if centres is None else centres
    pick = (words(seed + _SUB, lo, hi) % np.uint64(comps)).astype(np.int64)
    x = c[pick] + sigma * _rows_of(normal, seed, lo, hi, d)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    return x.astype(np.float32)


def c4_codes(seed: int, lo: int, hi: int, nbytes: int = 128) -> np.ndarray:
    """i.i.d. Bernoulli(1/2) bits, packed uint8 [hi - lo, nbytes]."""
    nw = (nbytes + 7) // 8
    w = words(seed, lo * nw, hi * nw).reshape(hi - lo, nw)
    return np.ascontiguousarray(w.view(np.uint8).reshape(hi - lo, nw * 8)[:, :nbytes])


def c4_queries(base_fn, n_base: int, seed: int, lo: int, hi: int,
               nbytes: int = 128, flips: int = 51):
    """Queries lo .. hi-1: base row src_j with `flips` distinct bits flipped.

    base_fn(lo, hi) returns base codes; returns (queries uint8, src int64)."""
    src = (words(seed + _SUB, lo, hi) % np.uint64(n_base)).astype(np.int64)
    nbits = nbytes * 8
    q = np.empty((hi - lo, nbytes), dtype=np.uint8)
    for j in range(hi - lo):
        row = base_fn(int(src[j]), int(src[j]) + 1)[0].copy()
        # `flips` distinct bit positions: a partial Fisher-Yates shuffle
        r = words(seed + 2 * _SUB, (lo + j) * flips, (lo + j + 1) * flips)
        perm = np.arange(nbits)
        for t in range(flips):
            u = t + int(r[t] % np.uint64(nbits - t))
            perm[t], perm[u] = perm[u], perm[t]
        for b in perm[:flips]:
            row[b // 8] ^= np.uint8(1 << (7 - b % 8))  # numpy.packbits bit order
        q[j] = row
    return q, src


def c5_centres(k: int = 512, d: int = 256) -> np.ndarray:
    return _rows_of(normal, 3, 0, k, d)


def c5_rows(seed: int, lo: int, hi: int, d: int = 256, comps: int = 512,
            sigma: float = 0.5, centres: np.ndarray | None = None) -> np.ndarray:
    """c + sigma N(0, I) rounded to float16 (configuration c5)."""
    c = c5_centres(comps, d) if centres is None else centres
    pick = (words(seed + _SUB, lo, hi) % np.uint64(comps)).astype(np.int64)
    x = c[pick] + sigma * _rows_of(normal, seed, lo, hi, d)
    return x.astype(np.float16)


def chunked(fn, n: int, chunk: int = 1 << 15, threads: int | None = None) -> np.ndarray:
    """Rows 0 .. n-1 of a row generator fn(lo, hi), built in chunks on a
    thread pool (numpy releases the GIL in the element-wise kernels).  The
    result does not depend on the chunking or the thread count."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    if n <= chunk:
        return fn(0, n)
    threads = threads or min(16, os.cpu_count() or 1)
    first = fn(0, chunk)
    out = np.empty((n,) + first.shape[1:], dtype=first.dtype)
    out[:chunk] = first

    def work(lo):
        hi = min(n, lo + chunk)
        out[lo:hi] = fn(lo, hi)

    with ThreadPoolExecutor(threads) as pool:
        list(pool.map(work, range(chunk, n, chunk)))
    return out
