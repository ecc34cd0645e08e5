"""Seeded synthetic workloads for the query path (numpy, vectorised).

Every draw comes from a SplitMix64 stream: the i-th 64-bit output for a seed
is a pure function of (seed, i), so streams are generated as whole arrays.

* uniform f32 in [0, 1):   (x >> 40) * 2**-24
* index in [0, bound):      high 64 bits of x * bound
* standard normal (f64):    Box-Muller on two draws per pair,
                            u1 = ((x0 >> 11) + 1) * 2**-53,  u2 = (x1 >> 11) * 2**-53,
                            z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = ... sin(2 pi u2)

Workloads (seeds 0xF0DB0000 + 16*cfg + {1 base, 2 query, 3 centres}):

  bf_small   10,000 x 128 U[0,1); 100 queries                     (cfg 1)
  bf_norm    N x 128 N(0,1) rows L2-normalised in f64, stored f32  (cfg 2)
  ivfpq_int  1024 centres U[0,255)^128; point = clip(round(centre +
             20 N(0,1)), 0, 255), component uniform                (cfg 3)
  mixture    4096 centres ~ N(0, 4)^dim; point = centre + N(0,1)   (cfg 4, 5)
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)
GAMMA = np.uint64(0x9E3779B97F4A7C15)


def seeds(cfg: int):
    base = 0xF0DB0000 + 16 * cfg
    return base + 1, base + 2, base + 3


def splitmix64(seed: int, start: int, count: int) -> np.ndarray:
    """Outputs start .. start+count-1 of the SplitMix64 stream for `seed`."""
    i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * GAMMA
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform_f32(seed: int, count: int, start: int = 0) -> np.ndarray:
    x = splitmix64(seed, start, count)
    return (x >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)


def indices(seed: int, count: int, bound: int, start: int = 0) -> np.ndarray:
    """floor(x * bound / 2**64) for bound < 2**32, as the 128-bit product does."""
    assert 0 < bound < 2 ** 32
    x = splitmix64(seed, start, count)
    b = np.uint64(bound)
    with np.errstate(over="ignore"):
        hi = (x >> np.uint64(32)) * b
        lo = ((x & np.uint64(0xFFFFFFFF)) * b) >> np.uint64(32)
        return ((hi + lo) >> np.uint64(32)).astype(np.int64)


def normal_f64(seed: int, count: int, start_pair: int = 0) -> np.ndarray:
    pairs = (count + 1) // 2
    x = splitmix64(seed, 2 * start_pair, 2 * pairs)
    u1 = ((x[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (x[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return out[:count]


def _chunked_rows(n: int, dim: int, fn, chunk_rows: int = 1 << 15) -> np.ndarray:
    """Row blocks are pure functions of their range, so they are generated on
    a thread pool (numpy's ufuncs release the GIL); the result does not
    depend on the number of workers."""
    out = np.empty((n, dim), np.float32)

    def block(s):
        e = min(n, s + chunk_rows)
        out[s:e] = fn(s, e)

    starts = range(0, n, chunk_rows)
    workers = min(16, os.cpu_count() or 1, max(1, len(starts)))
    if workers == 1:
        for s in starts:
            block(s)
    else:
        with ThreadPoolExecutor(workers) as pool:
            list(pool.map(block, starts))
    return out


def uniform_rows(seed: int, n: int, dim: int) -> np.ndarray:
    return uniform_f32(seed, n * dim).reshape(n, dim)


def normalized_gaussian_rows(seed: int, n: int, dim: int) -> np.ndarray:
    def rows(s, e):
        z = normal_f64(seed, (e - s) * dim, start_pair=s * dim // 2).reshape(e - s, dim)
        nrm = np.sqrt((z * z).sum(axis=1, keepdims=True))
        nrm[nrm == 0] = 1.0
        return (z / nrm).astype(np.float32)
    assert dim % 2 == 0
    return _chunked_rows(n, dim, rows)


def integer_mixture(seed: int, centres_seed: int, n: int, dim: int = 128, ncomp: int = 1024,
                    std: float = 20.0) -> np.ndarray:
    """clip(round(centre + std*N(0,1)), 0, 255) with uniform component choice."""
    cent = (uniform_f32(centres_seed, ncomp * dim).astype(np.float64) * 255.0).reshape(ncomp, dim)
    comp = indices(seed ^ 0xC0C0, n, ncomp)
    assert dim % 2 == 0

    def rows(s, e):
        z = normal_f64(seed, (e - s) * dim, start_pair=s * dim // 2).reshape(e - s, dim)
        return np.clip(np.rint(cent[comp[s:e]] + std * z), 0.0, 255.0).astype(np.float32)
    return _chunked_rows(n, dim, rows)


def gaussian_mixture(seed: int, centres_seed: int, n: int, dim: int, ncomp: int = 4096,
                     centre_std: float = 2.0) -> np.ndarray:
    """centre ~ N(0, centre_std^2)^dim; point = centre + N(0,1)."""
    assert dim % 2 == 0
    cent = centre_std * normal_f64(centres_seed, ncomp * dim).reshape(ncomp, dim)
    comp = indices(seed ^ 0xC0C0, n, ncomp)

    def rows(s, e):
        z = normal_f64(seed, (e - s) * dim, start_pair=s * dim // 2).reshape(e - s, dim)
        return (cent[comp[s:e]] + z).astype(np.float32)
    return _chunked_rows(n, dim, rows)


# ---------------------------------------------------------------------------
# Named workloads.  `scale` shrinks N and Q (tests use small scales).
# ---------------------------------------------------------------------------
def workload(name: str, n: int = None, nq: int = None):
    """Returns (base [n,dim] f32, queries [nq,dim] f32)."""
    if name == "bf_small":
        b, q, _ = seeds(1)
        n, nq = n or 10_000, nq or 100
        return uniform_rows(b, n, 128), uniform_rows(q, nq, 128)
    if name == "bf_norm":
        b, q, _ = seeds(2)
        n, nq = n or 1_000_000, nq or 10_000
        return normalized_gaussian_rows(b, n, 128), normalized_gaussian_rows(q, nq, 128)
    if name == "ivfpq_int":
        b, q, c = seeds(3)
        n, nq = n or 1_000_000, nq or 10_000
        return integer_mixture(b, c, n), integer_mixture(q, c, nq)
    if name == "ivf_flat":
        b, q, c = seeds(4)
        n, nq = n or 1_000_000, nq or 10_000
        return gaussian_mixture(b, c, n, 96), gaussian_mixture(q, c, nq, 96)
    if name == "ivfpq_large":
        b, q, c = seeds(5)
        n, nq = n or 10_000_000, nq or 10_000
        return gaussian_mixture(b, c, n, 96), gaussian_mixture(q, c, nq, 96)
    raise KeyError(name)
