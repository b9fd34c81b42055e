"""numpy restatement of the JAX random stream the reference's sampler draws from.

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` as the checker of ``g4_sample_tokens``, never by
the GPU library.

The reference seeds ``jax.random.PRNGKey(seed)`` (sampler.py:239-240), splits the loop key once per
step (sampler.py:265) and draws ``jax.random.categorical(sample_key, scores)`` (sampler.py:179).
That arithmetic lives in the third-party dependency ``jax`` (pyproject.toml:15, ``jax>=0.11.0``,
not vendored, not installed here), whose published algorithm is restated:

* ``threefry2x32``: Threefry-2x32 with 20 rounds (Salmon, Moraes, Dror, Shaw, "Parallel random
  numbers: as easy as 1, 2, 3", SC 2011), as in jax/_src/prng.py.
* ``prng_key``: ``(seed >> 32, seed & 0xffffffff)``.
* ``split``: the partitionable ("foldlike") layout, the default since JAX 0.5.0: key i of the
  split is ``threefry2x32(key, (0, i))``; ``split_original`` is the earlier layout.
* ``random_bits``: element i (row-major) of a shape is the xor of the two words of
  ``threefry2x32(key, (i >> 32, i & 0xffffffff))``.
* ``uniform``: ``bitcast((bits >> 9) | 0x3f800000) - 1`` scaled to ``[minval, maxval)``, floored at
  minval; ``gumbel``: ``-log(-log(uniform(minval=tiny)))``; ``categorical``:
  ``argmax(gumbel + scores)``.

Pins (tests/test_oracle_sampling.py): the three Random123 known-answer vectors of
threefry2x32_20 (the ones JAX's own random tests carry) and ``split(PRNGKey(0))`` in both layouts
as JAX's documentation prints them. The random_bits / uniform layout for non-scalar shapes has no
published vector: parity unpinned beyond the pins above (the GPU kernel is checked against this
restatement, and the distribution against the softmax, as the reference's tests do).
"""

from __future__ import annotations

import numpy as np

_ROT = ((13, 15, 26, 6), (17, 29, 16, 24))


def _rotl(x: np.ndarray, r: int) -> np.ndarray:
    return (x << np.uint32(r)) | (x >> np.uint32(32 - r))


def threefry2x32(key, x0, x1) -> tuple[np.ndarray, np.ndarray]:
    """Threefry-2x32-20 of the counter words ``(x0, x1)`` (broadcast uint32 arrays) under ``key``."""

    k0, k1 = np.uint32(key[0]), np.uint32(key[1])
    ks = (k0, k1, np.uint32(k0 ^ k1 ^ np.uint32(0x1BD11BDA)))
    with np.errstate(over="ignore"):
        a = np.asarray(x0, np.uint32) + ks[0]
        b = np.asarray(x1, np.uint32) + ks[1]
        for i in range(5):
            for r in _ROT[i % 2]:
                a = a + b
                b = _rotl(b, r) ^ a
            a = a + ks[(i + 1) % 3]
            b = b + ks[(i + 2) % 3] + np.uint32(i + 1)
    return a.astype(np.uint32), b.astype(np.uint32)


def prng_key(seed: int) -> np.ndarray:
    """jax.random.PRNGKey(seed) data: uint32 [2]."""

    return np.array([(int(seed) >> 32) & 0xFFFFFFFF, int(seed) & 0xFFFFFFFF], np.uint32)


def split(key, num: int = 2) -> np.ndarray:
    """jax.random.split (partitionable layout): uint32 [num, 2]."""

    a, b = threefry2x32(key, np.zeros(num, np.uint32), np.arange(num, dtype=np.uint32))
    return np.stack([a, b], axis=-1)


def split_original(key, num: int = 2) -> np.ndarray:
    """jax.random.split before partitionable threefry: counters iota(2 num) halved."""

    c = np.arange(2 * num, dtype=np.uint32)
    a, b = threefry2x32(key, c[:num], c[num:])
    return np.concatenate([a, b]).reshape(num, 2)


def random_bits(key, shape: tuple[int, ...]) -> np.ndarray:
    """32-bit random bits of ``shape`` (partitionable layout)."""

    n = int(np.prod(shape, dtype=np.int64))
    flat = np.arange(n, dtype=np.uint64)
    a, b = threefry2x32(key, (flat >> np.uint64(32)).astype(np.uint32), (flat & np.uint64(0xFFFFFFFF)).astype(np.uint32))
    return (a ^ b).reshape(shape)


def uniform(key, shape: tuple[int, ...], minval: float = 0.0, maxval: float = 1.0) -> np.ndarray:
    """float32 uniform in [minval, maxval) from the top 23 bits."""

    bits = random_bits(key, shape)
    f = ((bits >> np.uint32(9)) | np.uint32(0x3F800000)).view(np.float32) - np.float32(1.0)
    lo, hi = np.float32(minval), np.float32(maxval)
    return np.maximum(lo, f * (hi - lo) + lo).astype(np.float32)


def gumbel(key, shape: tuple[int, ...]) -> np.ndarray:
    """float32 standard Gumbel noise: ``-log(-log(u))``, u uniform on [tiny, 1)."""

    u = uniform(key, shape, minval=float(np.finfo(np.float32).tiny), maxval=1.0)
    return (-np.log(-np.log(u))).astype(np.float32)


def categorical(key, scores: np.ndarray) -> np.ndarray:
    """jax.random.categorical over the last axis: ``argmax(gumbel + scores)`` (first on ties)."""

    s = np.asarray(scores, np.float32)
    return np.argmax(gumbel(key, s.shape) + s, axis=-1).astype(np.int32)
