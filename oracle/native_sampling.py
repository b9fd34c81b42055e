"""Test infrastructure: numpy restatement of the native sampler's random stream and draw
(``g4_sample_tokens``), used only by tests.

The reference draws with ``jax.random.categorical`` (threefry); this build's sampler draws the
same distribution by Gumbel-max with Philox4x32-10 noise (Salmon, Moraes, Dror, Shaw, "Parallel
random numbers: as easy as 1, 2, 3", SC 2011), so its token stream is its own. Pinned by the
published Philox4x32-10 known-answer vectors (tests/test_native_sampling.py).
"""

from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)


def philox4x32_10(ctr: np.ndarray, key: np.ndarray) -> np.ndarray:
    """ctr uint32 [..., 4], key uint32 [..., 2] -> uint32 [..., 4] (10 rounds)."""

    c = [ctr[..., i].astype(np.uint64) for i in range(4)]
    k0, k1 = key[..., 0].astype(np.uint32), key[..., 1].astype(np.uint32)
    mask = np.uint64(0xFFFFFFFF)
    for _ in range(10):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & mask
        hi1, lo1 = p1 >> np.uint64(32), p1 & mask
        c = [hi1 ^ c[1] ^ k0.astype(np.uint64), lo1, hi0 ^ c[3] ^ k1.astype(np.uint64), lo0]
        k0 = (k0 + W0).astype(np.uint32)
        k1 = (k1 + W1).astype(np.uint32)
    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def uniforms(seed: int, step: int, batch: int, vocab: int) -> np.ndarray:
    """u [batch, vocab] in (0, 1): column j of row r from counter (j // 4, r, step, 0), word j % 4."""

    n4 = (vocab + 3) // 4
    ctr = np.zeros((batch, n4, 4), np.uint32)
    ctr[..., 0] = np.arange(n4, dtype=np.uint32)[None, :]
    ctr[..., 1] = np.arange(batch, dtype=np.uint32)[:, None]
    ctr[..., 2] = np.uint32(step)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], np.uint32)
    bits = philox4x32_10(ctr, np.broadcast_to(key, (batch, n4, 2))).reshape(batch, n4 * 4)[:, :vocab]
    return ((bits >> np.uint32(8)).astype(np.float64) + 0.5) / 16777216.0


def sample(logits: np.ndarray, temperature: float, seed: int, step: int) -> tuple[np.ndarray, np.ndarray]:
    """Greedy (temperature <= 0) or Gumbel-max draw on already-capped logits [B, V]; returns
    (token, full-vocab log-softmax at the token)."""

    x = logits.astype(np.float64)
    if temperature > 0:
        g = -np.log(-np.log(uniforms(seed, step, *x.shape)))
        tok = np.argmax(x / temperature + g, axis=-1)
    else:
        tok = np.argmax(x, axis=-1)
    m = x.max(-1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(x - m).sum(-1))
    return tok.astype(np.int32), (x[np.arange(len(tok)), tok] - lse)
