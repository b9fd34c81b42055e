"""Pins of the oracle's attention core (model.py:496-499): a float64 textbook softmax attention,
closed forms for degenerate rows, and the bf16 rounding points (CPU)."""

from __future__ import annotations

import numpy as np

from oracle import g4_oracle as O


def _textbook(q, k, v, mask):
    """float64 softmax(q k^T) v with masked keys excluded; fully masked rows average all keys."""

    B, S, R, H, D = q.shape
    out = np.zeros((B, S, R, H, D))
    for b in range(B):
        for s in range(S):
            for r in range(R):
                for h in range(H):
                    sc = k[b, :, h].astype(np.float64) @ q[b, s, r, h].astype(np.float64)
                    m = np.broadcast_to(mask, (B, 1, 1, S, k.shape[1]))[b, 0, 0, s]
                    if m.any():
                        sc = np.where(m, sc, -np.inf)
                        p = np.exp(sc - sc.max())
                        p /= p.sum()
                    else:
                        p = np.full(sc.shape, 1.0 / sc.size)
                    out[b, s, r, h] = p @ v[b, :, h].astype(np.float64)
    return out


def test_f32_attention_matches_float64_textbook():
    rng = np.random.default_rng(0)
    B, S, R, H, D, T = 2, 3, 2, 2, 16, 11
    q = rng.standard_normal((B, S, R, H, D)).astype(np.float32) * 0.5
    k = rng.standard_normal((B, T, H, D)).astype(np.float32) * 0.5
    v = rng.standard_normal((B, T, H, D)).astype(np.float32)
    mask = rng.random((B, 1, 1, S, T)) > 0.3
    mask[1, 0, 0, 2] = False  # a fully masked row
    got = O.attention_core(q, k, v, mask, O.F32)
    np.testing.assert_allclose(got, _textbook(q, k, v, mask), atol=2e-6, rtol=0)


def test_bf16_attention_is_close_to_textbook_and_exact_on_closed_forms():
    rng = np.random.default_rng(1)
    B, S, R, H, D, T = 1, 4, 1, 1, 32, 9
    q = O.bf16_round(rng.standard_normal((B, S, R, H, D)).astype(np.float32) * 0.3)
    k = O.bf16_round(rng.standard_normal((B, T, H, D)).astype(np.float32) * 0.3)
    v = O.bf16_round(rng.standard_normal((B, T, H, D)).astype(np.float32))
    mask = np.ones((B, 1, 1, S, T), bool)
    mask[0, 0, 0, 1] = False
    mask[0, 0, 0, 1, 4] = True  # row 1: exactly one valid key -> p = 1 -> out = v[4]
    mask[0, 0, 0, 2] = False  # row 2: fully masked -> bf16(1/T) weights on every key
    got = O.attention_core(q, k, v, mask, O.BF16)
    ref = _textbook(q, k, v, mask)
    assert np.abs(got[0, 0] - ref[0, 0]).max() < 3e-2  # bf16 scores / probs / output rounding
    np.testing.assert_array_equal(got[0, 1, 0, 0], v[0, 4, 0])
    uniform = O.bf16_round(np.float32(1.0 / T))
    np.testing.assert_array_equal(got[0, 2, 0, 0], O.bf16_round((uniform * v[0, :, 0].astype(np.float32)).sum(0)))
    # every output is bf16-representable
    np.testing.assert_array_equal(got, O.bf16_round(got))


def test_bf16_scores_are_rounded_before_softmax():
    """Two keys whose f32 scores differ by less than half a bf16 ulp get the same bf16 score and
    therefore equal probabilities (model.py:496: the einsum output is in the input dtype)."""

    D = 8
    q = np.zeros((1, 1, 1, 1, D), np.float32)
    q[..., 0] = 64.0
    k = np.zeros((1, 2, 1, D), np.float32)
    k[0, 0, 0, 0] = 1.0
    k[0, 1, 0, 0] = 1.0 + 2 ** -7  # score 64.5 vs 64: bf16 ulp at 64 is 0.5 -> distinct
    k[0, 1, 0, 1] = 0.0
    v = np.zeros((1, 2, 1, D), np.float32)
    v[0, 0, 0, 0] = 1.0
    v[0, 1, 0, 0] = -1.0
    mask = np.ones((1, 1, 1, 1, 2), bool)
    out_distinct = O.attention_core(q, k, v, mask, O.BF16)[0, 0, 0, 0, 0]
    assert out_distinct < 0  # key 1 wins
    k[0, 1, 0, 0] = 1.0 + 2 ** -9  # score 64.125 rounds to 64.0 in bf16 -> tie
    out_tie = O.attention_core(q, k, v, mask, O.BF16)[0, 0, 0, 0, 0]
    assert out_tie == 0.0
    out_f32 = O.attention_core(q, k, v, mask, O.F32)[0, 0, 0, 0, 0]
    assert out_f32 < 0  # f32 keeps the difference
