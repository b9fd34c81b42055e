"""Pins of the oracle's integer/index semantics: the reference's known-answer tests, closed forms
and brute-force enumeration (CPU)."""

from __future__ import annotations

import itertools

import numpy as np
import pytest

import hf_util as H
from oracle import g4_oracle as O

E2B_LIKE = dict(
    vocab_size=262144, hidden_size=2048, intermediate_size=8192, num_hidden_layers=30, num_attention_heads=8,
    num_key_value_heads=2, head_dim=256, global_head_dim=256,
    layer_types=(["sliding_attention"] * 4 + ["full_attention"]) * 6, sliding_window=512, num_kv_shared_layers=10,
    hidden_size_per_layer_input=0,
)


def test_kv_source_layer_reference_kat():
    """tests/test_model_ops.py:62 of the reference: TINY_A layer 4 <- 3, layer 5 <- 1."""

    cfg = O.config_from_hf(H.TINY_A)
    assert O.kv_source_layer(cfg, 4) == 3 and O.kv_source_layer(cfg, 5) == 1
    assert [O.is_kv_shared(cfg, i) for i in range(6)] == [False] * 4 + [True] * 2


def test_kv_source_layer_e2b_like_mapping():
    """SSSSG x6, last 10 shared -> sliding 20-23, 25-28 <- 18; global 24, 29 <- 19."""

    cfg = O.config_from_hf(E2B_LIKE)
    got = {i: O.kv_source_layer(cfg, i) for i in range(20, 30)}
    assert got == {20: 18, 21: 18, 22: 18, 23: 18, 24: 19, 25: 18, 26: 18, 27: 18, 28: 18, 29: 19}
    assert all(O.kv_source_layer(cfg, i) == i for i in range(20))


def test_kv_source_layer_brute_force():
    """Every 2-type pattern of up to 7 layers: the source is the largest j < first_shared with the
    same type (or a ValueError when there is none)."""

    for n in range(1, 8):
        for pattern in itertools.product([O.SLIDING, O.FULL], repeat=n):
            for shared in range(0, n + 1):
                cfg = O.Config(8, 8, 8, n, 2, 1, 8, 8, None, pattern, 4, num_kv_shared_layers=shared)
                first = n - shared
                for i in range(n):
                    same = [j for j in range(first) if pattern[j] == pattern[i]]
                    if shared == 0 or i < first:
                        assert O.kv_source_layer(cfg, i) == i
                    elif same:
                        assert O.kv_source_layer(cfg, i) == max(same)
                    else:
                        with pytest.raises(ValueError):
                            O.kv_source_layer(cfg, i)


def test_cache_shapes_reference_kat():
    """tests/test_sampler.py:25-37 of the reference: ring only on non-shared sliding layers."""

    cfg = O.config_from_hf(H.TINY_A)
    cache = O.init_kv_cache(cfg, 2, 11, O.F32)
    assert cache.key_mask.shape == (2, 11)
    for i, layer in enumerate(cache.layers):
        if O.is_kv_shared(cfg, i):
            assert layer is None
            continue
        expected = cfg.sliding_window if cfg.layer_types[i] == O.SLIDING else 11
        assert layer.key.shape[1] == expected and layer.value.shape == layer.key.shape


@pytest.mark.parametrize("wc", [1, 3, 16, 512])
def test_ring_slot_positions_match_simulated_writes(wc):
    """model.py:357 closed form == writing positions 0..n one by one into slot p % Wc."""

    for n in list(range(0, 3 * wc + 2)) + [2047, 4096 + wc // 2]:
        stored = np.full(wc, -1, np.int64)
        for p in range(n + 1):
            stored[p % wc] = p
        got = O.ring_slot_positions(n, wc)
        # never-written slots: the closed form yields a negative position
        np.testing.assert_array_equal(np.where(stored >= 0, got, -1), stored)
        assert np.all(got[stored < 0] < 0)


def test_cached_masks_match_brute_force():
    """make_cached_qk_masks (model.py:338-365) against a cache that records each slot's position,
    with left padding, a finished row and per-row query positions."""

    rng = np.random.default_rng(0)
    B, C, W = 4, 40, 7
    key_mask = rng.random((B, C)) > 0.2
    key_mask[2, :] = False
    q = np.array([3, 17, 39, 25])
    masks = O.make_cached_qk_masks(key_mask, W, q, 1)
    wc = min(W, C)
    for b in range(B):
        stored = np.full(wc, -1)
        for p in range(q[b] + 1):
            stored[p % wc] = p
        for r in range(wc):
            p = stored[r]
            want = p >= 0 and p <= q[b] and p > q[b] - W and key_mask[b, p]
            assert masks[O.SLIDING][b, 0, 0, 0, r] == want
        for t in range(C):
            assert masks[O.FULL][b, 0, 0, 0, t] == (t <= q[b] and key_mask[b, t])


def test_prefill_masks_brute_force():
    """make_qk_masks (model.py:320-335): causal, key padding, window in physical index space."""

    key_mask = np.array([[0, 0, 1, 1, 1, 1, 1, 1], [1] * 8], bool)
    masks = O.make_qk_masks(key_mask, 3, 0, 8)
    for b, s, t in itertools.product(range(2), range(8), range(8)):
        full = t <= s and key_mask[b, t]
        assert masks[O.FULL][b, 0, 0, s, t] == full
        assert masks[O.SLIDING][b, 0, 0, s, t] == (full and t > s - 3)


def test_append_slots_ring_keeps_last_window():
    """model.py:383-386: a chunk longer than the ring keeps only its last Wc tokens, slots unique."""

    dst, src = O.append_slots(5, 20, 8, True)
    np.testing.assert_array_equal(src, np.arange(12, 20))
    np.testing.assert_array_equal(np.sort(dst), np.arange(8))
    np.testing.assert_array_equal(dst, (np.arange(12, 20) + 5) % 8)
    layer = O.LayerKV(np.zeros((1, 8, 1, 2), np.float32), np.zeros((1, 8, 1, 2), np.float32))
    k = np.arange(20, dtype=np.float32)[None, :, None, None] * np.ones((1, 20, 1, 2), np.float32)
    out = O.update_layer_cache(layer, k, k, 5, True, O.F32)
    for r in range(8):  # the slot holds the latest position p with p % 8 == r among 5..24
        p = max(p for p in range(5, 25) if p % 8 == r)
        assert out.key[0, r, 0, 0] == p - 5


def test_linear_append_clamps_like_dynamic_update_slice():
    layer = O.LayerKV(np.zeros((1, 6, 1, 1), np.float32), np.zeros((1, 6, 1, 1), np.float32))
    k = np.ones((1, 3, 1, 1), np.float32)
    out = O.update_layer_cache(layer, k, k, 5, False, O.F32)
    np.testing.assert_array_equal(out.key[0, :, 0, 0], [0, 0, 0, 1, 1, 1])


def test_position_ids_kat():
    """sampler.py:63-67: left padding stays at 0; real tokens count from 0."""

    mask = np.array([[0, 0, 1, 1, 1], [1, 1, 1, 1, 1]], bool)
    np.testing.assert_array_equal(O.position_ids(mask), [[0, 0, 0, 1, 2], [0, 1, 2, 3, 4]])


def test_bf16_round_known_values():
    vals = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -9, -2.5, 3.4e38, np.inf], np.float32)
    got = O.bf16_round(vals)
    np.testing.assert_array_equal(got[:5], np.array([1.0, 1.0, 1.0 + 2 ** -6, 1.0, -2.5], np.float32))
    assert got[5] == np.inf and got[6] == np.inf  # 3.4e38 rounds past bf16 max
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32))[0])
    assert O.BF16_MIN == O.from_bf16_bits(np.array([0xFF7F], np.uint16))[0]
