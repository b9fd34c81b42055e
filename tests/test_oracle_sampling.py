"""The oracle's sampler (oracle/jax_random.py + g4_oracle.sample_token / generate), pinned:

* threefry2x32_20 against the Random123 known-answer vectors (the ones JAX's random tests carry);
* ``jax.random.split(PRNGKey(0))`` in the partitionable and the original layout, and
  ``jax.random.uniform(key(0), (3,))``, as JAX's documentation prints them;
* the sampled distribution against transformers' temperature / top-k / top-p warpers and the
  top-p threshold KAT, with the recorded logp the raw full policy's (tests/test_sampler.py:175-217
  of the reference, same logits, keys, counts and tolerances).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import g4_oracle as O
from oracle import jax_random as JR

KAT = [
    ((0, 0), (0, 0), (0x6B200159, 0x99BA4EFE)),
    ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF), (0x1CB996FC, 0xBB002BE7)),
    ((0x13198A2E, 0x03707344), (0x243F6A88, 0x85A308D3), (0xC4923A9C, 0x483DF7A0)),
]


@pytest.mark.parametrize("key,ctr,want", KAT)
def test_threefry_known_answers(key, ctr, want):
    a, b = JR.threefry2x32(key, np.uint32(ctr[0]), np.uint32(ctr[1]))
    assert (int(a), int(b)) == want


def test_split_and_uniform_match_jax_documentation():
    key = JR.prng_key(0)
    assert JR.split(key).tolist() == [[1797259609, 2579123966], [928981903, 3453687069]]
    assert JR.split_original(key).tolist() == [[4146024105, 967050713], [2718843009, 1272950319]]
    np.testing.assert_array_equal(JR.uniform(key, (3,)), np.float32([0.947667, 0.9785799, 0.33229148]))
    assert JR.prng_key(2 ** 32 + 5).tolist() == [1, 5]


def test_uniform_and_gumbel_moments():
    u = JR.uniform(JR.prng_key(7), (1 << 18,))
    assert u.min() >= 0 and u.max() < 1
    assert abs(u.mean() - 0.5) < 0.003 and abs(u.var() - 1 / 12) < 0.001
    g = JR.gumbel(JR.prng_key(8), (1 << 18,))
    assert abs(g.mean() - 0.5772157) < 0.01 and abs(g.var() - np.pi ** 2 / 6) < 0.03


LOGITS = np.float32([[1.1, -0.7, 0.3, 2.0, -2.0], [-1.0, 1.3, 0.6, -2.3, 0.1]])


def expected_distribution(temperature, top_k, top_p):
    from transformers.generation.logits_process import TemperatureLogitsWarper, TopKLogitsWarper, TopPLogitsWarper

    x = torch.from_numpy(LOGITS)
    scores = TemperatureLogitsWarper(temperature)(None, x)
    if top_k:
        scores = TopKLogitsWarper(top_k)(None, scores)
    if top_p < 1:
        scores = TopPLogitsWarper(top_p)(None, scores)
    return torch.softmax(scores, dim=-1).numpy(), torch.log_softmax(x, dim=-1).numpy()


DIST_CASES = [(1.0, 0, 1.0), (0.7, 0, 1.0), (0.8, 3, 1.0), (0.8, 0, 0.85), (0.8, 4, 0.7), (0.8, 0, 1e-50)]


@pytest.mark.parametrize("temperature,top_k,top_p", DIST_CASES)
def test_sampling_distribution_matches_transformers(temperature, top_k, top_p):
    expected, raw = expected_distribution(temperature, top_k, top_p)
    count = 8192
    tokens, logps = O.sample_token(np.repeat(LOGITS, count, axis=0), temperature=temperature, top_k=top_k,
                                   top_p=top_p, key=JR.prng_key(128))
    tokens, logps = tokens.reshape(2, count), logps.reshape(2, count)
    for row in range(2):
        freq = np.bincount(tokens[row], minlength=5) / count
        assert np.all(expected[row, tokens[row]] > 0), "a token outside the truncated set was drawn"
        np.testing.assert_allclose(freq, expected[row], atol=0.025, rtol=0)
        np.testing.assert_allclose(logps[row], raw[row, tokens[row]], atol=2e-6, rtol=0)


def test_top_p_keeps_the_threshold_crossing_token():
    values = np.broadcast_to(np.log(np.float32([0.5, 0.3, 0.2])), (8192, 3)).astype(np.float32)
    tokens, logps = O.sample_token(values, temperature=1.0, top_k=0, top_p=0.6, key=JR.prng_key(29))
    assert set(tokens.tolist()) == {0, 1}
    assert abs(float(np.mean(tokens == 0)) - 0.625) <= 0.025
    np.testing.assert_allclose(logps, np.log(np.float32([0.5, 0.3, 0.2]))[tokens], atol=2e-6)


def test_generate_key_schedule_is_split_per_step():
    """generate draws step t with split(key_t)[1] and carries split(key_t)[0]: the same tokens as
    sample_token fed that schedule by hand."""

    cfg = O.config_from_hf(__import__("hf_util").TINY_A)
    params = O.init_params(cfg, seed=0, dtype=O.F32)
    ids = np.array([[5, 6, 7], [8, 9, 10]], np.int32)
    sc = O.SamplerConfig(3, 4, temperature=1.0, seed=11)
    seen = []
    rb = O.generate(params, cfg, ids, np.ones_like(ids, bool), sampler_config=sc,
                    step_hook=lambda step, logits, cache: seen.append(logits))
    key = JR.prng_key(11)
    for t, logits in enumerate(seen):
        key, sub = JR.split(key)
        tok, _ = O.sample_token(logits, temperature=1.0, key=sub)
        np.testing.assert_array_equal(rb.completion_ids[:, t], tok)


@pytest.mark.parametrize("kw,msg", [(dict(top_k=10 ** 6), "exceeds vocab_size"),
                                    (dict(temperature=float("inf")), "temperature must be finite"),
                                    (dict(temperature=float("nan")), "temperature must be finite"),
                                    (dict(top_p=0.0), "top_p")])
def test_generate_rejects_the_references_invalid_configs(kw, msg):
    """generate raises on the reference's invalid sampler configs (sampler.py:215-224): top_k above
    the vocabulary, a non-finite temperature, top_p outside (0, 1]."""

    cfg = O.config_from_hf(__import__("hf_util").TINY_A)
    params = O.init_params(cfg, seed=0, dtype=O.F32)
    ids = np.array([[5, 6, 7]], np.int32)
    with pytest.raises(ValueError, match=msg):
        O.generate(params, cfg, ids, np.ones_like(ids, bool), sampler_config=O.SamplerConfig(3, 2, **kw))
