"""Pins of the oracle's model forward and decode against HF transformers' Gemma4ForCausalLM (the
reference's own oracle), the committed golden fixture, and the reference's relational
invariants (CPU)."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import hf_util as H
from oracle import g4_oracle as O

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden" / "cfg1_hf.npz"


@pytest.fixture(scope="module", params=["TINY_A", "TINY_B"])
def tiny(request):
    torch.set_grad_enabled(False)
    kw = getattr(H, request.param)
    model = H.build_hf_model(kw, seed=0 if request.param == "TINY_A" else 1)
    cfg = O.config_from_hf(kw)
    return model, H.hf_to_params(model, cfg), cfg


def _close(a, b, rel):
    np.testing.assert_allclose(a, b, atol=rel * max(1.0, float(np.abs(b).max())), rtol=0)


def test_rms_norm_and_rotary_match_hf(tiny):
    """tests/test_model_ops.py:65-86 of the reference."""

    model, params, cfg = tiny
    x = torch.randn(2, 5, cfg.hidden_size)
    _close(O.rms_norm(params.layers[0].input_norm, x.numpy(), cfg.rms_norm_eps, O.F32),
           model.model.layers[0].input_layernorm(x).numpy(), 2e-5)
    pos = np.array([[0, 1, 2, 3, 7], [3, 4, 5, 6, 40]])
    rot = O.make_rotary(cfg, pos)
    for lt in (O.SLIDING, O.FULL):
        cos, sin = model.model.rotary_emb(torch.zeros(2, 5, cfg.hidden_size), torch.from_numpy(pos), lt)
        _close(rot[lt][0], cos.numpy(), 2e-5)
        _close(rot[lt][1], sin.numpy(), 2e-5)


def test_logits_with_left_padding_match_hf(tiny):
    """tests/test_model_ops.py:170-189 of the reference (rel 2e-4 on valid positions)."""

    model, params, cfg = tiny
    rng = np.random.default_rng(2)
    ids = rng.integers(3, cfg.vocab_size, (2, 8))
    mask = np.ones((2, 8), bool)
    mask[1, :3] = False
    ids[1, :3] = cfg.pad_token_id
    pos = np.tile(np.arange(8), (2, 1))
    ref = H.hf_logits(model, ids, mask, pos)
    ours, _, _ = O.forward_lm(params, ids, pos, cfg=cfg, attention_mask=mask)
    _close(ours[mask], ref[mask], 2e-4)
    assert np.abs(ours).max() <= cfg.final_logit_softcapping


def test_kv_cache_decode_matches_full_forward_and_hf(tiny):
    """tests/test_model_ops.py:192-228 of the reference: prefill + one-token appends equal the full
    forward and HF's cached decode (rel 1e-4; see the note on BLAS order below)."""

    model, params, cfg = tiny
    rng = np.random.default_rng(3)
    B, S, k = 2, 9, 5
    ids = rng.integers(3, cfg.vocab_size, (B, S))
    pos = np.tile(np.arange(S), (B, 1))
    full, _, _ = O.forward_lm(params, ids, pos, cfg=cfg)
    cache = O.init_kv_cache(cfg, B, S + 2, O.F32)
    pre, _, cache = O.forward_lm(params, ids[:, :k], pos[:, :k], cfg=cfg, kv_cache=cache)
    # numpy's BLAS sums a 5-row and a 9-row product in different orders (the effect
    # tests/test_sampler.py:20 of the reference describes for XLA); with these std-0.2 weights the
    # f32 difference reaches ~3e-5 of max|x|, so the bar here is the cross-implementation one.
    _close(pre, full[:, :k], 1e-4)
    steps = []
    for t in range(k, S):
        out, _, cache = O.forward_lm(params, ids[:, t:t + 1], pos[:, t:t + 1], cfg=cfg, kv_cache=cache,
                                     cache_mode="append")
        steps.append(out)
    ours = np.concatenate(steps, axis=1)
    _close(ours, full[:, k:], 1e-4)
    hf_pre = model(input_ids=torch.from_numpy(ids[:, :k]), position_ids=torch.from_numpy(pos[:, :k]), use_cache=True)
    hf_rest = model(input_ids=torch.from_numpy(ids[:, k:]), position_ids=torch.from_numpy(pos[:, k:]),
                    past_key_values=hf_pre.past_key_values, use_cache=True)
    _close(ours, hf_rest.logits.numpy(), 1e-4)


def test_decode_across_ring_wraps_matches_full_forward():
    """tests/test_sampler.py:40-79 of the reference: prefill + decode across >= 2 ring wraps."""

    torch.set_grad_enabled(False)
    model = H.build_hf_model(H.TINY_A, seed=0)
    cfg = O.config_from_hf(H.TINY_A)
    params = H.hf_to_params(model, cfg)
    rng = np.random.default_rng(91)
    B, S, P = 2, 10, 5
    ids = rng.integers(3, cfg.vocab_size, (B, S))
    pos = np.tile(np.arange(S), (B, 1))
    logits, _, cache = O.prefill(params, cfg, ids[:, :P], np.ones((B, P), bool), max_new_tokens=S - P)
    full, _, _ = O.forward_lm(params, ids[:, :P], pos[:, :P], cfg=cfg, logits_to_keep=1)
    _close(logits[:, -1], full[:, -1], 1e-4)
    for t in range(P, S):
        out, _, cache = O.decode_step(params, cfg, ids[:, t], pos[:, t], cache)
        full, _, _ = O.forward_lm(params, ids[:, :t + 1], pos[:, :t + 1], cfg=cfg, logits_to_keep=1)
        _close(out[:, -1], full[:, -1], 1e-4)
    assert cache.length == S and S > 2 * cfg.sliding_window


def test_golden_cfg1_greedy_rollout():
    """BASELINE config 1 through the oracle's generate: HF's greedy tokens exactly, logits within
    the reference's HF bar (rel 1e-4, tests/test_model_ops.py:228)."""

    g = np.load(GOLDEN)
    cfg, params = make_golden.cfg1_params()
    np.testing.assert_array_equal(g["prompt_ids"], make_golden.cfg1_prompt())
    steps = []
    rb = O.generate(params, cfg, g["prompt_ids"], np.ones((2, 24), bool),
                    sampler_config=O.SamplerConfig(24, 32, temperature=0.0),
                    step_hook=lambda s, lg, c: steps.append(lg.copy()))
    np.testing.assert_array_equal(rb.completion_ids, g["tokens"])
    _close(np.stack(steps), g["logits"], 1e-4)
    assert rb.lengths.tolist() == [32, 32]


def test_bf16_mode_tracks_f32_mode():
    """The bf16 emulation stays near the f32 forward (catches a wrong rounding point that blows
    up, not bit-level choices)."""

    cfg = O.config_from_hf(dict(H.CFG1, num_hidden_layers=2, layer_types=["sliding_attention", "full_attention"]))
    p32 = O.init_params(cfg, seed=5, dtype=O.BF16, std=0.02)
    ids = np.random.default_rng(0).integers(0, 1024, (2, 12))
    pos = np.tile(np.arange(12), (2, 1))
    a, _, _ = O.forward_lm(p32, ids, pos, cfg=cfg, dtype=O.F32)
    b, _, _ = O.forward_lm(p32, ids, pos, cfg=cfg, dtype=O.BF16)
    assert np.abs(a - b).max() < 0.1
    np.testing.assert_array_equal(b, O.bf16_round(b))


def test_prefill_into_a_filled_cache_attends_to_the_chunk_only(tiny):
    """model.py:604-623 with kv_cache.length > 0 in prefill mode: the chunk's attention uses its own
    K/V and mask only (make_qk_masks over the chunk, query_start 0), so its hidden states equal the
    cache-less forward of the chunk; its K/V land at slots length + s (ring: modulo the window,
    only the last Wc kept), every other slot keeps its contents, and the key mask gains the chunk's
    mask at length."""

    _, params, cfg = tiny
    rng = np.random.default_rng(9)
    B, P0, S, C = 2, 5, 4, 16
    cache = O.init_kv_cache(cfg, B, C, O.F32)
    first = rng.integers(3, cfg.vocab_size, (B, P0))
    _, _, cache = O.forward_lm(params, first, np.tile(np.arange(P0), (B, 1)), cfg=cfg,
                               attention_mask=np.ones((B, P0), bool), kv_cache=cache, cache_mode="prefill")
    chunk = rng.integers(3, cfg.vocab_size, (B, S))
    cmask = np.array([[True] * S, [False] + [True] * (S - 1)])
    cpos = P0 + np.tile(np.arange(S), (B, 1))
    hidden, new = O.forward_text(params, chunk, cpos, cfg=cfg, attention_mask=cmask, kv_cache=cache,
                                 cache_mode="prefill")
    alone, _ = O.forward_text(params, chunk, cpos, cfg=cfg, attention_mask=cmask)
    np.testing.assert_array_equal(hidden, alone)
    fresh = O.init_kv_cache(cfg, B, S, O.F32)
    _, chunk_cache = O.forward_text(params, chunk, cpos, cfg=cfg, attention_mask=cmask, kv_cache=fresh,
                                    cache_mode="prefill")
    for i, (old, got, ref) in enumerate(zip(cache.layers, new.layers, chunk_cache.layers)):
        if old is None:
            assert got is None
            continue
        ring = cfg.layer_types[i] == O.SLIDING
        wc = old.key.shape[1]
        keep = min(S, wc)
        slots = [(P0 + s) % wc if ring else P0 + s for s in range(S - keep, S)]
        # a fresh ring of min(W, S) slots holds the chunk's last tokens at slot s mod min(W, S)
        src = [s % ref.key.shape[1] if ring else s for s in range(S - keep, S)]
        np.testing.assert_array_equal(got.key[:, slots], ref.key[:, src])
        np.testing.assert_array_equal(got.value[:, slots], ref.value[:, src])
        others = [c for c in range(wc) if c not in slots]
        np.testing.assert_array_equal(got.key[:, others], old.key[:, others])
    np.testing.assert_array_equal(new.key_mask[:, P0:P0 + S], cmask)
    np.testing.assert_array_equal(new.key_mask[:, :P0], cache.key_mask[:, :P0])
    assert new.length == P0 + S
