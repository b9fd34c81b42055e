"""The native sampler (g4_sample_tokens): its Philox4x32-10 stream against the published
known-answer vectors (CPU), and on the GPU: greedy tokens and full-policy log-probabilities, the
exact token stream against the numpy restatement, the sampled distribution, the soft-cap."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import native_sampling as NS

# Philox4x32-10 known-answer vectors of the Random123 distribution (kat_vectors)
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = NS.philox4x32_10(np.array(ctr, np.uint32), np.array(key, np.uint32))
    assert [int(x) for x in got] == list(want)


def test_uniforms_are_open_interval_and_uniform():
    u = NS.uniforms(seed=5, step=3, batch=64, vocab=4096)
    assert u.min() > 0 and u.max() < 1
    assert abs(u.mean() - 0.5) < 0.005 and abs(u.var() - 1 / 12) < 0.002


gpu = pytest.mark.gpu


@gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_greedy_tokens_and_logps(device, dtype):
    from gemma4_posttrain_jax_amd import kernels

    rng = np.random.default_rng(1)
    x = (rng.standard_normal((7, 5003)) * 3).astype(np.float32)
    xd = torch.from_numpy(x).to(device).to(dtype)
    tok, logp = kernels.sample_tokens(xd, softcap=None, temperature=0.0, seed=0, step=0)
    xr = xd.float().cpu().numpy()
    want_tok, want_logp = NS.sample(xr, 0.0, 0, 0)
    np.testing.assert_array_equal(tok.cpu().numpy(), want_tok)
    np.testing.assert_allclose(logp.cpu().numpy(), want_logp, rtol=0, atol=2e-5)


@gpu
def test_sampled_tokens_follow_the_philox_stream(device):
    """Same seed/step -> the numpy restatement's Gumbel-max tokens (a near-tie may resolve
    differently under the device's fast logs: allow one mismatching row in 512)."""

    from gemma4_posttrain_jax_amd import kernels

    rng = np.random.default_rng(2)
    x = rng.standard_normal((512, 1000)).astype(np.float32)
    xd = torch.from_numpy(x).to(device)
    step = torch.tensor([9], dtype=torch.int32, device=device)
    tok, logp = kernels.sample_tokens(xd, softcap=None, temperature=0.7, seed=123456789, step=step)
    want_tok, want_logp = NS.sample(x, 0.7, 123456789, 9)
    got = tok.cpu().numpy()
    assert (got != want_tok).sum() <= 1
    ok = got == want_tok
    np.testing.assert_allclose(logp.cpu().numpy()[ok], want_logp[ok], rtol=0, atol=2e-5)
    tok2, _ = kernels.sample_tokens(xd, softcap=None, temperature=0.7, seed=123456789, step=9)
    np.testing.assert_array_equal(tok2.cpu().numpy(), got)  # device counter == scalar step
    tok3, _ = kernels.sample_tokens(xd, softcap=None, temperature=0.7, seed=123456789, step=10)
    assert (tok3.cpu().numpy() != got).mean() > 0.5  # a new step draws new noise


@gpu
def test_sampled_distribution_matches_softmax(device):
    """65536 independent rows of the same 6 logits: token frequencies against softmax(x / T)
    (chi-square, 5 degrees of freedom, p ~ 1e-4 threshold)."""

    from gemma4_posttrain_jax_amd import kernels

    x = np.array([1.0, 0.5, -0.3, 2.0, 0.0, -1.5], np.float32)
    T = 0.8
    B = 65536
    xd = torch.from_numpy(np.tile(x, (B, 1))).to(device)
    tok, _ = kernels.sample_tokens(xd, softcap=None, temperature=T, seed=77, step=0)
    counts = np.bincount(tok.cpu().numpy(), minlength=6)
    p = np.exp(x / T - (x / T).max())
    p /= p.sum()
    chi2 = (((counts - B * p) ** 2) / (B * p)).sum()
    assert chi2 < 25.7, f"chi2 {chi2}, counts {counts}, expected {B * p}"


@gpu
def test_softcap_matches_torch(device):
    """softcap > 0: x = cast(tanh(l / cap) * cap) in the logits' dtype, then greedy / logp."""

    from gemma4_posttrain_jax_amd import kernels

    rng = np.random.default_rng(3)
    raw = torch.from_numpy((rng.standard_normal((5, 777)) * 40).astype(np.float32)).to(device).to(torch.bfloat16)
    tok, logp = kernels.sample_tokens(raw, softcap=30.0, temperature=0.0, seed=0, step=0)
    capped = (torch.tanh(raw.float() / 30.0) * 30.0).to(torch.bfloat16).float().cpu().numpy()
    want_tok, want_logp = NS.sample(capped, 0.0, 0, 0)
    np.testing.assert_array_equal(tok.cpu().numpy(), want_tok)
    np.testing.assert_allclose(logp.cpu().numpy(), want_logp, rtol=0, atol=2e-5)
