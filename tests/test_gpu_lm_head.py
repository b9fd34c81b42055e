"""GPU parity of the LM head with the sampler in its epilogue (g4_lm_head_sample).

The logits it can write (logits_out, before the soft-cap) are checked against the f64 product
rounded to bf16; its draw is checked token for token against the oracle's _sample_token
(oracle/g4_oracle.py, whose JAX random stream the threefry known-answer vectors pin) over those
same logits soft-capped in bf16, and against g4_sample_tokens run on them: greedy and categorical,
with and without the soft-cap, batches from 1 row to 256, the benchmarked shape (262,144 columns,
hidden 2048), ties, the key split and back-to-back calls that share one workspace."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import g4_oracle as O
from oracle import jax_random as JR

from gemma4_posttrain_jax_amd import kernels
from gemma4_posttrain_jax_amd import sampler as SMP

pytestmark = pytest.mark.gpu

LOGP_ATOL = 2e-6  # the reference's logp tolerance (tests/test_sampler.py:204, 217)


def _words(t: torch.Tensor) -> list[int]:
    return [int(w) & 0xFFFFFFFF for w in t.cpu().tolist()]


def _operands(device, B, V, M, seed, scale=0.05):
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((B, M)).astype(np.float32)).to(device).to(torch.bfloat16)
    e = torch.from_numpy((rng.standard_normal((V, M)) * scale).astype(np.float32)).to(device).to(torch.bfloat16)
    return x, e


def _check_logits(x, e, logits):
    """bf16 logits of an f32-accumulated product: within one bf16 rounding (2^-8 relative) of the
    f64 product, plus the f32 accumulation's bound (2^-20 of sum |x||e|)."""

    xd, ed = x.double().cpu(), e.double().cpu()
    ref = (xd @ ed.T).numpy()
    mag = (xd.abs() @ ed.abs().T).numpy()
    got = logits.double().cpu().numpy()
    err = np.abs(got - ref)
    bound = np.abs(ref) * 2.0 ** -8 + mag * 2.0 ** -20
    assert (err <= bound).all(), f"max excess {float((err - bound).max())}"


def _capped(logits: torch.Tensor, cap) -> np.ndarray:
    """The soft-cap as forward_lm_head applies it: tanh(l / cap) * cap in f32, rounded to bf16."""

    if cap is None:
        return logits.float().cpu().numpy()
    return (torch.tanh(logits.float() / cap) * cap).to(torch.bfloat16).float().cpu().numpy()


@pytest.mark.parametrize("B,V,M", [(1, 128, 128), (7, 1024, 192), (256, 2048, 256), (100, 4096, 1536), (37, 66048, 128)])
def test_lm_head_logits(device, B, V, M):
    x, e = _operands(device, B, V, M, seed=B + V)
    logits = kernels.lm_head(x, e)
    torch.cuda.synchronize()
    _check_logits(x, e, logits)


def _draw_and_check(device, B, V, M, temperature, cap, seed, key_words=(7, 123)):
    x, e = _operands(device, B, V, M, seed=seed)
    key = SMP.key_tensor(list(key_words), device)
    logits = torch.empty((B, V), dtype=torch.bfloat16, device=device)
    tok, logp = kernels.lm_head_sample(x, e, softcap=cap, temperature=temperature, key=key, logits_out=logits)
    torch.cuda.synchronize()
    _check_logits(x, e, logits)
    nxt, sub = JR.split(np.uint32(key_words))
    want_tok, want_logp = O.sample_token(_capped(logits, cap), temperature=temperature, key=sub)
    np.testing.assert_array_equal(tok.cpu().numpy(), want_tok)
    np.testing.assert_allclose(logp.cpu().numpy(), want_logp, rtol=0, atol=LOGP_ATOL)
    if temperature > 0:
        assert _words(key) == nxt.tolist()  # the loop key advanced to split(key)[0]
    # g4_sample_tokens on the same logits draws the same tokens
    key2 = SMP.key_tensor(list(key_words), device)
    tok2, logp2 = kernels.sample_tokens(logits, softcap=cap, temperature=temperature, key=key2)
    np.testing.assert_array_equal(tok2.cpu().numpy(), tok.cpu().numpy())
    np.testing.assert_allclose(logp2.cpu().numpy(), logp.cpu().numpy(), rtol=0, atol=LOGP_ATOL)
    return tok, logp


@pytest.mark.parametrize("B,V,M,temperature,cap", [
    (7, 1024, 128, 1.0, 30.0),
    (7, 1024, 128, 0.7, None),
    (1, 128, 128, 1.0, 30.0),
    (33, 2048, 192, 0.0, 30.0),
    (256, 4096, 128, 1.0, 30.0),
    (200, 8192, 256, 0.8, 5.0),
    (37, 66048, 128, 1.0, 30.0),
    (256, 99968, 128, 0.9, 30.0),
])
def test_fused_draw_matches_oracle(device, B, V, M, temperature, cap):
    """Vocabularies of up to 256 tiles of 128 give each workgroup one tile (one team multiplies it,
    then runs its epilogue while the other team idles); 66,048 and 99,968 columns give every
    workgroup two or three (the teams' GEMM and epilogue phases overlap)."""

    _draw_and_check(device, B, V, M, temperature, cap, seed=V + B)


def test_fused_draw_matches_oracle_at_the_e2b_shape(device):
    """B = 256 rows over the 262,144-entry vocabulary with hidden 2048 (the benchmarked decode
    step's LM head), T = 1, soft-cap 30."""

    _draw_and_check(device, 256, 262144, 2048, 1.0, 30.0, seed=11)


def test_fused_greedy_ties_take_the_first_column(device):
    """Row b's logits are embed[:, b]: a tie between columns 17 and 4000 (row 0), one maximum in
    the last column (row 1), an all-zero row (row 2: column 0, logp = -log V)."""

    B, V, M = 3, 4096, 128
    x = torch.zeros((B, M), dtype=torch.bfloat16, device=device)
    x[torch.arange(B), torch.arange(B)] = 1.0
    e = torch.zeros((V, M), dtype=torch.bfloat16, device=device)
    e[17, 0] = e[4000, 0] = 1.0
    e[V - 1, 1] = 2.0
    tok, logp = kernels.lm_head_sample(x, e, softcap=30.0, temperature=0.0, key=None)
    assert tok.cpu().tolist() == [17, V - 1, 0]
    np.testing.assert_allclose(logp[2].item(), -np.log(float(V)), atol=LOGP_ATOL)


def test_fused_sample_key_without_split_stays(device):
    x, e = _operands(device, 5, 1024, 128, seed=5)
    sub = JR.split(np.uint32([3, 4]))[1]
    key = SMP.key_tensor(list(map(int, sub)), device)
    logits = torch.empty((5, 1024), dtype=torch.bfloat16, device=device)
    tok, _ = kernels.lm_head_sample(x, e, softcap=30.0, temperature=1.0, key=key, split_key=False, logits_out=logits)
    want, _ = O.sample_token(_capped(logits, 30.0), temperature=1.0, key=sub)
    np.testing.assert_array_equal(tok.cpu().numpy(), want)
    assert _words(key) == [int(w) for w in sub]


def test_fused_back_to_back_calls(device):
    """A 256-row call then a 9-row call (the second leaves most of the per-workgroup states from the
    first in place): each equals its own oracle draw."""

    _draw_and_check(device, 256, 2048, 128, 1.0, 30.0, seed=21, key_words=(1, 2))
    _draw_and_check(device, 9, 2048, 128, 1.0, 30.0, seed=22, key_words=(1, 2))


@pytest.mark.parametrize("temperature", [0.0, 1.0, 0.7])
def test_fused_draw_takes_the_first_nan_column(device, temperature):
    """jnp.argmax's rule (the greedy argmax and the one inside jax.random.categorical,
    sampler.py:145-183): a NaN score beats every number and the first NaN column wins. Embedding
    rows 7 and 3000 hold a NaN, so every row's logits there are NaN: every row draws column 7 with
    a NaN log-probability, as the oracle's numpy argmax gives."""

    B, V, M = 6, 4096, 128
    x, e = _operands(device, B, V, M, seed=3)
    e[7, 5] = float("nan")
    e[3000, 9] = float("nan")
    key = SMP.key_tensor([5, 6], device)
    logits = torch.empty((B, V), dtype=torch.bfloat16, device=device)
    tok, logp = kernels.lm_head_sample(x, e, softcap=30.0, temperature=temperature, key=key, logits_out=logits)
    torch.cuda.synchronize()
    assert tok.cpu().tolist() == [7] * B
    assert torch.isnan(logp).all()
    want_tok, _ = O.sample_token(_capped(logits, 30.0), temperature=temperature, key=JR.split(np.uint32([5, 6]))[1])
    np.testing.assert_array_equal(tok.cpu().numpy(), want_tok)
