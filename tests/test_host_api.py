"""Host-side pieces of the drop-in API on the CPU: the one-GPU sharding identities and the top-p
proposal's cumulative mass, each against the reference's definition (no GPU needed)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import g4_oracle as O

from gemma4_posttrain_jax_amd import sampler as SMP
from gemma4_posttrain_jax_amd import sharding as SH


def test_constrain_batch_is_the_identity_without_a_mesh():
    """sharding.py:186-199: with the whole batch on one device the constraint changes nothing; a
    mesh is rejected, as everywhere on this path."""

    x = torch.arange(12, dtype=torch.int32).reshape(3, 4)
    assert SH.constrain_batch(x) is x
    tree = SMP.RolloutBatch(x, x, x.bool(), x.float(), x[:, 0])
    assert SH.constrain_batch_tree(tree) is tree
    assert SH.constrain_batch_tree({"a": x, "s": torch.tensor(1.0), "n": None}, None)["a"] is x
    with pytest.raises(ValueError, match="one GPU"):
        SH.constrain_batch(x, mesh=object())
    with pytest.raises(ValueError, match="one GPU"):
        SH.constrain_batch_tree(tree, mesh=object())


def _oracle_keep(scores: np.ndarray, top_p: float) -> np.ndarray:
    """The keep mask of sampler.py:172-178 on descending-sorted scores, through the oracle's
    formula (previous mass = 0 followed by the cumulative sum without its last entry)."""

    w = np.exp(scores - scores.max(axis=-1, keepdims=True))
    probs = w / w.sum(axis=-1, keepdims=True, dtype=np.float32)
    prev = np.concatenate([np.zeros_like(probs[:, :1]), np.cumsum(probs, axis=-1, dtype=np.float32)[:, :-1]], -1)
    return (prev < np.float32(top_p)) | (np.arange(scores.shape[-1])[None, :] == 0)


@pytest.mark.parametrize("vocab,index", [(3, 2), (11, 6), (12, 6)])
def test_top_p_keeps_the_reference_boundary_token(vocab, index):
    """Equal logits make every probability 1/V. top_p is set to the previous mass of column
    ``index`` exactly as the reference forms it (sampler.py:172-174: concatenated zero and
    cumulative sum), a value where ``cumsum - probs`` rounds one ulp lower. The reference drops
    that column (previous < top_p is false); the other formula would keep it."""

    logits = np.zeros((1, vocab), np.float32)
    probs = np.full(vocab, np.float32(1.0) / np.float32(vocab), np.float32)
    cum = np.cumsum(probs, dtype=np.float32)
    top_p = float(cum[index - 1])
    assert np.float32(cum[index] - probs[index]) < np.float32(top_p)  # the case the formulas disagree on
    want = _oracle_keep(logits, top_p)
    assert not want[0, index] and want[0, index - 1]
    scores, ids = SMP._proposal(torch.from_numpy(logits), 1.0, 0, top_p)
    np.testing.assert_array_equal(ids.numpy(), np.arange(vocab)[None])  # stable order of equal scores
    np.testing.assert_array_equal(torch.isfinite(scores).numpy(), want)


def test_top_p_matches_the_oracle_on_random_rows():
    """Truncation of sampler.py:162-178 (temperature, top-k, top-p) against the oracle's keep mask
    on random rows, with and without top-k."""

    rng = np.random.default_rng(5)
    logits = rng.standard_normal((6, 300)).astype(np.float32) * 3
    for temperature, top_k, top_p in ((0.7, 0, 0.9), (1.3, 40, 0.5), (1.0, 0, 0.3)):
        scores, ids = SMP._proposal(torch.from_numpy(logits), temperature, top_k, top_p)
        s = logits / np.float32(temperature)
        order = np.argsort(-s, axis=-1, kind="stable")
        if top_k:
            order = order[:, :top_k]
        np.testing.assert_array_equal(ids.numpy(), order)
        sorted_scores = np.take_along_axis(s, order, axis=-1)
        np.testing.assert_array_equal(torch.isfinite(scores).numpy(), _oracle_keep(sorted_scores, top_p))


def test_softcap_of_zero_or_below_is_rejected_on_every_path():
    """One behaviour for a non-positive final_logit_softcapping: ValueError from the check every LM-head
    path applies (forward_lm_head here; the graphed step and generate call the same check)."""

    from gemma4_posttrain_jax_amd import model as M

    e = torch.randn(16, 8)
    h = torch.randn(1, 2, 8)
    for cap in (0.0, -3.0, float("nan"), float("inf")):
        with pytest.raises(ValueError, match="final_logit_softcapping"):
            M.forward_lm_head(e, h, cap)
    assert M.checked_softcap(None) is None and M.checked_softcap(30) == 30.0
    # f32: the product accumulates in f64 and rounds once (model._mm)
    np.testing.assert_array_equal(M.forward_lm_head(e, h, None).numpy(), (h.double() @ e.double().t()).float().numpy())
