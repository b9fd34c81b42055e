"""Pins of the oracle's bf16 rounding points against Hugging Face's Gemma 4 modules run in torch
bf16 on the CPU (an implementation independent of the oracle, the one the reference is tested
against: tests/test_model_ops.py of the reference).

Where the reference rounds explicitly, HF rounds at the same points, and the oracle must equal
HF's bf16 output bit for bit:
- attention core (model.py:496-499): bf16 scores, masked fill, f32 softmax, bf16 probabilities,
  bf16 output -- HF's ``eager_attention_forward``;
- RMSNorm (model.py:278-285): f32 statistics, one rounding -- ``Gemma4RMSNorm``;
- the embedding scale (model.py:600): bf16 embedding times the bf16-rounded sqrt(M) --
  ``Gemma4TextScaledWordEmbedding``.

Where a reference line is an elementwise chain (RoPE with cos/sin cast to the activation dtype,
model.py:309-317; gelu(gate) * up, model.py:396; the soft-cap, model.py:679), XLA evaluates the
fused chain in f32 and rounds once; torch rounds after every op (HF's per-op bf16 results agree
with the fused ones on only 68-93 % of the elements). There the oracle must equal HF's own
formula evaluated in f32 on the same bf16 inputs (HF's bf16 cos/sin included) and rounded once.

Each pin is shown to catch a plausible mistake: the same comparison on an oracle with a rounding
point removed or added (planted here, on the CPU) fails.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import hf_util as H
from oracle import g4_oracle as O

MG = pytest.importorskip("transformers.models.gemma4.modeling_gemma4")

EXACT = 0.999  # bit-equal fraction required where only libm last-ulp differences may remain


def _bf(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy()


def _exact(a, b) -> float:
    return float((np.asarray(a, np.float32) == np.asarray(b, np.float32)).mean())


def _spacing(a) -> np.ndarray:
    """bf16 spacing at the magnitude of each element (2^(e - 7) for |a| in [2^e, 2^(e+1)))."""

    mag = np.abs(np.asarray(a, np.float32))
    return np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.maximum(mag, 1e-30))) - 7), 0.0)


@pytest.fixture(scope="module", autouse=True)
def _no_grad():
    with torch.no_grad():
        yield


# --- attention core ---------------------------------------------------------------------------


class _AttnModule:
    training = False

    def __init__(self, R: int, D: int):
        self.num_key_value_groups = R
        self.head_dim = D


def _attention_case(seed: int):
    rng = np.random.default_rng(seed)
    B, S, R, Hh, D = 2, 40, 4, 2, 64
    q = O.cast(rng.standard_normal((B, S, R, Hh, D)).astype(np.float32), O.BF16)
    k = O.cast(rng.standard_normal((B, S, Hh, D)).astype(np.float32), O.BF16)
    v = O.cast(rng.standard_normal((B, S, Hh, D)).astype(np.float32), O.BF16)
    km = np.ones((B, S), bool)
    km[1, :5] = False  # left padding: five fully masked query rows
    mask = O.make_qk_masks(km, 16, 0, S)[O.SLIDING]
    qh = _bf(q.transpose(0, 3, 2, 1, 4).reshape(B, Hh * R, S, D))  # HF head order h * R + r
    kh, vh = _bf(k.transpose(0, 2, 1, 3)), _bf(v.transpose(0, 2, 1, 3))
    fill = torch.finfo(torch.bfloat16).min
    am = torch.where(torch.from_numpy(mask[:, 0]), 0.0, fill).to(torch.bfloat16)
    out, _ = MG.eager_attention_forward(_AttnModule(R, D), qh, kh, vh, am, scaling=1.0)
    hf = _np(out).reshape(B, S, Hh, R, D).transpose(0, 1, 3, 2, 4)
    return q, k, v, mask, hf


def _attention_variant(q, k, v, mask, *, round_scores=True, round_probs=True):
    """attention_core with one of its roundings removed (a planted mistake)."""

    B, S, R, Hh, D = q.shape
    T = k.shape[1]
    sc = np.matmul(q.transpose(0, 2, 3, 1, 4), k.transpose(0, 2, 3, 1)[:, None]).astype(np.float32)
    if round_scores:
        sc = O.cast(sc, O.BF16)
    sc = np.where(np.broadcast_to(mask, (B, R, Hh, S, T)), sc, O.BF16_MIN)
    e = np.exp(sc - sc.max(-1, keepdims=True))
    p = e / e.sum(-1, keepdims=True)
    if round_probs:
        p = O.cast(p, O.BF16)
    return O.cast(np.matmul(p, v.transpose(0, 2, 1, 3)[:, None]), O.BF16).transpose(0, 3, 1, 2, 4)


@pytest.mark.parametrize("seed", [0, 1])
def test_attention_core_equals_hf_eager_bf16(seed):
    q, k, v, mask, hf = _attention_case(seed)
    assert _exact(O.attention_core(q, k, v, mask, O.BF16), hf) == 1.0
    # planted: the probability rounding or the score rounding dropped
    assert _exact(_attention_variant(q, k, v, mask, round_probs=False), hf) < 0.9
    assert _exact(_attention_variant(q, k, v, mask, round_scores=False), hf) < 0.9


# --- RMSNorm, embedding scale -----------------------------------------------------------------


def test_rms_norm_equals_hf_bf16():
    rng = np.random.default_rng(2)
    x = O.cast(rng.standard_normal((3, 7, 256)).astype(np.float32) * 2, O.BF16)
    w = O.cast(1 + 0.3 * rng.standard_normal(256).astype(np.float32), O.BF16)
    norm = MG.Gemma4RMSNorm(256, eps=1e-6).to(torch.bfloat16)
    norm.weight.copy_(_bf(w))
    hf = _np(norm(_bf(x)))
    assert _exact(O.rms_norm(w, x, 1e-6, O.BF16), hf) == 1.0
    bare = MG.Gemma4RMSNorm(256, eps=1e-6, with_scale=False).to(torch.bfloat16)
    assert _exact(O.rms_norm(None, x, 1e-6, O.BF16), _np(bare(_bf(x)))) == 1.0
    # planted: the statistics in bf16 instead of f32 (a missing upcast)
    x16 = O.cast(x, O.BF16)
    ms = O.cast(np.mean(O.cast(np.square(x16), O.BF16), axis=-1, keepdims=True), O.BF16)
    planted = O.cast(O.cast(x16 * O.cast(np.power(ms + np.float32(1e-6), -0.5), O.BF16), O.BF16) * w, O.BF16)
    assert _exact(planted, hf) < 0.9


def test_embedding_scale_equals_hf_bf16():
    rng = np.random.default_rng(3)
    M = 256
    E = O.cast(rng.standard_normal((50, M)).astype(np.float32) * 0.02, O.BF16)
    emb = MG.Gemma4TextScaledWordEmbedding(50, M, 0, embed_scale=M ** 0.5).to(torch.bfloat16)
    emb.weight.copy_(_bf(E))
    emb.embed_scale.copy_(torch.tensor(M ** 0.5))
    ids = rng.integers(0, 50, (2, 9))
    ours = O.cast(E[ids] * O.cast(np.float32(np.sqrt(M)), O.BF16), O.BF16)  # forward_text's embedding
    assert _exact(ours, _np(emb(torch.from_numpy(ids)))) == 1.0


# --- fused elementwise chains -----------------------------------------------------------------


@pytest.mark.parametrize("layer_type", [O.SLIDING, O.FULL])
def test_rope_equals_hf_formula_with_hf_bf16_tables(layer_type):
    """RoPE: HF's rotary module (f32 inverse frequencies, cos/sin cast to the activation dtype, as
    model.py:313-314 casts them) and HF's apply_rotary_pos_emb formula, evaluated in f32 and
    rounded once, equal the oracle's rope (bar the rare element where torch's and numpy's f32
    cos/sin differ in the last bit and the cast rounds differently). A planted oracle that skips
    the cos/sin cast fails."""

    rng = np.random.default_rng(4)
    cfg = H.CFG1
    rot = MG.Gemma4TextRotaryEmbedding(MG.Gemma4TextConfig(**cfg))
    pos = np.tile(np.arange(0, 3000, 97), (2, 1))
    x = O.cast(rng.standard_normal((2, pos.shape[1], 4, 64)).astype(np.float32), O.BF16)
    cos, sin = rot(torch.zeros(1, dtype=torch.bfloat16), torch.from_numpy(pos), layer_type)
    assert cos.dtype == torch.bfloat16
    fused = O.bf16_round(MG.apply_rotary_pos_emb(_bf(x).float(), cos.float(), sin.float(), unsqueeze_dim=2).numpy())
    c32, s32 = O.make_rotary(O.config_from_hf(cfg), pos)[layer_type]
    ours = O.rope(x, c32, s32, O.BF16)
    assert _exact(ours, fused) >= EXACT
    assert (np.abs(ours - fused) <= _spacing(fused)).all()
    half = x.shape[-1] // 2
    rotated = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    shape = x.shape[:2] + (1,) + x.shape[-1:]
    planted = O.bf16_round(x * c32.reshape(shape) + rotated * s32.reshape(shape))  # no cos/sin cast
    assert _exact(planted, fused) < EXACT


def test_gelu_gate_times_up_equals_hf_formula_rounded_once():
    """forward_mlp's activation (model.py:396): HF's gelu_pytorch_tanh times up, in f32, rounded
    once; a planted extra rounding after the gelu fails."""

    rng = np.random.default_rng(5)
    g = O.cast(rng.standard_normal((4, 1000)).astype(np.float32) * 2, O.BF16)
    u = O.cast(rng.standard_normal((4, 1000)).astype(np.float32) * 2, O.BF16)
    act = MG.ACT2FN[MG.Gemma4TextConfig(**H.CFG1).hidden_activation]
    fused = O.bf16_round((act(_bf(g).float()) * _bf(u).float()).numpy())
    ours = O.cast(O.gelu_tanh(g) * u, O.BF16)
    assert _exact(ours, fused) >= 0.99  # tanh implementations differ in the last f32 bits
    assert np.abs(ours - fused).max() <= 1e-5
    planted = O.cast(O.cast(O.gelu_tanh(g), O.BF16) * u, O.BF16)
    assert _exact(planted, fused) < 0.9


def test_softcap_equals_hf_formula_rounded_once():
    """forward_lm_head's soft-cap (model.py:676-680) as lm_head applies it."""

    rng = np.random.default_rng(6)
    x = O.cast(rng.standard_normal((4, 5000)).astype(np.float32) * 20, O.BF16)
    cap = 30.0
    fused = O.bf16_round((torch.tanh(_bf(x).float() / cap) * cap).numpy())
    E = np.eye(5000, dtype=np.float32)[:64]  # lm_head(embed, hidden): hidden @ embed.T, then the cap
    ours = O.lm_head(E, x[:, None, :], cap, O.BF16)[:, 0]
    assert _exact(ours, fused[:, :64]) == 1.0
    planted = O.cast(O.cast(np.tanh(O.cast(x / np.float32(cap), O.BF16)), O.BF16) * np.float32(cap), O.BF16)
    assert _exact(planted, fused) < 0.9
