"""Decode attention with the fused preparation (G4DecodePrep): the raw q/k/v projection rows in,
g4_kv_append's norms, RoPE and cache append done inside the two-launch attention. The output and
the cache must equal, bit for bit, g4_kv_append (or the q-only preparation of a kv-shared layer)
followed by the same two-launch attention on the prepared rows."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gemma4_posttrain_jax_amd import _lib, kernels
from gemma4_posttrain_jax_amd.kvcache import new_layer_cache
from gemma4_posttrain_jax_amd.model import rotary_tables

pytestmark = pytest.mark.gpu

FLAGS_Q = _lib.G4_APPEND_NORM_Q | _lib.G4_APPEND_ROPE_Q
FLAGS_KV = _lib.G4_APPEND_NORM_K | _lib.G4_APPEND_ROPE_K | _lib.G4_APPEND_NORM_V


@pytest.mark.parametrize("B,D,ring,cap,shared", [(8, 256, True, 512, False), (8, 256, False, 768, False),
                                                 (256, 256, True, 512, False), (8, 256, True, 512, True),
                                                 (6, 128, False, 300, False)])
def test_decode_fused_prep_matches_append_then_attention(device, B, D, ring, cap, shared):
    H, R = 2, 4
    W = 512 if ring else 0
    g = torch.Generator(device="cuda").manual_seed(B + cap + shared)
    rng = np.random.default_rng(B + cap)
    qkv = torch.randn((B, 1, (H * R + 2 * H) * D), device="cuda", generator=g).to(torch.bfloat16)
    q = qkv[..., :H * R * D].view(B, 1, H, R, D)
    k = qkv[..., H * R * D:(H * R + H) * D].view(B, 1, H, D)
    v = qkv[..., (H * R + H) * D:].view(B, 1, H, D)
    layer = new_layer_cache(B, H, D, cap, ring, torch.bfloat16, device)
    layer.key.normal_(generator=g)
    layer.value_t.normal_(generator=g)
    ref_layer = new_layer_cache(B, H, D, cap, ring, torch.bfloat16, device)
    ref_layer.key.copy_(layer.key)
    ref_layer.value_t.copy_(layer.value_t)
    q_pos_np = rng.integers(cap, 3 * cap, B) if ring else rng.integers(0, cap, B)
    q_pos = torch.from_numpy(q_pos_np.astype(np.int32)).to(device)
    km = torch.ones((B, max(cap, int(q_pos_np.max()) + 1)), dtype=torch.bool, device=device)
    km[0, : int(q_pos_np[0]) // 2] = False  # a left-padded row
    qn = (1 + 0.1 * torch.randn(D, device="cuda", generator=g)).to(torch.bfloat16)
    kn = (1 + 0.1 * torch.randn(D, device="cuda", generator=g)).to(torch.bfloat16)
    inv = (1.0 / (10000.0 ** (torch.arange(0, D, 2, device="cuda", dtype=torch.float32) / D))).contiguous()
    cos, sin = rotary_tables(inv, q_pos[:, None])  # [B, 1, D]

    q_out = torch.empty((B, 1, H, R, D), dtype=torch.bfloat16, device=device)
    if shared:
        kernels.prepare_q(q, q_out, flags=FLAGS_Q, eps=1e-6, q_norm_weight=qn, rope_cos=cos, rope_sin=sin)
    else:
        kernels.kv_append(ref_layer, k, v, write_pos=q_pos, flags=FLAGS_Q | FLAGS_KV, eps=1e-6, q=q, q_out=q_out,
                          q_norm_weight=qn, k_norm_weight=kn, rope_cos=cos, rope_sin=sin)
    want = kernels.decode_attention(ref_layer, q_out.view(B, H, R, D), km, q_pos=q_pos, window=W,
                                    num_splits=_lib.G4_DECODE_TWO_PASS)
    got = kernels.decode_attention_fused(
        layer, q[:, 0], km, q_pos=q_pos, window=W, k_raw=None if shared else k[:, 0], v_raw=None if shared else v[:, 0],
        q_norm_weight=qn, k_norm_weight=kn, rope_cos=cos[:, 0].contiguous(), rope_sin=sin[:, 0].contiguous(), eps=1e-6,
        flags=FLAGS_Q | (0 if shared else FLAGS_KV))
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(layer.key.view(torch.int16), ref_layer.key.view(torch.int16))
    assert torch.equal(layer.value_t.view(torch.int16), ref_layer.value_t.view(torch.int16))


PREP_CFG = dict(
    vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=5, num_attention_heads=8,
    num_key_value_heads=2, head_dim=128, global_head_dim=128,
    layer_types=["sliding_attention", "sliding_attention", "full_attention", "sliding_attention", "full_attention"],
    sliding_window=16, num_kv_shared_layers=2, hidden_size_per_layer_input=0, final_logit_softcapping=30.0,
)


def test_graphed_decode_with_fused_preparation_matches_unfused(device, monkeypatch):
    """The model's graphed decode step at 256 (b, kv head) pairs takes the fused preparation (own
    and kv-shared layers, a wrapping ring, a finished row, a left-padded row): its logits and caches
    equal, bit for bit, the same step with g4_kv_append run separately."""

    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
    from oracle import g4_oracle as O

    from gemma4_posttrain_jax_amd import config as C
    from gemma4_posttrain_jax_amd import model as M
    from gemma4_posttrain_jax_amd import sampler as SMP

    ocfg = O.config_from_hf(PREP_CFG)
    oparams = O.init_params(ocfg, seed=5, dtype=O.BF16, std=0.03, norm_std=0.05, layer_scalar_min=0.8)
    cfg = C.config_from_hf(PREP_CFG)
    params = M.params_from_numpy(oparams, cfg, dtype=torch.bfloat16, device=device)
    B = 128
    rng = np.random.default_rng(13)
    ids = torch.from_numpy(rng.integers(3, 512, (B, 12)).astype(np.int32)).to(device)
    mask = torch.ones_like(ids, dtype=torch.bool)
    mask[1, :5] = False
    runs = []
    for fused in (True, False):
        if not fused:
            monkeypatch.setattr(M, "_fused_decode_prep", lambda *args: False)
        out = SMP.prefill(params, cfg, ids, mask, max_new_tokens=10)
        engine = SMP.GraphedDecodeStep(params, cfg, out.kv_cache)
        pos0 = mask.sum(-1, dtype=torch.int32)
        tok = out.logits[:, -1].argmax(-1).to(torch.int32)
        seen = []
        for step in range(9):  # 12 prompt slots + 9 steps: the 16-slot ring wraps
            active = torch.ones(B, dtype=torch.bool, device=device)
            active[2] = step < 3
            logits = engine.step(tok, pos0 + step, active).clone()
            seen.append(logits)
            tok = logits.argmax(-1).to(torch.int32)
        runs.append((seen, engine.kv_cache))
    (la, ca), (lb, cb) = runs
    for step, (x, y) in enumerate(zip(la, lb)):
        assert torch.equal(x, y), f"step {step}: max diff {(x - y).abs().max().item()}"
    for i, (x, y) in enumerate(zip(ca.layers, cb.layers)):
        if x is not None:
            assert torch.equal(x.key, y.key) and torch.equal(x.value_t, y.value_t), f"layer {i}"
