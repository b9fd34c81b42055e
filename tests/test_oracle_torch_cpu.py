"""The torch-CPU restatement that bench.py times as the CPU baseline computes the oracle's decode
step (oracle/torch_cpu.py against oracle/g4_oracle.py, bf16, CPU)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import g4_oracle as O
from oracle import torch_cpu as T

CFG = dict(
    vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=5, num_attention_heads=8,
    num_key_value_heads=2, head_dim=64, global_head_dim=64,
    layer_types=["sliding_attention", "sliding_attention", "full_attention", "sliding_attention", "full_attention"],
    sliding_window=8, num_kv_shared_layers=2, hidden_size_per_layer_input=0, final_logit_softcapping=30.0,
)


def test_torch_cpu_decode_steps_track_the_oracle():
    """Prefill by the oracle, then five decode steps (the ring wraps) by both: the log-probabilities
    agree to the bf16 level (torch rounds elementwise chains per op, the oracle per fused line) and
    the caches hold the same K/V."""

    torch.set_grad_enabled(False)
    cfg = O.config_from_hf(CFG)
    params = O.init_params(cfg, seed=2, dtype=O.BF16, std=0.02, norm_std=0.05, qk_norm_scale=0.25)
    rng = np.random.default_rng(3)
    B, P, N = 3, 6, 6
    ids = rng.integers(3, 512, (B, P)).astype(np.int32)
    logits, _, rc = O.prefill(params, cfg, ids, np.ones((B, P), bool), max_new_tokens=N, dtype=O.BF16)
    model = T.TorchCPUModel(params, cfg)
    cache = model.init_cache(B, P + N)
    for i, layer in enumerate(rc.layers):
        if layer is not None:
            cache["layers"][i][0].copy_(torch.from_numpy(layer.key).transpose(1, 2))
            cache["layers"][i][1].copy_(torch.from_numpy(layer.value).transpose(1, 2))
    cache["key_mask"].copy_(torch.from_numpy(rc.key_mask))
    cache["length"] = rc.length
    tok = logits[:, -1].argmax(-1).astype(np.int32)
    for step in range(N - 1):
        pos = np.full(B, P + step, np.int32)
        ref, _, rc = O.decode_step(params, cfg, tok, pos, rc, dtype=O.BF16)
        logp, cache = T.decode_step(model, torch.from_numpy(tok), torch.from_numpy(pos), cache)
        want = O.log_softmax_f32(ref[:, -1])
        assert np.abs(logp.numpy() - want).max() < 0.05, f"step {step}"
        tok = ref[:, -1].argmax(-1).astype(np.int32)
    for i, layer in enumerate(rc.layers):
        if layer is not None:
            np.testing.assert_allclose(cache["layers"][i][0].transpose(1, 2).float().numpy(), layer.key, atol=0.05,
                                       rtol=0)
            np.testing.assert_allclose(cache["layers"][i][1].transpose(1, 2).float().numpy(), layer.value, atol=0.05,
                                       rtol=0)
    assert cache["length"] == rc.length


def test_torch_cpu_ring_decode_attention_equals_the_oracle():
    """The config-2 CPU baseline step (append + dense attention over the ring) against the oracle:
    wrapped ring, a left-padded row, a row whose ring has not filled."""

    rng = np.random.default_rng(0)
    B, W, H, R, D = 4, 16, 2, 4, 64
    k = O.cast(rng.standard_normal((B, W, H, D)).astype(np.float32), O.BF16)
    v = O.cast(rng.standard_normal((B, W, H, D)).astype(np.float32), O.BF16)
    q = O.cast(rng.standard_normal((B, 1, R, H, D)).astype(np.float32), O.BF16)
    nk = O.cast(rng.standard_normal((B, 1, H, D)).astype(np.float32), O.BF16)
    nv = O.cast(rng.standard_normal((B, 1, H, D)).astype(np.float32), O.BF16)
    pos = np.array([3, 20, 40, 33])
    km = np.ones((B, 64), bool)
    km[1, :5] = False
    layer = O.update_layer_cache(O.LayerKV(k.copy(), v.copy()), nk, nv, pos, True, O.BF16)
    mask = O.make_cached_qk_masks(km, W, pos, 1)[O.SLIDING]
    ref = O.attention_core(q, layer.key, layer.value, mask, O.BF16)[:, 0]

    def t(a):
        return torch.from_numpy(a).to(torch.bfloat16)

    ck, cv = t(k).transpose(1, 2).contiguous(), t(v).transpose(1, 2).contiguous()  # head-major
    got = T.ring_decode_attention(t(q[:, 0]), ck, cv, t(nk[:, 0]), t(nv[:, 0]),
                                  torch.from_numpy(pos.astype(np.int32)), torch.from_numpy(km), W)
    assert np.abs(got.float().numpy() - ref).max() <= 2e-2
    np.testing.assert_array_equal(ck.transpose(1, 2).float().numpy(), layer.key)
    np.testing.assert_array_equal(cv.transpose(1, 2).float().numpy(), layer.value)
