"""Hugging Face ``Gemma4ForCausalLM`` helpers for pinning the oracle (CPU tests only).

HF transformers' Gemma 4 is the independent implementation the reference itself is tested
against (tests/conftest.py:67-110 and tests/test_model_ops.py of the reference). The weight
layout conversion follows weights.py:54-75 (q head index ``h*R + r``) and its inverse
(weights.py:166-200).
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import g4_oracle as O

ROPE = {
    "sliding_attention": {"rope_type": "default", "rope_theta": 10_000.0},
    "full_attention": {"rope_type": "proportional", "partial_rotary_factor": 0.25, "rope_theta": 1_000_000.0},
}

# The reference's test configs (tests/conftest.py:23-64 of the reference), restated.
TINY_A: dict = dict(
    vocab_size=97, hidden_size=32, intermediate_size=48, num_hidden_layers=6, num_attention_heads=4,
    num_key_value_heads=2, head_dim=8, global_head_dim=16,
    layer_types=["sliding_attention", "full_attention", "sliding_attention", "sliding_attention",
                 "sliding_attention", "full_attention"],
    sliding_window=3, num_kv_shared_layers=2, use_double_wide_mlp=True, hidden_size_per_layer_input=8,
    vocab_size_per_layer_input=97, rms_norm_eps=1e-6, rope_parameters=ROPE, final_logit_softcapping=30.0,
    attention_k_eq_v=False, max_position_embeddings=64, bos_token_id=2, eos_token_id=1, pad_token_id=0,
    tie_word_embeddings=True,
)
TINY_B: dict = {**TINY_A, "num_kv_shared_layers": 0, "use_double_wide_mlp": False, "hidden_size_per_layer_input": 0,
                "attention_k_eq_v": True, "num_global_key_value_heads": 1}

# 4 layers (3 sliding W=16, 1 global), M=256, Hq=4, Hkv=1, D=64, V=1024.
CFG1: dict = dict(
    vocab_size=1024, hidden_size=256, intermediate_size=1024, num_hidden_layers=4, num_attention_heads=4,
    num_key_value_heads=1, head_dim=64, global_head_dim=64,
    layer_types=["sliding_attention", "sliding_attention", "sliding_attention", "full_attention"],
    sliding_window=16, num_kv_shared_layers=0, use_double_wide_mlp=False, hidden_size_per_layer_input=0,
    vocab_size_per_layer_input=1024, rms_norm_eps=1e-6, rope_parameters=ROPE, final_logit_softcapping=30.0,
    attention_k_eq_v=False, max_position_embeddings=128, bos_token_id=2, eos_token_id=1, pad_token_id=0,
    tie_word_embeddings=True,
)


def build_hf_model(kwargs: dict, seed: int = 0, *, weight_std: float = 0.2, norm_std: float = 0.3,
                   layer_scalar_min: float = 0.1):
    """tests/conftest.py:67-87 of the reference: random weights, norms ``1 + 0.3 N``."""

    from transformers import Gemma4ForCausalLM, Gemma4TextConfig

    torch.manual_seed(seed)
    cfg = Gemma4TextConfig(**kwargs)
    cfg._attn_implementation = "eager"
    model = Gemma4ForCausalLM(cfg).eval()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.copy_(1.0 + norm_std * torch.randn_like(p))
            else:
                p.normal_(0.0, weight_std)
        for layer in model.model.layers:
            layer.layer_scalar.copy_(torch.rand(1) * (1.0 - layer_scalar_min) + layer_scalar_min)
    return model


def hf_to_params(model, cfg: O.Config) -> O.Params:
    """weights.py:54-133: HF state dict -> reference-layout params (float32 numpy)."""

    sd = {k: v.detach().float().numpy() for k, v in model.state_dict().items()}

    def g(k):
        return sd["model." + k]

    M, L, P = cfg.hidden_size, cfg.num_hidden_layers, cfg.hidden_size_per_layer_input
    layers = []
    for i in range(L):
        key = f"layers.{i}."
        D, H = O.layer_head_dim(cfg, i), O.layer_kv_heads(cfg, i)
        R = cfg.num_attention_heads // H
        q = g(key + "self_attn.q_proj.weight").T.reshape(M, H, R, D).transpose(0, 2, 1, 3)
        o = g(key + "self_attn.o_proj.weight").T.reshape(H, R, D, M).transpose(1, 0, 2, 3)
        qn = g(key + "self_attn.q_norm.weight")
        if O.is_kv_shared(cfg, i):
            k = v = kn = None
        else:
            k = g(key + "self_attn.k_proj.weight").T.reshape(M, H, D)
            v = g(key + "self_attn.v_proj.weight").T.reshape(M, H, D) if O.layer_has_v_proj(cfg, i) else None
            kn = g(key + "self_attn.k_norm.weight")
        mlp = O.MLPParams(g(key + "mlp.gate_proj.weight").T, g(key + "mlp.up_proj.weight").T,
                          g(key + "mlp.down_proj.weight").T)
        ple = None
        if P:
            ple = O.PLEParams(g(key + "per_layer_input_gate.weight").T, g(key + "per_layer_projection.weight").T,
                              g(key + "post_per_layer_input_norm.weight"))
        layers.append(O.LayerParams(
            g(key + "input_layernorm.weight"), O.AttnParams(q, k, v, o, qn, kn),
            g(key + "post_attention_layernorm.weight"), g(key + "pre_feedforward_layernorm.weight"), mlp,
            g(key + "post_feedforward_layernorm.weight"), ple, np.float32(g(key + "layer_scalar").reshape(()))))
    ple_t = ple_p = ple_n = None
    if P:
        ple_t = g("embed_tokens_per_layer.weight").reshape(-1, L, P)
        ple_p = g("per_layer_model_projection.weight").T.reshape(M, L, P)
        ple_n = g("per_layer_projection_norm.weight")
    return O.Params(np.ascontiguousarray(g("embed_tokens.weight")), ple_t, ple_p, ple_n, tuple(layers),
                    g("norm.weight"))


def params_to_hf(model, params: O.Params, cfg: O.Config) -> None:
    """weights.py:166-200 (inverse conversion): load reference-layout params into an HF model."""

    M, L, P = cfg.hidden_size, cfg.num_hidden_layers, cfg.hidden_size_per_layer_input
    out = {"model.embed_tokens.weight": params.embed_tokens, "model.norm.weight": params.final_norm}
    if P:
        out["model.embed_tokens_per_layer.weight"] = params.embed_tokens_per_layer.reshape(-1, L * P)
        out["model.per_layer_model_projection.weight"] = params.per_layer_model_projection.reshape(M, L * P).T
        out["model.per_layer_projection_norm.weight"] = params.per_layer_projection_norm
    for i, lp in enumerate(params.layers):
        key = f"model.layers.{i}."
        a = lp.attention
        D, H = O.layer_head_dim(cfg, i), O.layer_kv_heads(cfg, i)
        R = cfg.num_attention_heads // H
        out[key + "self_attn.q_proj.weight"] = a.q_proj.transpose(0, 2, 1, 3).reshape(M, H * R * D).T
        out[key + "self_attn.o_proj.weight"] = a.o_proj.transpose(1, 0, 2, 3).reshape(H * R * D, M).T
        out[key + "self_attn.q_norm.weight"] = a.q_norm
        if a.k_proj is not None:
            out[key + "self_attn.k_proj.weight"] = a.k_proj.reshape(M, H * D).T
            out[key + "self_attn.k_norm.weight"] = a.k_norm
        if a.v_proj is not None:
            out[key + "self_attn.v_proj.weight"] = a.v_proj.reshape(M, H * D).T
        out[key + "mlp.gate_proj.weight"] = lp.mlp.gate_proj.T
        out[key + "mlp.up_proj.weight"] = lp.mlp.up_proj.T
        out[key + "mlp.down_proj.weight"] = lp.mlp.down_proj.T
        out[key + "input_layernorm.weight"] = lp.input_norm
        out[key + "post_attention_layernorm.weight"] = lp.post_attention_norm
        out[key + "pre_feedforward_layernorm.weight"] = lp.pre_feedforward_norm
        out[key + "post_feedforward_layernorm.weight"] = lp.post_feedforward_norm
        out[key + "layer_scalar"] = np.asarray([lp.layer_scalar], np.float32)
        if lp.per_layer_input is not None:
            out[key + "per_layer_input_gate.weight"] = lp.per_layer_input.gate.T
            out[key + "per_layer_projection.weight"] = lp.per_layer_input.projection.T
            out[key + "post_per_layer_input_norm.weight"] = lp.per_layer_input.post_norm
    sd = model.state_dict()
    with torch.no_grad():
        for k, v in out.items():
            t = sd[k]
            t.copy_(torch.from_numpy(np.ascontiguousarray(v, np.float32)).reshape(t.shape))
    if "lm_head.weight" in sd and sd["lm_head.weight"].data_ptr() != sd["model.embed_tokens.weight"].data_ptr():
        with torch.no_grad():
            sd["lm_head.weight"].copy_(sd["model.embed_tokens.weight"])


def hf_logits(model, ids: np.ndarray, mask: np.ndarray | None = None, pos: np.ndarray | None = None) -> np.ndarray:
    with torch.no_grad():
        kw = {}
        if mask is not None:
            kw["attention_mask"] = torch.from_numpy(mask.astype(np.int64))
        if pos is not None:
            kw["position_ids"] = torch.from_numpy(pos.astype(np.int64))
        return model(input_ids=torch.from_numpy(ids.astype(np.int64)), **kw).logits.float().numpy()
