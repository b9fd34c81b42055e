"""torch-CPU restatement of the reference's decode step, for the timed CPU baseline.

TEST INFRASTRUCTURE ONLY: used by ``bench.py``'s ``cpu_baseline`` legs (and checked against the
numpy oracle by tests/test_oracle_torch_cpu.py), never by the GPU library.

The reference's JAX path cannot run here (no JAX), so the CPU baseline is this restatement of
gemma4_posttrain_jax/model.py + sampler.py in torch on the host cores, with the reference's
costs: bf16 tensors and bf16 matmuls (f32 accumulation), dense masked attention over the whole
cache capacity with full score tensors (model.py:496-499), f32 softmax, the per-layer op order of
forward_decoder_layer (model.py:505-554), the full-vocab f32 log-softmax of _sample_token
(sampler.py:151-159). Elementwise chains round after every torch op (torch's bf16 semantics; the
numpy oracle rounds once per XLA-fused line), which changes no cost. The caches are held
head-major, ``[B, H, C, D]``, so both attention products read them in place (the key operand as a
transposed view): no per-layer copy of a cache, which makes the baseline faster, not slower.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import g4_oracle as O

BF16 = torch.bfloat16


def _t(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(BF16)


class TorchCPUModel:
    """The oracle's parameter pytree (float32 numpy holding bf16 values) as bf16 CPU tensors."""

    def __init__(self, params: O.Params, cfg: O.Config):
        if cfg.hidden_size_per_layer_input:
            raise ValueError("the CPU baseline covers configs without per-layer inputs")
        self.cfg = cfg
        self.embed = _t(params.embed_tokens)
        self.final_norm = _t(params.final_norm)
        self.layers = []
        for lp in params.layers:
            a = lp.attention
            self.layers.append(dict(
                input_norm=_t(lp.input_norm), q=_t(a.q_proj), k=_t(a.k_proj), v=_t(a.v_proj), o=_t(a.o_proj),
                q_norm=_t(a.q_norm), k_norm=_t(a.k_norm), post_attn=_t(lp.post_attention_norm),
                pre_ff=_t(lp.pre_feedforward_norm), gate=_t(lp.mlp.gate_proj), up=_t(lp.mlp.up_proj),
                down=_t(lp.mlp.down_proj), post_ff=_t(lp.post_feedforward_norm),
                scalar=torch.tensor(float(np.asarray(lp.layer_scalar).reshape(-1)[0]), dtype=BF16)))
        inv = O.rope_inv_freq(cfg)
        self.inv_freq = {k: torch.from_numpy(v) for k, v in inv.items()}

    def init_cache(self, batch: int, capacity: int):
        """model.py:557-568: bf16 key / value per non-shared layer, head-major [B, H, C_i, D]."""

        cfg, layers = self.cfg, []
        for i in range(cfg.num_hidden_layers):
            if O.is_kv_shared(cfg, i):
                layers.append(None)
                continue
            c = min(cfg.sliding_window, capacity) if cfg.layer_types[i] == O.SLIDING else capacity
            shape = (batch, O.layer_kv_heads(cfg, i), c, O.layer_head_dim(cfg, i))
            layers.append([torch.zeros(shape, dtype=BF16), torch.zeros(shape, dtype=BF16)])
        return dict(layers=layers, key_mask=torch.zeros((batch, capacity), dtype=torch.bool), length=0)


def _rms(x, w, eps):
    """model.py:278-285."""

    x32 = x.float()
    y = x32 * torch.pow(x32.square().mean(-1, keepdim=True) + eps, -0.5)
    if w is not None:
        y = y * w.float()
    return y.to(x.dtype)


def _rope(x, cos, sin):
    """model.py:309-317: cos / sin cast to the activation dtype first; x [B, S, ..., D]."""

    shape = x.shape[:2] + (1,) * (x.dim() - 3) + x.shape[-1:]
    c, s = cos.reshape(shape).to(x.dtype), sin.reshape(shape).to(x.dtype)
    half = x.shape[-1] // 2
    return x * c + torch.cat([-x[..., half:], x[..., :half]], -1) * s


def decode_step(model: TorchCPUModel, tokens: torch.Tensor, positions: torch.Tensor, cache: dict,
                attention_mask: torch.Tensor | None = None) -> tuple[torch.Tensor, dict]:
    """sampler.py:109-142 -> model.py:571-709 in append mode for one token per row, then the f32
    log-softmax of the full vocabulary (sampler.py:151-159). Returns (f32 log-probabilities [B, V],
    the cache, updated in place as XLA does inside the reference's while_loop)."""

    cfg = model.cfg
    B = tokens.shape[0]
    eps = cfg.rms_norm_eps
    if attention_mask is None:
        attention_mask = torch.ones(B, dtype=torch.bool)
    length = cache["length"]
    x = model.embed[tokens.long()][:, None]  # [B, 1, M]
    x = x * torch.tensor(math.sqrt(cfg.hidden_size), dtype=BF16)
    key_mask = cache["key_mask"]
    key_mask[:, length] = attention_mask
    C = key_mask.shape[1]
    # make_cached_qk_masks (model.py:338-365) for the one query at position `length`
    full_mask = key_mask & (torch.arange(C)[None, :] <= length)
    rots = {}
    for lt in (O.SLIDING, O.FULL):
        f = positions.float()[:, None, None] * model.inv_freq[lt][None, None, :]
        emb = torch.cat([f, f], -1)
        rots[lt] = (torch.cos(emb), torch.sin(emb))
    masks = {O.FULL: full_mask}
    wc = min(cfg.sliding_window, C)
    slots = torch.arange(wc)
    pos = slots + torch.div(length - slots, wc, rounding_mode="floor") * wc
    valid = (pos >= 0) & (pos <= length) & (pos > length - cfg.sliding_window)
    masks[O.SLIDING] = valid[None, :] & key_mask[:, pos.clamp(0, C - 1)]
    fill = torch.finfo(BF16).min
    shared: dict = {}
    for i, lp in enumerate(model.layers):
        lt = cfg.layer_types[i]
        residual = x
        h = _rms(x, lp["input_norm"], eps)
        M_, R, H, D = lp["q"].shape
        q = (h.reshape(B, M_) @ lp["q"].reshape(M_, R * H * D)).reshape(B, 1, R, H, D)
        q = _rope(_rms(q, lp["q_norm"], eps), *rots[lt])
        if O.is_kv_shared(cfg, i):
            kc, vc = shared[lt]
        else:
            k = (h.reshape(B, M_) @ lp["k"].reshape(M_, H * D)).reshape(B, 1, H, D)
            v = (h.reshape(B, M_) @ lp["v"].reshape(M_, H * D)).reshape(B, 1, H, D) if lp["v"] is not None else k
            k = _rope(_rms(k, lp["k_norm"], eps), *rots[lt])
            v = _rms(v, None, eps)
            kc, vc = cache["layers"][i]
            slot = length % kc.shape[2] if lt == O.SLIDING else length
            kc[:, :, slot] = k[:, 0]
            vc[:, :, slot] = v[:, 0]
            shared[lt] = (kc, vc)
        # dense attention over the whole capacity (model.py:496-499)
        qh = q[:, 0].permute(0, 2, 1, 3)  # [B, H, R, D]
        scores = qh @ kc.transpose(-1, -2)  # [B, H, R, T]
        scores = torch.where(masks[lt][:, None, None, :], scores, torch.full_like(scores, fill))
        probs = torch.softmax(scores.float(), -1).to(BF16)
        attn = probs @ vc  # [B, H, R, D]
        attn = attn.permute(0, 2, 1, 3).reshape(B, R * H * D)
        o = (attn @ lp["o"].reshape(R * H * D, M_)).reshape(B, 1, M_)
        x = residual + _rms(o, lp["post_attn"], eps)
        residual = x
        h = _rms(x, lp["pre_ff"], eps).reshape(B, M_)
        act = torch.nn.functional.gelu(h @ lp["gate"], approximate="tanh") * (h @ lp["up"])
        x = residual + _rms((act @ lp["down"]).reshape(B, 1, M_), lp["post_ff"], eps)
        x = x * lp["scalar"]
    hidden = _rms(x, model.final_norm, eps)
    logits = hidden.reshape(B, -1) @ model.embed.t()
    cap = cfg.final_logit_softcapping
    if cap is not None:
        logits = torch.tanh(logits / cap) * cap
    logits32 = logits.float()
    shifted = logits32 - logits32.max(-1, keepdim=True).values
    logp = shifted - torch.log(torch.exp(shifted).sum(-1, keepdim=True))
    cache["length"] = length + 1
    return logp, cache


def ring_decode_attention(q: torch.Tensor, cache_k: torch.Tensor, cache_v: torch.Tensor, new_k: torch.Tensor,
                          new_v: torch.Tensor, q_pos: torch.Tensor, key_mask: torch.Tensor,
                          window: int) -> torch.Tensor:
    """One sliding-window layer's decode attention with its append (model.py:338-390, 496-499), per
    row b at position q_pos[b]: K/V stored at ring slot q_pos mod Wc, then dense masked attention
    over every ring slot. q [B, R, H, D], caches head-major [B, H, Wc, D] (updated in place), new_k /
    new_v [B, H, D], key_mask [B, C] over absolute positions. Returns [B, R, H, D]."""

    B, Wc = cache_k.shape[0], cache_k.shape[2]
    rows = torch.arange(B)
    slot = q_pos.long() % Wc
    cache_k[rows, :, slot] = new_k
    cache_v[rows, :, slot] = new_v
    slots = torch.arange(Wc)[None, :]
    qp = q_pos.long()[:, None]
    pos = slots + torch.div(qp - slots, Wc, rounding_mode="floor") * Wc  # [B, Wc]
    valid = (pos >= 0) & (pos <= qp) & (pos > qp - window)
    valid &= torch.gather(key_mask, 1, pos.clamp(0, key_mask.shape[1] - 1))
    scores = q.permute(0, 2, 1, 3) @ cache_k.transpose(-1, -2)  # [B, H, R, Wc]
    scores = torch.where(valid[:, None, None, :], scores, torch.full_like(scores, torch.finfo(BF16).min))
    probs = torch.softmax(scores.float(), -1).to(BF16)
    return (probs @ cache_v).permute(0, 2, 1, 3)
