"""Gemma 4 text decoder forward on MI355X: the drop-in for gemma4_posttrain_jax/model.py's
generation path (``init_kv_cache``, ``forward_gemma4_text``, ``forward_gemma4_lm``).

Parameters use the reference's pytree (``Gemma4TextParams`` and friends, model.py:193-235) with
torch device tensors. On first use each params object is packed once into the kernel-friendly
layout (``PackedWeights``): q/k/v projections fused into one ``[M, (H*R + 2H)*D]`` matrix with
query columns in (kv head, r) order, o_proj rows in the same order, gate|up fused; the MLP
matrices are stored output-major (``[N, K]``), which hipBLASLt runs faster at decode batch sizes. Per layer the
forward runs one hipBLASLt GEMM for q/k/v, the native ``g4_kv_append`` (q/k norms, RoPE, v norm,
cache append), the native prefill or decode attention kernel, and GEMMs for o_proj and the MLP.
The norm / residual / activation glue runs as three fused native kernels per layer with the
reference's f32 rounding points: ``g4_residual_norm`` (post-attention norm + residual + pre-MLP
norm, and post-MLP norm + residual + layer scalar + the next layer's input norm) and
``g4_gelu_mul``; the per-layer-input branch of configs that have one uses PyTorch-ROCm ops.
"""

from __future__ import annotations

import math
from typing import Literal, NamedTuple

import numpy as np
import torch

from . import _lib, kernels
from .config import (
    FULL,
    SLIDING,
    Gemma4TextConfig,
    is_kv_shared,
    kv_source_layers,
    layer_has_v_proj,
    layer_head_dim,
    layer_intermediate_size,
    layer_kv_heads,
)
from .kvcache import KVCache, LayerKVCache, init_kv_cache, key_shape, slot_stride_for

# --- parameter pytree (model.py:193-235) -----------------------------------------------------------


class RMSNormParams(NamedTuple):
    weight: torch.Tensor  # [dim]


class AttentionParams(NamedTuple):
    q_proj: torch.Tensor  # [M, R, H, D]
    k_proj: torch.Tensor | None  # [M, H, D]
    v_proj: torch.Tensor | None  # [M, H, D]
    o_proj: torch.Tensor  # [R, H, D, M]
    q_norm: RMSNormParams
    k_norm: RMSNormParams | None


class MLPParams(NamedTuple):
    gate_proj: torch.Tensor  # [M, F]
    up_proj: torch.Tensor  # [M, F]
    down_proj: torch.Tensor  # [F, M]


class PerLayerInputParams(NamedTuple):
    gate: torch.Tensor  # [M, P]
    projection: torch.Tensor  # [P, M]
    post_norm: RMSNormParams


class DecoderLayerParams(NamedTuple):
    input_norm: RMSNormParams
    attention: AttentionParams
    post_attention_norm: RMSNormParams
    pre_feedforward_norm: RMSNormParams
    mlp: MLPParams
    post_feedforward_norm: RMSNormParams
    per_layer_input: PerLayerInputParams | None
    layer_scalar: torch.Tensor  # []


class Gemma4TextParams(NamedTuple):
    embed_tokens: torch.Tensor  # [V, M]
    embed_tokens_per_layer: torch.Tensor | None  # [Vp, L, P]
    per_layer_model_projection: torch.Tensor | None  # [M, L, P]
    per_layer_projection_norm: RMSNormParams | None
    layers: tuple
    final_norm: RMSNormParams


class Gemma4Output(NamedTuple):
    logits: torch.Tensor  # [B, S', V]
    hidden: torch.Tensor  # [B, S, M]
    kv_cache: KVCache | None


def params_from_numpy(p, config: Gemma4TextConfig, *, dtype=torch.bfloat16, device="cuda") -> Gemma4TextParams:
    """Build device params from an object with the reference's field names holding numpy arrays
    (plain arrays for norm weights)."""

    def t(x):
        return None if x is None else torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dtype).to(device)

    def n(x):
        return None if x is None else RMSNormParams(t(x))

    layers = []
    for lp in p.layers:
        a = lp.attention
        ple = None
        if lp.per_layer_input is not None:
            ple = PerLayerInputParams(t(lp.per_layer_input.gate), t(lp.per_layer_input.projection),
                                      n(lp.per_layer_input.post_norm))
        layers.append(DecoderLayerParams(
            n(lp.input_norm), AttentionParams(t(a.q_proj), t(a.k_proj), t(a.v_proj), t(a.o_proj), n(a.q_norm),
                                              n(a.k_norm)),
            n(lp.post_attention_norm), n(lp.pre_feedforward_norm),
            MLPParams(t(lp.mlp.gate_proj), t(lp.mlp.up_proj), t(lp.mlp.down_proj)), n(lp.post_feedforward_norm), ple,
            t(np.asarray(lp.layer_scalar, np.float32)).reshape(())))
    return Gemma4TextParams(t(p.embed_tokens), t(p.embed_tokens_per_layer), t(p.per_layer_model_projection),
                            n(p.per_layer_projection_norm), tuple(layers), n(p.final_norm))


# --- packed device weights ---------------------------------------------------------------------------


class PackedLayer(NamedTuple):
    # every projection in the [N, K] (output-row-major) layout of g4_linear_bf16
    w_qkv_t: torch.Tensor  # [(H*R [+ H [+ H]])*D, M]: q rows in (h, r) order, then k, then v
    w_o_t: torch.Tensor  # [M, H*R*D], columns in (h, r, d) order
    w_gate_up_t: torch.Tensor  # [2F, M]: gate rows then up rows (output-major: a faster GEMM at small M)
    w_down_t: torch.Tensor  # [M, F]
    heads: int
    group: int
    head_dim: int
    has_k: bool
    has_v: bool
    scalar_f32: torch.Tensor  # [1] f32 layer_scalar (model.py:553)


class PackedWeights(NamedTuple):
    layers: tuple
    embed_scale: torch.Tensor  # bf16/f32 scalar sqrt(M) rounded to the param dtype (model.py:600)
    inv_freq: dict  # layer type -> f32 [D/2] device tensor (model.py:294-302)
    embed_scale_f: float  # the same rounded scale as a host float (no device read inside a graph)


_PACKED_BY_ID: dict = {}


def _rope_inv_freq(config: Gemma4TextConfig) -> dict:
    """model.py:294-302 in numpy float32 (host-side configuration constants)."""

    dim = config.head_dim
    inv_s = (np.float32(1.0) / np.power(np.float32(config.rope_theta_sliding),
                                        np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim))).astype(np.float32)
    dim = config.global_head_dim
    angles = int(config.full_partial_rotary_factor * dim // 2)
    inv_r = (np.float32(1.0) / np.power(np.float32(config.rope_theta_full),
                                        np.arange(0, 2 * angles, 2, dtype=np.float32) / np.float32(dim))).astype(np.float32)
    inv_f = np.concatenate([inv_r, np.zeros(dim // 2 - angles, np.float32)])
    return {SLIDING: inv_s, FULL: inv_f}


def _tensor_versions(tree) -> tuple:
    """The version counters of every tensor in a params pytree (torch bumps a tensor's counter on
    each in-place write: ``copy_``, ``mul_``, optimizer steps)."""

    if isinstance(tree, torch.Tensor):
        return (tree._version,)
    if isinstance(tree, (tuple, list)):
        return sum((_tensor_versions(x) for x in tree), ())
    return ()


def pack_weights(params: Gemma4TextParams, config: Gemma4TextConfig) -> PackedWeights:
    """Fuse and reorder the projection weights once per params object (cached).

    The packed copy is rebuilt when ``params`` is another object or when any of its tensors was
    written in place since the packing (their version counters moved), so an in-place weight
    update is never served stale weights. Writes that bypass the counters (through ``.data`` or
    another framework's view of the memory) are not seen: pass a new params object after those."""

    key = id(params)
    versions = _tensor_versions(params)
    hit = _PACKED_BY_ID.get(key)
    if hit is not None and hit[0] is params and hit[2] == versions:
        return hit[1]
    layers = []
    for i, lp in enumerate(params.layers):
        a = lp.attention
        M, R, H, D = a.q_proj.shape
        wq = a.q_proj.permute(0, 2, 1, 3).reshape(M, H * R * D)
        parts = [wq]
        has_k = a.k_proj is not None
        has_v = a.v_proj is not None
        if has_k:
            parts.append(a.k_proj.reshape(M, H * D))
        if has_v:
            parts.append(a.v_proj.reshape(M, H * D))
        w_qkv_t = torch.cat(parts, dim=1).t().contiguous()
        w_o_t = a.o_proj.permute(1, 0, 2, 3).reshape(H * R * D, M).t().contiguous()
        w_gu_t = torch.cat([lp.mlp.gate_proj, lp.mlp.up_proj], dim=1).t().contiguous()
        layers.append(PackedLayer(w_qkv_t, w_o_t, w_gu_t, lp.mlp.down_proj.t().contiguous(), H, R, D, has_k, has_v,
                                  lp.layer_scalar.float().reshape(1).contiguous()))
    dev = params.embed_tokens.device
    dt = params.embed_tokens.dtype
    inv = {k: torch.from_numpy(v).to(dev) for k, v in _rope_inv_freq(config).items()}
    scale = torch.tensor(math.sqrt(config.hidden_size), dtype=dt)
    packed = PackedWeights(tuple(layers), scale.to(dev), inv, float(scale.float()))
    _PACKED_BY_ID.clear()  # one live params object at a time (rollout reuses the same weights)
    _PACKED_BY_ID[key] = (params, packed, versions)
    return packed


# K splits of the decode-batch down projection (measured best at M=256, N=2048, K=8192: 8 splits,
# 256 workgroups; hipBLASLt's tile re-reads each weight block once per 32-row tile)
DOWN_KSPLIT = 8


def _split_down(act: torch.Tensor, w_t: torch.Tensor) -> bool:
    """Whether the down projection runs as g4_linear_bf16 split-K partials fed to the residual norm:
    a bf16 decode batch of at most 256 rows and shapes the kernels take."""

    n, k = w_t.shape
    return (act.dtype == torch.bfloat16 and act.shape[0] <= 256 and n % 64 == 0 and n % 8 == 0 and n <= 4096
            and k % (64 * DOWN_KSPLIT) == 0 and act.is_contiguous() and w_t.is_contiguous())


def _fused_decode_prep(x: torch.Tensor, pairs: int, head_dim: int, cache) -> bool:
    """Whether a decode layer's q/k/v preparation and append run inside the two-launch attention
    (G4DecodePrep): the path the library takes at the rollout batch (>= 256 (b, kv head) pairs,
    rows of at most 1024 slots, head dims 128 / 256 / 512, bf16)."""

    return (x.dtype == torch.bfloat16 and pairs >= 256 and head_dim in (128, 256, 512) and cache is not None
            and cache.capacity <= 1024)


def _native_gate_up(h: torch.Tensor, w_t: torch.Tensor) -> bool:
    """Whether the gate/up projection + gated GELU run as one g4_linear_bf16 launch (its
    gated-GELU epilogue): a bf16 decode batch of at most 256 rows and shapes the kernel takes."""

    n, k = w_t.shape
    rows = h.numel() // h.shape[-1]
    return (h.dtype == torch.bfloat16 and rows <= 256 and n % 64 == 0 and k % 64 == 0 and h.is_contiguous()
            and w_t.is_contiguous())


def _mm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a @ b`` in a's dtype. bf16: hipBLASLt, f32 accumulation, one rounding. f32 (the parity
    configs): the product accumulates in f64 and rounds once to f32, i.e. the exactly rounded dot
    products up to one f64 rounding. Two f32 accumulation orders disagree by more than the 1e-5
    fp32 bar at the model level (BASELINE config 1's logits: the oracle's f32 matmuls against its
    f64-accumulated ones 2.7e-5, HF's torch-CPU f32 against the latter 4.1e-5); the exactly rounded
    product is the one every order approximates."""

    if a.dtype == torch.float32:
        return (a.double() @ b.double()).float()
    return a @ b


def _proj(x: torch.Tensor, w_t: torch.Tensor) -> torch.Tensor:
    """``x [T, K] . w_t[N, K]^T`` in x's dtype (hipBLASLt; the [N, K] weight layout is its faster
    one for the prefill shapes and equal at decode)."""

    return _mm(x, w_t.t())


# --- elementwise glue (PyTorch-ROCm ops, reference rounding points) ----------------------------------


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """model.py:278-285: f32 ``x * (mean(x^2) + eps)^-0.5 * w``, cast back to x's dtype. f32 x: each
    f32 operation rounded once, the sum of the squares and x^-0.5 evaluated in f64 (the native
    norms' f32 path)."""

    x32 = x.float()
    if x.dtype == torch.float32:
        ms = (x32 * x32).double().sum(-1, keepdim=True).float() / x.shape[-1]
        y = x32 * (1.0 / (ms + eps).double().sqrt()).float()
        return y * weight.float() if weight is not None else y
    y = x32 * torch.pow(x32.square().mean(-1, keepdim=True) + eps, -0.5)
    if weight is not None:
        y = y * weight.float()
    return y.to(x.dtype)


def gelu_tanh_f32(x: torch.Tensor, exact: bool = False) -> torch.Tensor:
    """jax.nn.gelu(approximate=True) in f32. ``exact``: its own op order,
    ``x * (0.5 * (1 + tanh(c * (x + 0.044715 * ((x * x) * x)))))``, each op rounded to f32 and tanh
    evaluated in f64 (the fp32 parity configs)."""

    x = x.float()
    if exact:
        inner = math.sqrt(2.0 / math.pi) * (x + 0.044715 * ((x * x) * x))
        return x * (0.5 * (1.0 + torch.tanh(inner.double()).float()))
    return torch.nn.functional.gelu(x, approximate="tanh")


def rotary_tables(inv_freq: torch.Tensor, position_ids: torch.Tensor,
                  exact: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """model.py:288-291: f32 cos/sin ``[B, S, D]`` of ``concat(f, f)``, f = pos * inv_freq
    (``exact``: cos / sin evaluated in f64 and rounded once, for f32 models)."""

    freqs = position_ids.float()[..., None] * inv_freq[None, None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    if exact:
        return torch.cos(emb.double()).float().contiguous(), torch.sin(emb.double()).float().contiguous()
    return torch.cos(emb).contiguous(), torch.sin(emb).contiguous()


# --- forward ----------------------------------------------------------------------------------------------


def _per_layer_inputs(params: Gemma4TextParams, config: Gemma4TextConfig, ids: torch.Tensor, x: torch.Tensor):
    """model.py:414-426."""

    P = config.hidden_size_per_layer_input
    L = config.num_hidden_layers
    B, S, M = x.shape
    dt = x.dtype
    token = params.embed_tokens_per_layer[ids]  # [B, S, L, P]
    scale = float(torch.tensor(math.sqrt(P), dtype=dt))  # sqrt(P) rounded to the activation dtype, on the host
    token = (token.float() * scale).to(dt)
    ctx = _mm(x.reshape(B * S, M), params.per_layer_model_projection.reshape(M, L * P)).reshape(B, S, L, P)
    ctx = (ctx.float() * (config.hidden_size ** -0.5)).to(dt)
    ctx = rms_norm(ctx, params.per_layer_projection_norm.weight, config.rms_norm_eps)
    return ((ctx.float() + token.float()).to(dt).float() * (2.0 ** -0.5)).to(dt)


def forward_gemma4_text(
    params: Gemma4TextParams,
    input_ids: torch.Tensor,
    position_ids: torch.Tensor,
    *,
    config: Gemma4TextConfig,
    attention_mask: torch.Tensor | None = None,
    kv_cache: KVCache | None = None,
    cache_mode: Literal["prefill", "append"] = "prefill",
    layer_outputs: list | None = None,
    remat_layers: bool = False,
    lora=None,
    write_pos: torch.Tensor | None = None,
) -> tuple[torch.Tensor, KVCache | None]:
    """model.py:571-673: hidden after the final norm and the updated cache.

    Without a cache the forward runs in prefill form over a scratch cache (the reference's
    cache-less path computes the same attention). ``layer_outputs`` collects every decoder
    layer's output (the reference's parity hook, model.py:580). ``remat_layers`` is accepted for
    the reference's signature: it only changes which activations the reference's backward keeps
    (jax.checkpoint, model.py:651), and this forward-only path keeps none. ``lora`` must be None:
    the rollout path runs without adapters (the reference applies LoRA inside the projections,
    lora.py:107-113).

    Prefill mode into a cache that already holds ``length`` positions (model.py:604-623): the
    chunk attends to itself only (its own key mask, physical query indices from 0), its K/V are
    written from slot ``length`` (ring slots modulo the window; a linear cache's start and the key
    mask's are clamped into the capacity like ``lax.dynamic_update_slice``), and ``length``
    grows by the chunk.

    The caches are written in place, and the returned ``KVCache`` shares them. A later call on
    the input ``KVCache`` object (its own ``length``) still computes what the reference computes
    on it: an append at ``length`` overwrites the one slot this call wrote before anything reads it
    (a ring slot's earlier position lies outside the window of every query from ``length`` on).
    Only a caller that reads the input cache's arrays directly sees this call's writes.

    ``write_pos`` (append mode only): int32 ``[B]`` device tensor holding the physical slot of
    this step (``kv_cache.length``) for every row. The kernels then read the slot on the device
    and the key mask is updated in place, so the step has no host-side value baked in and can be
    captured in a HIP graph and replayed."""

    if lora is not None:
        raise NotImplementedError("LoRA adapters are not supported by the native rollout path")
    B, S = input_ids.shape
    dev = input_ids.device
    pw = pack_weights(params, config)
    eps = config.rms_norm_eps
    if attention_mask is None:
        attention_mask = torch.ones((B, S), dtype=torch.bool, device=dev)
    attention_mask = attention_mask.to(torch.bool)

    # graphed decode step: the embedding, key-mask update and rotary tables in one native launch
    fused_prologue = (write_pos is not None and cache_mode == "append" and kv_cache is not None and S == 1
                      and params.embed_tokens.dtype == torch.bfloat16 and not config.hidden_size_per_layer_input
                      and params.embed_tokens.shape[1] % 8 == 0)
    if fused_prologue:
        tabs = (SLIDING, FULL)
        x, tables = kernels.decode_prologue(
            params.embed_tokens, input_ids[:, 0], position_ids[:, 0], attention_mask[:, 0], write_pos,
            kv_cache.key_mask, embed_scale=pw.embed_scale_f, inv_freq=[pw.inv_freq[t] for t in tabs])
        x = x.view(B, 1, -1)
        rot = {t: (c.view(B, 1, -1), sn.view(B, 1, -1)) for t, (c, sn) in zip(tabs, tables)}
        pli = None
    else:
        x = params.embed_tokens[input_ids.long()]
        x = (x.float() * pw.embed_scale.float()).to(x.dtype)
        pli = _per_layer_inputs(params, config, input_ids.long(), x) if config.hidden_size_per_layer_input else None

    scratch_cache = kv_cache is None
    if scratch_cache:
        kv_cache = init_kv_cache(config, B, S, x.dtype, dev)
        cache_mode = "prefill"
    if cache_mode == "append" and S != 1:
        raise ValueError(f'cache_mode="append" requires one token, got {S}')
    length = int(kv_cache.length)
    capacity = kv_cache.key_mask.shape[1]
    if S > capacity:
        raise ValueError(f"{S} tokens do not fit a cache of {capacity} positions")
    if write_pos is not None:
        if cache_mode != "append":
            raise ValueError("write_pos is only used in append mode")
        key_mask = kv_cache.key_mask
        if not fused_prologue:
            key_mask.scatter_(1, write_pos[:, None].long(), attention_mask)
        slot = write_pos
    else:
        key_mask = kv_cache.key_mask.clone()
        mask_start = min(max(length, 0), capacity - S)  # lax.dynamic_update_slice's clamp (model.py:602)
        key_mask[:, mask_start:mask_start + S] = attention_mask
        slot = length
    chunk_prefill = cache_mode == "prefill" and length != 0  # model.py:615-617: the chunk attends to itself
    if not fused_prologue:
        exact = x.dtype == torch.float32
        rot = {t: rotary_tables(pw.inv_freq[t], position_ids, exact) for t in (SLIDING, FULL)}
    sources = kv_source_layers(config)

    flags_q = _lib.G4_APPEND_NORM_Q | _lib.G4_APPEND_ROPE_Q
    flags_kv = _lib.G4_APPEND_NORM_K | _lib.G4_APPEND_ROPE_K | _lib.G4_APPEND_NORM_V
    prompt_kv: dict = {}  # layer index -> (k [B,H,Sp,D], vt [B,H,D,Sp]) for prefill attention
    new_layers = []
    n_layers = len(params.layers)
    h = kernels.rms_norm(x, params.layers[0].input_norm.weight, eps)  # layer 0's input norm
    for i, (lp, pk) in enumerate(zip(params.layers, pw.layers)):
        lt = config.layer_types[i]
        window = config.sliding_window if lt == SLIDING else 0
        H, R, D = pk.heads, pk.group, pk.head_dim
        qkv = _proj(h.reshape(B * S, -1), pk.w_qkv_t).reshape(B, S, -1)
        q = qkv[..., : H * R * D].view(B, S, H, R, D)
        cos, sin = rot[lt]
        layer_cache = kv_cache.layers[i]
        shared = is_kv_shared(config, i)
        if write_pos is not None and _fused_decode_prep(x, B * H, D, new_layers[sources[i]] if shared else layer_cache):
            # graphed decode step at the rollout batch: g4_kv_append's work runs inside the
            # two-launch attention (G4DecodePrep) on the raw projection rows
            if shared:
                src_cache, kr, vr, flags = new_layers[sources[i]], None, None, flags_q
                new_layers.append(None)
            else:
                k = qkv[..., H * R * D: (H * R + H) * D].view(B, S, H, D)
                v = qkv[..., (H * R + H) * D:].view(B, S, H, D) if pk.has_v else k
                src_cache, kr, vr, flags = layer_cache, k[:, 0], v[:, 0], flags_q | flags_kv
                new_layers.append(layer_cache)
            attn = kernels.decode_attention_fused(
                src_cache, q[:, 0], key_mask, q_pos=slot, window=config.sliding_window, k_raw=kr, v_raw=vr,
                q_norm_weight=lp.attention.q_norm.weight,
                k_norm_weight=None if lp.attention.k_norm is None else lp.attention.k_norm.weight,
                rope_cos=cos[:, 0], rope_sin=sin[:, 0], eps=eps, flags=flags).view(B, 1, H, R, D)
        else:
            q_out = torch.empty((B, S, H, R, D), dtype=x.dtype, device=dev)
            if shared:
                kernels.prepare_q(q, q_out, q_norm_weight=lp.attention.q_norm.weight, eps=eps, rope_cos=cos,
                                  rope_sin=sin, flags=flags_q)
                src = sources[i]
                src_cache = new_layers[src]
                new_layers.append(None)
            else:
                k = qkv[..., H * R * D: (H * R + H) * D].view(B, S, H, D)
                v = qkv[..., (H * R + H) * D:].view(B, S, H, D) if pk.has_v else k
                k_out = vt_out = None
                if cache_mode == "prefill" and (layer_cache.ring or chunk_prefill):
                    sp = slot_stride_for(S)
                    k_out = torch.empty(key_shape(B, H, sp, D), dtype=x.dtype, device=dev)
                    vt_out = torch.zeros((B, H, sp // 8, D, 8), dtype=x.dtype, device=dev)
                kernels.kv_append(layer_cache, k, v, write_pos=slot, flags=flags_q | flags_kv, eps=eps, q=q,
                                  q_out=q_out, q_norm_weight=lp.attention.q_norm.weight,
                                  k_norm_weight=lp.attention.k_norm.weight, rope_cos=cos, rope_sin=sin, k_out=k_out,
                                  vt_out=vt_out)
                if k_out is not None:
                    prompt_kv[i] = (k_out, vt_out)
                src = i
                src_cache = layer_cache
                new_layers.append(layer_cache)
            if cache_mode == "prefill":
                if src in prompt_kv:
                    kk, vt = prompt_kv[src]
                else:
                    kk, vt = src_cache.key, src_cache.value_t
                attn = kernels.prefill_attention(q_out, kk, vt, attention_mask.contiguous() if chunk_prefill else key_mask,
                                                 window=window)
            else:
                attn = kernels.decode_attention(src_cache, q_out.view(B, H, R, D), key_mask, q_pos=slot,
                                                window=config.sliding_window).view(B, 1, H, R, D)
        o = _proj(attn.reshape(B * S, H * R * D), pk.w_o_t).reshape(B, S, -1)
        # post-attention norm + residual, then the pre-feedforward norm (one pass)
        x, h = kernels.residual_norm(o, lp.post_attention_norm.weight, x, scalar=None,
                                     next_weight=lp.pre_feedforward_norm.weight, eps=eps)
        if _native_gate_up(h, pk.w_gate_up_t):  # decode batch: projection and activation in one launch
            act = kernels.linear_gelu(h.reshape(B * S, -1), pk.w_gate_up_t)
        else:
            gu = _proj(h.reshape(B * S, -1), pk.w_gate_up_t)
            act = kernels.gelu_mul(gu)
        next_w = params.layers[i + 1].input_norm.weight if i + 1 < n_layers else params.final_norm.weight
        if lp.per_layer_input is None and _split_down(act, pk.w_down_t):
            # decode batch: the down projection's split-K partial sums go straight into the
            # post-feedforward norm + residual (+ layer scalar) + next norm
            part = kernels.linear_partials(act, pk.w_down_t, ksplit=DOWN_KSPLIT)
            x, h = kernels.residual_norm_splitk(part, lp.post_feedforward_norm.weight, x, scalar=pk.scalar_f32,
                                                next_weight=next_w, eps=eps)
            if layer_outputs is not None:
                layer_outputs.append(x)
            continue
        d = _proj(act, pk.w_down_t).reshape(B, S, -1)
        if lp.per_layer_input is None:
            # post-feedforward norm + residual, layer scalar, then the next layer's input norm
            # (the final norm after the last layer)
            x, h = kernels.residual_norm(d, lp.post_feedforward_norm.weight, x, scalar=pk.scalar_f32,
                                         next_weight=next_w, eps=eps)
        else:
            x, _ = kernels.residual_norm(d, lp.post_feedforward_norm.weight, x, scalar=None, next_weight=None,
                                         eps=eps, with_next=False)
            g = _mm(x.reshape(B * S, -1), lp.per_layer_input.gate)
            g = (gelu_tanh_f32(g, x.dtype == torch.float32) * pli[:, :, i].reshape(B * S, -1).float()).to(x.dtype)
            g = _mm(g, lp.per_layer_input.projection).reshape(B, S, -1)
            g = rms_norm(g, lp.per_layer_input.post_norm.weight, eps)
            x = x + g
            x = (x.float() * lp.layer_scalar.float()).to(x.dtype)
            h = kernels.rms_norm(x, next_w, eps)
        if layer_outputs is not None:
            layer_outputs.append(x)
    hidden = h
    if scratch_cache:
        return hidden, None
    return hidden, KVCache(tuple(new_layers), key_mask, length + S)


def checked_softcap(cap: float | None) -> float | None:
    """``final_logit_softcapping`` as every LM-head path here applies it (``forward_lm_head``, the
    graphed decode step's fused draw, ``generate``): None (no cap) or a positive finite float.
    A cap of 0 or below would make the reference's ``tanh(x / cap) * cap`` (model.py:678-679) all
    zeros or NaN; every path rejects it with the same ``ValueError`` instead."""

    if cap is None:
        return None
    cap = float(cap)
    if not (math.isfinite(cap) and cap > 0):
        raise ValueError(f"final_logit_softcapping must be None or a positive finite number, got {cap}")
    return cap


def forward_lm_head(embed_tokens: torch.Tensor, hidden: torch.Tensor, softcap: float | None) -> torch.Tensor:
    """model.py:676-680: tied-embedding logits, ``tanh(x / cap) * cap``."""

    softcap = checked_softcap(softcap)
    B, S, M = hidden.shape
    x = hidden.reshape(B * S, M)
    if x.is_cuda and kernels.lm_head_supported(x, embed_tokens):
        # the decode batch (<= 256 rows): the native LM head, the GEMM g4_lm_head_sample runs when it
        # samples in its epilogue, so a step's logits and its fused draw see the same bf16 values
        logits = kernels.lm_head(x.contiguous(), embed_tokens).reshape(B, S, -1)
    else:
        logits = _proj(x, embed_tokens).reshape(B, S, -1)
    if softcap is not None:
        if logits.dtype == torch.bfloat16 and logits.is_cuda and logits.is_contiguous():
            logits = kernels.softcap(logits, softcap, out=logits)  # one native pass, the same bits
        elif logits.dtype == torch.float32:  # tanh in f64, rounded once; the division and product in f32
            logits = torch.tanh((logits / softcap).double()).float() * softcap
        else:
            logits = (torch.tanh(logits.float() / softcap) * softcap).to(logits.dtype)
    return logits


def forward_gemma4_lm(
    params: Gemma4TextParams,
    input_ids: torch.Tensor,
    position_ids: torch.Tensor,
    *,
    config: Gemma4TextConfig,
    attention_mask: torch.Tensor | None = None,
    kv_cache: KVCache | None = None,
    cache_mode: Literal["prefill", "append"] = "prefill",
    logits_to_keep: int = 0,
    lora=None,
    write_pos: torch.Tensor | None = None,
) -> Gemma4Output:
    """model.py:683-709 (``write_pos``: see forward_gemma4_text)."""

    hidden, cache = forward_gemma4_text(params, input_ids, position_ids, config=config,
                                        attention_mask=attention_mask, kv_cache=kv_cache, cache_mode=cache_mode,
                                        lora=lora, write_pos=write_pos)
    head_in = hidden[:, -logits_to_keep:] if logits_to_keep > 0 else hidden
    return Gemma4Output(forward_lm_head(params.embed_tokens, head_in, config.final_logit_softcapping), hidden, cache)


__all__ = [
    "RMSNormParams", "AttentionParams", "MLPParams", "PerLayerInputParams", "DecoderLayerParams",
    "Gemma4TextParams", "Gemma4Output", "Gemma4TextConfig", "KVCache", "LayerKVCache", "init_kv_cache",
    "forward_gemma4_text", "forward_gemma4_lm", "forward_lm_head", "checked_softcap", "params_from_numpy", "pack_weights",
    "rms_norm", "layer_head_dim", "layer_kv_heads", "layer_has_v_proj", "layer_intermediate_size",
]
