"""numpy restatement of the reference's Gemma 4 prefill + KV-cache decode path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` as the checker / the timed CPU path, never by the GPU library.

Every function names the reference code it restates (``model.py`` / ``sampler.py`` of
``gemma4_posttrain_jax``). Two arithmetic modes mirror the reference's dtypes:

* ``"float32"`` — every array is float32; elementwise ops round to f32 once per numpy op.
* ``"bfloat16"`` — arrays hold bf16-representable float32 values. Matmuls/einsums accumulate in
  f32 and round the result to bf16 once (round-to-nearest-even); RMSNorm and softmax compute in
  f32 and round once; an elementwise chain written on one reference line (RoPE, gelu, softcap) is
  evaluated in f32 and rounded once, which is what XLA's fused elementwise kernels do with its
  default ``xla_allow_excess_precision``. Explicit ``astype`` casts in the reference (cos/sin to the
  activation dtype, scores to f32, probs to bf16) are kept as explicit roundings.

Pinning (which check fixes which part) is listed per function; the tests under ``tests/`` that
exercise the pins are ``test_oracle_*.py``.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import numpy as np

from . import jax_random as JR

SLIDING = "sliding_attention"
FULL = "full_attention"

F32 = "float32"
BF16 = "bfloat16"

# jnp.finfo(bf16).min and jnp.finfo(f32).min: the masked-score fill of model.py:497.
BF16_MIN = np.float32(-3.3895313892515355e38)
F32_MIN = np.float32(np.finfo(np.float32).min)


# --- bf16 helpers -------------------------------------------------------------------------------


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even); NaN stays NaN. Returns float32."""

    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).reshape(x.shape)
    return np.where(np.isnan(x), np.float32(np.nan), out).astype(np.float32)


def bf16_bits(x) -> np.ndarray:
    """uint16 storage bits of ``bf16_round(x)``."""

    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def cast(x, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return bf16_round(x) if dtype == BF16 else x


def fill_min(dtype: str) -> np.float32:
    return BF16_MIN if dtype == BF16 else F32_MIN


# --- config (model.py:32-58, 100-147) -----------------------------------------------------------


class Config(NamedTuple):
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    global_head_dim: int
    num_global_key_value_heads: int | None
    layer_types: tuple
    sliding_window: int
    num_kv_shared_layers: int = 0
    use_double_wide_mlp: bool = False
    attention_k_eq_v: bool = False
    hidden_size_per_layer_input: int = 0
    vocab_size_per_layer_input: int = 0
    rms_norm_eps: float = 1e-6
    rope_theta_sliding: float = 10_000.0
    rope_theta_full: float = 1_000_000.0
    full_partial_rotary_factor: float = 0.25
    final_logit_softcapping: float | None = 30.0
    bos_token_id: int = 2
    eos_token_id: int = 1
    pad_token_id: int = 0


def config_from_hf(hf: dict) -> Config:
    """model.py:100-147 for configs without ``per_layer_config`` (last layer forced FULL, line 112)."""

    text = hf.get("text_config", hf)
    if "per_layer_config" in text:
        raise ValueError("per_layer_config is not handled by the oracle")
    n = int(text["num_hidden_layers"])
    layer_types = list(text["layer_types"])
    if len(layer_types) != n:
        raise ValueError("layer_types length mismatch")
    layer_types[-1] = FULL
    rope = text.get("rope_parameters") or {}
    sliding_rope = rope.get(SLIDING) or {}
    full_rope = rope.get(FULL) or {}
    return Config(
        vocab_size=int(text["vocab_size"]),
        hidden_size=int(text["hidden_size"]),
        intermediate_size=int(text["intermediate_size"]),
        num_hidden_layers=n,
        num_attention_heads=int(text["num_attention_heads"]),
        num_key_value_heads=int(text["num_key_value_heads"]),
        head_dim=int(text.get("head_dim", 256)),
        global_head_dim=int(text.get("global_head_dim", 512)),
        num_global_key_value_heads=text.get("num_global_key_value_heads"),
        layer_types=tuple(layer_types),
        sliding_window=int(text.get("sliding_window", 512)),
        num_kv_shared_layers=int(text.get("num_kv_shared_layers", 0)),
        use_double_wide_mlp=bool(text.get("use_double_wide_mlp", False)),
        attention_k_eq_v=bool(text.get("attention_k_eq_v", False)),
        hidden_size_per_layer_input=int(text.get("hidden_size_per_layer_input", 256)),
        vocab_size_per_layer_input=int(text.get("vocab_size_per_layer_input", 262144)),
        rms_norm_eps=float(text.get("rms_norm_eps", 1e-6)),
        rope_theta_sliding=float(sliding_rope.get("rope_theta", 10_000.0)),
        rope_theta_full=float(full_rope.get("rope_theta", 1_000_000.0)),
        full_partial_rotary_factor=float(full_rope.get("partial_rotary_factor", 0.25)),
        final_logit_softcapping=text.get("final_logit_softcapping"),
        bos_token_id=int(text.get("bos_token_id", 2)),
        eos_token_id=int(text.get("eos_token_id", 1)),
        pad_token_id=int(text.get("pad_token_id", 0)),
    )


# --- static per-layer derivations (model.py:153-187) --------------------------------------------


def is_kv_shared(cfg: Config, i: int) -> bool:
    """model.py:153-155."""

    return cfg.num_kv_shared_layers > 0 and i >= cfg.num_hidden_layers - cfg.num_kv_shared_layers


def kv_source_layer(cfg: Config, i: int) -> int:
    """model.py:158-168: last non-shared layer of the same type. Pinned by the KAT
    ``kv_source_layer(TINY_A, 4) == 3, (5) == 1`` (tests/test_model_ops.py:62) and brute force."""

    if not is_kv_shared(cfg, i):
        return i
    first_shared = cfg.num_hidden_layers - cfg.num_kv_shared_layers
    for j in range(first_shared - 1, -1, -1):
        if cfg.layer_types[j] == cfg.layer_types[i]:
            return j
    raise ValueError(f"no non-shared {cfg.layer_types[i]} layer before layer {i}")


def layer_head_dim(cfg: Config, i: int) -> int:
    """model.py:171-172."""

    return cfg.global_head_dim if cfg.layer_types[i] == FULL else cfg.head_dim


def layer_kv_heads(cfg: Config, i: int) -> int:
    """model.py:175-178."""

    if cfg.layer_types[i] == FULL and cfg.attention_k_eq_v and cfg.num_global_key_value_heads:
        return int(cfg.num_global_key_value_heads)
    return cfg.num_key_value_heads


def layer_has_v_proj(cfg: Config, i: int) -> bool:
    """model.py:181-182."""

    return not (cfg.attention_k_eq_v and cfg.layer_types[i] == FULL)


def layer_intermediate_size(cfg: Config, i: int) -> int:
    """model.py:185-187."""

    return cfg.intermediate_size * (2 if (cfg.use_double_wide_mlp and is_kv_shared(cfg, i)) else 1)


# --- parameters (model.py:193-235), random init for the synthetic configs -----------------------


class AttnParams(NamedTuple):
    q_proj: np.ndarray  # [M, R, H, D]
    k_proj: np.ndarray | None  # [M, H, D]
    v_proj: np.ndarray | None  # [M, H, D]
    o_proj: np.ndarray  # [R, H, D, M]
    q_norm: np.ndarray  # [D]
    k_norm: np.ndarray | None  # [D]


class MLPParams(NamedTuple):
    gate_proj: np.ndarray  # [M, F]
    up_proj: np.ndarray  # [M, F]
    down_proj: np.ndarray  # [F, M]


class PLEParams(NamedTuple):
    gate: np.ndarray  # [M, P]
    projection: np.ndarray  # [P, M]
    post_norm: np.ndarray  # [M]


class LayerParams(NamedTuple):
    input_norm: np.ndarray
    attention: AttnParams
    post_attention_norm: np.ndarray
    pre_feedforward_norm: np.ndarray
    mlp: MLPParams
    post_feedforward_norm: np.ndarray
    per_layer_input: PLEParams | None
    layer_scalar: np.float32


class Params(NamedTuple):
    embed_tokens: np.ndarray  # [V, M]
    embed_tokens_per_layer: np.ndarray | None  # [Vp, L, P]
    per_layer_model_projection: np.ndarray | None  # [M, L, P]
    per_layer_projection_norm: np.ndarray | None  # [P]
    layers: tuple
    final_norm: np.ndarray  # [M]


def init_params(
    cfg: Config,
    seed: int,
    dtype: str = F32,
    *,
    std: float = 0.02,
    norm_std: float = 0.0,
    layer_scalar_min: float = 1.0,
    qk_norm_scale: float = 1.0,
) -> Params:
    """Seeded random weights ~N(0, std); norms ``1 + norm_std*N``; ``layer_scalar`` U[min, 1]
    (the recipe of tests/conftest.py:67-87 with BASELINE's N(0, 0.02) default). Values are
    rounded to ``dtype``. Generation order is fixed so the GPU tests can rebuild the same weights.

    ``qk_norm_scale`` multiplies the q / k norm weights (drawn as above). With weights near 1 the
    normed q and k have unit RMS and the scale-1.0 scores reach ~sqrt(D) in magnitude, where one
    bf16 ulp of a score moves a probability by several percent; bf16 test models that must be
    determined to 2e-2 at the logits use ~0.35, which keeps scores O(1)."""

    rng = np.random.default_rng(seed)
    M, Hq = cfg.hidden_size, cfg.num_attention_heads

    def w(*shape):
        return cast(rng.standard_normal(shape, dtype=np.float32) * np.float32(std), dtype)

    def norm(n):
        return cast(1.0 + np.float32(norm_std) * rng.standard_normal(n, dtype=np.float32), dtype)

    embed = w(cfg.vocab_size, M)
    L, P = cfg.num_hidden_layers, cfg.hidden_size_per_layer_input
    ple_table = ple_proj = ple_norm = None
    if P:
        ple_table = w(cfg.vocab_size_per_layer_input, L, P)
        ple_proj = w(M, L, P)
        ple_norm = norm(P)
    layers = []
    for i in range(L):
        D, H = layer_head_dim(cfg, i), layer_kv_heads(cfg, i)
        R = Hq // H
        shared = is_kv_shared(cfg, i)
        q = w(M, R, H, D)
        k = None if shared else w(M, H, D)
        v = None if (shared or not layer_has_v_proj(cfg, i)) else w(M, H, D)
        o = w(R, H, D, M)
        qn = cast(norm(D) * np.float32(qk_norm_scale), dtype)
        kn = None if shared else cast(norm(D) * np.float32(qk_norm_scale), dtype)
        F = layer_intermediate_size(cfg, i)
        mlp = MLPParams(w(M, F), w(M, F), w(F, M))
        ple = PLEParams(w(M, P), w(P, M), norm(M)) if P else None
        in_n, post_a, pre_f, post_f = norm(M), norm(M), norm(M), norm(M)
        scalar = np.float32(rng.uniform(layer_scalar_min, 1.0)) if layer_scalar_min < 1.0 else np.float32(1.0)
        layers.append(
            LayerParams(in_n, AttnParams(q, k, v, o, qn, kn), post_a, pre_f, mlp, post_f, ple, cast(scalar, dtype)[()])
        )
    return Params(embed, ple_table, ple_proj, ple_norm, tuple(layers), norm(M))


# --- primitives (model.py:272-317) --------------------------------------------------------------


_ACCUMULATE = [np.float32]


class accumulate_f64:
    """Context manager: matmuls accumulate in float64 (then round as usual). Two valid f32
    accumulation orders of the reference differ about as much as f32 and f64 accumulation do;
    the tests use this pair to measure how precisely the reference's output is determined."""

    def __enter__(self):
        _ACCUMULATE.append(np.float64)

    def __exit__(self, *exc):
        _ACCUMULATE.pop()


def exact_f32(dtype: str) -> bool:
    """Under ``accumulate_f64`` an f32 model is evaluated exactly rounded: besides the products,
    every reduction (the norms' sums of squares, the softmax sums) is summed in f64 and rounded
    once, and every transcendental (exp, tanh, x^-0.5, cos, sin) is evaluated in f64 and rounded
    once, while the reference's single IEEE operations (+, -, *, /) round to f32 one at a time in
    its own order. Every f32 evaluation order (XLA's, numpy's, torch's) lies within its own rounding
    noise of this one; the native fp32 path computes it too. bf16 models keep the f32 evaluation."""

    return dtype == F32 and _ACCUMULATE[-1] is np.float64


def _f32(x) -> np.ndarray:
    return np.asarray(x, np.float64).astype(np.float32)


def matmul(x: np.ndarray, w: np.ndarray, dtype: str) -> np.ndarray:
    """f32-accumulated product rounded once to ``dtype`` (an einsum / ``@`` in the reference)."""

    acc = _ACCUMULATE[-1]
    return cast(np.matmul(x.astype(acc), w.astype(acc)).astype(np.float32), dtype)


def scale(x: np.ndarray, factor: float, dtype: str) -> np.ndarray:
    """model.py:272-275: f32 multiply then round."""

    return cast(x.astype(np.float32) * np.float32(factor), dtype)


def rms_norm(weight: np.ndarray | None, x: np.ndarray, eps: float, dtype: str) -> np.ndarray:
    """model.py:278-285: f32 ``x * (mean(x^2) + eps)^-0.5 * w``; ``None`` = no scale.
    Pinned against HF ``Gemma4RMSNorm`` (test_oracle_model.py) and the closed form on constants."""

    x32 = x.astype(np.float32)
    if exact_f32(dtype):  # square, sum (f64, one rounding), / n, + eps, ^-0.5 (f64), * r, * w
        sq = x32 * x32
        ms = _f32(sq.astype(np.float64).sum(axis=-1, keepdims=True)) / np.float32(x.shape[-1])
        r = _f32(1.0 / np.sqrt((ms + np.float32(eps)).astype(np.float64)))
        y = x32 * r
        return y * weight.astype(np.float32) if weight is not None else y
    ms = np.mean(np.square(x32), axis=-1, keepdims=True, dtype=np.float32)
    y = x32 * np.power(ms + np.float32(eps), np.float32(-0.5), dtype=np.float32)
    if weight is not None:
        y = y * weight.astype(np.float32)
    return cast(y, dtype)


def rope_inv_freq(cfg: Config) -> dict:
    """model.py:294-302: default RoPE on sliding layers, 'proportional' partial RoPE on full layers."""

    dim = cfg.head_dim
    inv_sliding = (
        np.float32(1.0)
        / np.power(np.float32(cfg.rope_theta_sliding), np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim))
    ).astype(np.float32)
    dim = cfg.global_head_dim
    angles = int(cfg.full_partial_rotary_factor * dim // 2)
    inv_rot = (
        np.float32(1.0)
        / np.power(np.float32(cfg.rope_theta_full), np.arange(0, 2 * angles, 2, dtype=np.float32) / np.float32(dim))
    ).astype(np.float32)
    inv_full = np.concatenate([inv_rot, np.zeros(dim // 2 - angles, np.float32)])
    return {SLIDING: inv_sliding, FULL: inv_full}


def rotary_values(inv_freq: np.ndarray, position_ids: np.ndarray, exact: bool = False) -> tuple[np.ndarray, np.ndarray]:
    """model.py:288-291: ``emb = concat(f, f)``, f = pos * inv_freq; f32 cos/sin ``[B, S, D]``
    (``exact``: cos / sin in f64, rounded once)."""

    freqs = position_ids.astype(np.float32)[..., None] * inv_freq[None, None, :]
    emb = np.concatenate([freqs, freqs], axis=-1).astype(np.float32)
    if exact:
        e64 = emb.astype(np.float64)
        return _f32(np.cos(e64)), _f32(np.sin(e64))
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def make_rotary(cfg: Config, position_ids: np.ndarray, dtype: str | None = None) -> dict:
    inv = rope_inv_freq(cfg)
    exact = dtype is not None and exact_f32(dtype)
    return {t: rotary_values(inv[t], position_ids, exact) for t in (SLIDING, FULL)}


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, dtype: str) -> np.ndarray:
    """model.py:309-317: ``x*cos + rotate_half(x)*sin``; cos/sin cast to the activation dtype first.

    ``x`` is ``[B, S, ..., D]`` and cos/sin ``[B, S, D]``. In f32 mode each product and the sum
    round to f32 separately (numpy op order). In bf16 mode the bf16×bf16 products are exact in f32,
    the sum rounds to f32 and then once to bf16."""

    shape = x.shape[:2] + (1,) * (x.ndim - 3) + x.shape[-1:]
    c = cast(cos, dtype).reshape(shape)
    s = cast(sin, dtype).reshape(shape)
    half = x.shape[-1] // 2
    x32 = x.astype(np.float32)
    rotated = np.concatenate([-x32[..., half:], x32[..., :half]], axis=-1)
    return cast(x32 * c + rotated * s, dtype)


def gelu_tanh(x: np.ndarray, exact: bool = False) -> np.ndarray:
    """jax.nn.gelu(approximate=True) in f32 (model.py:396). ``exact``: its own op order,
    ``x * (0.5 * (1 + tanh(c * (x + 0.044715 * ((x * x) * x)))))``, each op rounded to f32 and
    tanh evaluated in f64."""

    x = x.astype(np.float32)
    if exact:
        u = x + np.float32(0.044715) * ((x * x) * x)
        th = _f32(np.tanh((np.float32(math.sqrt(2.0 / math.pi)) * u).astype(np.float64)))
        return x * (np.float32(0.5) * (np.float32(1.0) + th))
    inner = np.float32(math.sqrt(2.0 / math.pi)) * (x + np.float32(0.044715) * x * x * x)
    return (np.float32(0.5) * x * (np.float32(1.0) + np.tanh(inner))).astype(np.float32)


# --- masks and ring-slot arithmetic (model.py:320-365) ------------------------------------------


def make_qk_masks(key_mask: np.ndarray, window: int, query_start: int, num_queries: int) -> dict:
    """model.py:320-335: ``[B,1,1,S,T]``; causal ``k <= q`` + key padding; sliding adds ``k > q-W``
    in physical index space (pads count toward the window). Pinned by brute force in tests."""

    T = key_mask.shape[1]
    q = (np.arange(num_queries) + query_start)[:, None]
    k = np.arange(T)[None, :]
    full = (k <= q)[None] & key_mask[:, None, :].astype(bool)
    sliding = full & (k > q - window)[None]
    return {FULL: full[:, None, None], SLIDING: sliding[:, None, None]}


def ring_slot_positions(last_written, window_capacity: int) -> np.ndarray:
    """model.py:357: slot ``r`` holds the greatest position ``p <= last_written`` with
    ``p % Wc == r`` (negative = never written). ``last_written`` may be a scalar or ``[B]``."""

    slots = np.arange(window_capacity, dtype=np.int64)
    n = np.asarray(last_written, dtype=np.int64)[..., None]
    return slots + np.floor_divide(n - slots, window_capacity) * window_capacity


def make_cached_qk_masks(key_mask: np.ndarray, window: int, query_start, num_queries: int) -> dict:
    """model.py:338-365, generalized to a per-row ``query_start`` ``[B]`` (the reference's scalar
    ``length`` is the special case of equal rows). Returns ``{FULL: [B,1,1,S,C], SLIDING: [B,1,1,S,Wc]}``."""

    B, capacity = key_mask.shape
    wc = min(window, capacity)
    qs = np.broadcast_to(np.asarray(query_start, dtype=np.int64), (B,))
    q_abs = qs[:, None] + np.arange(num_queries)[None, :]  # [B, S]
    full_k = np.arange(capacity)[None, None, :]
    full = (full_k <= q_abs[:, :, None]) & key_mask[:, None, :].astype(bool)
    last = qs + num_queries - 1
    sk = ring_slot_positions(last, wc)  # [B, Wc]
    valid = sk >= 0
    gathered = np.take_along_axis(key_mask.astype(bool), np.clip(sk, 0, capacity - 1), axis=1) & valid
    sliding = (
        (sk[:, None, :] <= q_abs[:, :, None]) & (sk[:, None, :] > q_abs[:, :, None] - window) & valid[:, None, :]
    )
    sliding = sliding & gathered[:, None, :]
    return {FULL: full[:, None, None], SLIDING: sliding[:, None, None]}


# --- KV cache (model.py:238-255, 368-390, 557-568) ----------------------------------------------


class LayerKV(NamedTuple):
    key: np.ndarray  # [B, C, H, D]
    value: np.ndarray  # [B, C, H, D]


class KVCache(NamedTuple):
    layers: tuple  # LayerKV or None (kv-shared)
    key_mask: np.ndarray  # [B, C] bool
    length: int


def init_kv_cache(cfg: Config, batch: int, capacity: int, dtype: str) -> KVCache:
    """model.py:557-568: ring of ``min(W, C)`` slots on sliding layers, ``C`` on full layers,
    ``None`` on kv-shared layers."""

    layers = []
    for i in range(cfg.num_hidden_layers):
        if is_kv_shared(cfg, i):
            layers.append(None)
            continue
        c = min(cfg.sliding_window, capacity) if cfg.layer_types[i] == SLIDING else capacity
        shape = (batch, c, layer_kv_heads(cfg, i), layer_head_dim(cfg, i))
        layers.append(LayerKV(np.zeros(shape, np.float32), np.zeros(shape, np.float32)))
    return KVCache(tuple(layers), np.zeros((batch, capacity), bool), 0)


_INPLACE = [False]


class inplace_cache_updates:
    """Context manager: cache appends write into the existing arrays instead of copying them
    (what XLA does inside the reference's while_loop); used when the oracle is timed."""

    def __enter__(self):
        _INPLACE.append(True)

    def __exit__(self, *exc):
        _INPLACE.pop()


def append_slots(start: int, num_new: int, capacity: int, circular: bool) -> tuple[np.ndarray, np.ndarray]:
    """Destination slots and source rows of one ``_update_layer_cache`` call (model.py:368-390).
    Linear: rows ``0..S-1`` -> slots ``start..start+S-1``. Ring: the last ``keep = min(S, Wc)`` rows
    -> ``(abs) mod Wc``."""

    if not circular:
        return np.arange(start, start + num_new), np.arange(num_new)
    keep = min(num_new, capacity)
    src = np.arange(num_new - keep, num_new)
    return np.mod(src + start, capacity), src


def update_layer_cache(layer: LayerKV, k: np.ndarray, v: np.ndarray, start, circular: bool, dtype: str) -> LayerKV:
    """model.py:368-390 on ``[B, C, H, D]`` caches; ``start`` is a scalar (the reference) or ``[B]``
    per-row write positions (each row then follows the reference as a batch-1 cache)."""

    k = cast(k, dtype)
    v = cast(v, dtype)
    if _INPLACE[-1]:
        ck, cv = layer.key, layer.value
    else:
        ck, cv = layer.key.copy(), layer.value.copy()
    C = ck.shape[1]
    starts = np.broadcast_to(np.asarray(start, dtype=np.int64), (ck.shape[0],))
    S = k.shape[1]
    for b in range(ck.shape[0]):
        st = int(starts[b])
        if not circular:
            # lax.dynamic_update_slice clamps the start into [0, C - S] so the update fits.
            st = min(max(st, 0), C - S)
        dst, src = append_slots(st, S, C, circular)
        ck[b, dst] = k[b, src]
        cv[b, dst] = v[b, src]
    return LayerKV(ck, cv)


# --- attention core (model.py:496-499) ----------------------------------------------------------


def attention_core(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray, dtype: str) -> np.ndarray:
    """model.py:496-499 with scale 1.0.

    q ``[B,S,R,H,D]``, k/v ``[B,T,H,D]``, mask broadcastable to ``[B,1,1,S,T]`` (or ``[B,R,H,S,T]``).
    scores = einsum in ``dtype`` (f32 accumulation, one rounding); masked -> ``finfo(dtype).min``;
    softmax in f32; probs rounded to ``dtype``; ``probs @ v`` accumulated in f32, rounded once.
    Under ``accumulate_f64`` both products accumulate in f64 (then round through f32), which gives
    the rounding of the exact dot product wherever f32 accumulation orders disagree near a bf16
    rounding boundary.
    A fully-masked row therefore averages all T keys (every score equals the fill value).
    Pinned against a float64 textbook softmax-attention and the fully-masked / single-key closed
    forms in tests/test_oracle_attention.py."""

    B, S, R, H, D = q.shape
    T = k.shape[1]
    acc = _ACCUMULATE[-1]  # f32, or f64 under accumulate_f64 (the exactly rounded products)
    out = np.empty((B, S, R, H, D), np.float32)
    qt = q.astype(acc).transpose(0, 2, 3, 1, 4)  # [B,R,H,S,D]
    kt = k.astype(acc).transpose(0, 2, 3, 1)  # [B,H,D,T]
    vt = v.astype(acc).transpose(0, 2, 1, 3)  # [B,H,T,D]
    mask = np.broadcast_to(mask, (B, R, H, S, T)) if mask.shape[1] != R else mask
    fill = fill_min(dtype)
    blk = max(1, min(S, (1 << 24) // max(1, B * R * H * T)))
    for s0 in range(0, S, blk):
        s1 = min(S, s0 + blk)
        sc = cast(np.matmul(qt[:, :, :, s0:s1], kt[:, None]).astype(np.float32), dtype)  # [B,R,H,s,T]
        sc = np.where(np.broadcast_to(mask, (B, R, H, S, T))[:, :, :, s0:s1], sc, fill)
        m = sc.max(axis=-1, keepdims=True)
        if exact_f32(dtype):  # exp in f64, the sum in f64, each rounded once
            e = _f32(np.exp((sc - m).astype(np.float64)))
            p = e / _f32(e.astype(np.float64).sum(axis=-1, keepdims=True))
        else:
            e = np.exp(sc - m)
            p = cast(e / e.sum(axis=-1, keepdims=True, dtype=np.float32), dtype)
        o = cast(np.matmul(p.astype(acc), vt[:, None]).astype(np.float32), dtype)  # [B,R,H,s,D]
        out[:, s0:s1] = o.transpose(0, 3, 1, 2, 4)
    return out


# --- model forward (model.py:438-709) -----------------------------------------------------------


def forward_attention(
    p: AttnParams,
    seq: np.ndarray,
    qk_mask: np.ndarray,
    rot: tuple,
    *,
    layer_index: int,
    cfg: Config,
    shared_kv: dict,
    layer_cache: LayerKV | None,
    cache_length,
    cache_mode: str,
    dtype: str,
):
    """model.py:438-502 (LoRA omitted: ``lora=None`` on the rollout path)."""

    layer_type = cfg.layer_types[layer_index]
    eps = cfg.rms_norm_eps
    B, S, M = seq.shape
    _, R, H, D = p.q_proj.shape
    q = matmul(seq, p.q_proj.reshape(M, R * H * D), dtype).reshape(B, S, R, H, D)
    q = rms_norm(p.q_norm, q, eps, dtype)
    q = rope(q, rot[0], rot[1], dtype)
    new_cache = None
    if is_kv_shared(cfg, layer_index):
        k, v = shared_kv[layer_type]
    else:
        k = matmul(seq, p.k_proj.reshape(M, H * D), dtype).reshape(B, S, H, D)
        v = matmul(seq, p.v_proj.reshape(M, H * D), dtype).reshape(B, S, H, D) if p.v_proj is not None else k
        k = rms_norm(p.k_norm, k, eps, dtype)
        k = rope(k, rot[0], rot[1], dtype)
        v = rms_norm(None, v, eps, dtype)
        if layer_cache is not None:
            new_cache = update_layer_cache(layer_cache, k, v, cache_length, layer_type == SLIDING, dtype)
            if cache_mode == "append":
                k, v = new_cache
        shared_kv[layer_type] = (k, v)
    out = attention_core(q, k, v, qk_mask, dtype)
    proj = matmul(out.reshape(B, S, R * H * D), p.o_proj.reshape(R * H * D, M), dtype)
    return proj, new_cache


def forward_mlp(p: MLPParams, x: np.ndarray, dtype: str) -> np.ndarray:
    """model.py:393-396: ``down(gelu_tanh(gate(x)) * up(x))``."""

    g = matmul(x, p.gate_proj, dtype)
    u = matmul(x, p.up_proj, dtype)
    h = cast(gelu_tanh(g) * u, dtype) if dtype == BF16 else gelu_tanh(g, exact_f32(dtype)) * u
    return matmul(h, p.down_proj, dtype)


def forward_per_layer_inputs(params: Params, cfg: Config, ids: np.ndarray, embeds: np.ndarray, dtype: str):
    """model.py:414-426."""

    P = cfg.hidden_size_per_layer_input
    token = params.embed_tokens_per_layer[ids]  # [B,S,L,P]
    token = cast(token * cast(np.float32(math.sqrt(P)), dtype), dtype)
    B, S, M = embeds.shape
    L = cfg.num_hidden_layers
    ctx = matmul(embeds, params.per_layer_model_projection.reshape(M, L * P), dtype).reshape(B, S, L, P)
    ctx = scale(ctx, cfg.hidden_size**-0.5, dtype)
    ctx = rms_norm(params.per_layer_projection_norm, ctx, cfg.rms_norm_eps, dtype)
    return scale(cast(ctx + token, dtype), 2.0**-0.5, dtype)


def forward_decoder_layer(lp: LayerParams, seq, pli, masks, rots, *, layer_index, cfg, shared_kv, layer_cache,
                          cache_length, cache_mode, dtype):
    """model.py:505-554."""

    lt = cfg.layer_types[layer_index]
    eps = cfg.rms_norm_eps
    residual = seq
    h = rms_norm(lp.input_norm, seq, eps, dtype)
    h, new_cache = forward_attention(
        lp.attention, h, masks[lt], rots[lt], layer_index=layer_index, cfg=cfg, shared_kv=shared_kv,
        layer_cache=layer_cache, cache_length=cache_length, cache_mode=cache_mode, dtype=dtype,
    )
    h = rms_norm(lp.post_attention_norm, h, eps, dtype)
    seq = cast(residual + h, dtype)
    residual = seq
    h = rms_norm(lp.pre_feedforward_norm, seq, eps, dtype)
    h = forward_mlp(lp.mlp, h, dtype)
    h = rms_norm(lp.post_feedforward_norm, h, eps, dtype)
    seq = cast(residual + h, dtype)
    if lp.per_layer_input is not None:
        g = matmul(seq, lp.per_layer_input.gate, dtype)
        g = cast(gelu_tanh(g, exact_f32(dtype)) * pli, dtype)
        g = matmul(g, lp.per_layer_input.projection, dtype)
        g = rms_norm(lp.per_layer_input.post_norm, g, eps, dtype)
        seq = cast(seq + g, dtype)
    return cast(seq * np.float32(lp.layer_scalar), dtype), new_cache


def forward_text(params: Params, ids, position_ids, *, cfg: Config, attention_mask=None, kv_cache: KVCache | None = None,
                 cache_mode: str = "prefill", dtype: str = F32, layer_outputs: list | None = None):
    """model.py:571-673 (per-row cache positions are not needed here: the reference's scalar
    ``length`` applies to every row)."""

    B, S = ids.shape
    if attention_mask is None:
        attention_mask = np.ones((B, S), bool)
    attention_mask = attention_mask.astype(bool)
    x = params.embed_tokens[ids]
    x = cast(x * cast(np.float32(math.sqrt(cfg.hidden_size)), dtype), dtype)
    pli = forward_per_layer_inputs(params, cfg, ids, x, dtype) if cfg.hidden_size_per_layer_input else None
    if kv_cache is None:
        key_mask = attention_mask
        cache_length = None
    else:
        key_mask = kv_cache.key_mask.copy()
        start = min(max(kv_cache.length, 0), key_mask.shape[1] - S)  # lax.dynamic_update_slice clamps (model.py:602)
        key_mask[:, start:start + S] = attention_mask
        cache_length = kv_cache.length
    if kv_cache is not None and cache_mode == "append":
        if S != 1:
            raise ValueError('cache_mode="append" requires one token')
        masks = make_cached_qk_masks(key_mask, cfg.sliding_window, kv_cache.length, S)
    elif kv_cache is not None:
        masks = make_qk_masks(attention_mask, cfg.sliding_window, 0, S)
    else:
        masks = make_qk_masks(key_mask, cfg.sliding_window, 0, S)
    rots = make_rotary(cfg, position_ids, dtype)
    shared: dict = {}
    new_layers = []
    for i, lp in enumerate(params.layers):
        layer_in = pli[:, :, i] if pli is not None else None
        lc = kv_cache.layers[i] if kv_cache is not None else None
        x, nc = forward_decoder_layer(lp, x, layer_in, masks, rots, layer_index=i, cfg=cfg, shared_kv=shared,
                                      layer_cache=lc, cache_length=cache_length, cache_mode=cache_mode, dtype=dtype)
        new_layers.append(nc)
        if layer_outputs is not None:
            layer_outputs.append(x)
    hidden = rms_norm(params.final_norm, x, cfg.rms_norm_eps, dtype)
    if kv_cache is None:
        return hidden, None
    return hidden, KVCache(tuple(new_layers), key_mask, kv_cache.length + S)


def lm_head(embed: np.ndarray, hidden: np.ndarray, softcap: float | None, dtype: str) -> np.ndarray:
    """model.py:676-680: tied-embedding logits, ``tanh(x / cap) * cap``."""

    logits = matmul(hidden, embed.T, dtype)
    if softcap is not None:
        if exact_f32(dtype):
            logits = _f32(np.tanh((logits / np.float32(softcap)).astype(np.float64))) * np.float32(softcap)
        else:
            logits = cast(np.tanh(logits / np.float32(softcap)) * np.float32(softcap), dtype)
    return logits


def forward_lm(params: Params, ids, position_ids, *, cfg: Config, attention_mask=None, kv_cache=None,
               cache_mode="prefill", logits_to_keep: int = 0, dtype: str = F32):
    """model.py:683-709 -> ``(logits, hidden, cache)``."""

    hidden, cache = forward_text(params, ids, position_ids, cfg=cfg, attention_mask=attention_mask,
                                 kv_cache=kv_cache, cache_mode=cache_mode, dtype=dtype)
    head_in = hidden[:, -logits_to_keep:] if logits_to_keep > 0 else hidden
    return lm_head(params.embed_tokens, head_in, cfg.final_logit_softcapping, dtype), hidden, cache


# --- sampler (sampler.py:30-322) ----------------------------------------------------------------


class SamplerConfig(NamedTuple):
    """sampler.py:30-44."""

    max_prompt_len: int
    max_new_tokens: int
    temperature: float = 1.0
    top_k: int = 0
    eos_ids: tuple = ()
    seed: int = 0
    top_p: float = 1.0


class RolloutBatch(NamedTuple):
    """sampler.py:47-52."""

    prompt_ids: np.ndarray
    completion_ids: np.ndarray
    completion_mask: np.ndarray
    rollout_logps: np.ndarray
    lengths: np.ndarray


def position_ids(mask: np.ndarray) -> np.ndarray:
    """sampler.py:63-67: ``max(cumsum(mask) - 1, 0)``."""

    return np.maximum(np.cumsum(mask.astype(np.int32), axis=-1) - 1, 0).astype(np.int32)


def prefill(params, cfg, prompt_ids, prompt_mask, *, max_new_tokens: int, dtype: str = F32):
    """sampler.py:70-106: cache capacity ``P + N``; prefill-mode forward; last-position logits."""

    if prompt_ids.ndim != 2 or prompt_mask.shape != prompt_ids.shape:
        raise ValueError("prompt ids/mask must have the same [B, P] shape")
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be non-negative")
    B, P = prompt_ids.shape
    cache = init_kv_cache(cfg, B, P + max_new_tokens, dtype)
    return forward_lm(params, prompt_ids, position_ids(prompt_mask), cfg=cfg, attention_mask=prompt_mask,
                      kv_cache=cache, cache_mode="prefill", logits_to_keep=1, dtype=dtype)


def decode_step(params, cfg, token_ids, pos_ids, cache: KVCache, *, attention_mask=None, dtype: str = F32):
    """sampler.py:109-142: one-token append forward."""

    if token_ids.ndim != 1 or pos_ids.shape != token_ids.shape:
        raise ValueError("token/position must have the same [B] shape")
    if attention_mask is None:
        attention_mask = np.ones(token_ids.shape, bool)
    return forward_lm(params, token_ids[:, None], pos_ids[:, None], cfg=cfg, attention_mask=attention_mask[:, None],
                      kv_cache=cache, cache_mode="append", logits_to_keep=1, dtype=dtype)


def log_softmax_f32(logits: np.ndarray) -> np.ndarray:
    """sampler.py:151-159: f32 ``shifted - log(sum(exp(shifted)))``."""

    x = logits.astype(np.float32)
    shifted = x - x.max(axis=-1, keepdims=True)
    return (shifted - np.log(np.exp(shifted).sum(axis=-1, keepdims=True, dtype=np.float32))).astype(np.float32)


def sample_token(logits: np.ndarray, *, temperature: float, top_k: int = 0, top_p: float = 1.0, key=None):
    """sampler.py:145-183: greedy argmax, or ``jax.random.categorical(key, scores)`` over the
    temperature-scaled, top-k / top-p truncated scores (noise drawn with the scores' shape, from
    oracle/jax_random.py). The recorded logp is always the full unmodified f32 policy's."""

    x = logits.astype(np.float32)
    full = log_softmax_f32(x)
    V = x.shape[-1]
    if temperature <= 0:
        token = np.argmax(x, axis=-1).astype(np.int32)
    else:
        scores = x / np.float32(temperature)
        order = None
        if 0 < top_k < V:
            order = np.argsort(-scores, axis=-1, kind="stable")[:, :top_k]
            scores = np.take_along_axis(scores, order, axis=-1)
        elif top_p < 1:
            order = np.argsort(-scores, axis=-1, kind="stable")
            scores = np.take_along_axis(scores, order, axis=-1)
        if top_p < 1:
            w = np.exp(scores - scores.max(axis=-1, keepdims=True))
            probs = w / w.sum(axis=-1, keepdims=True)
            prev = np.concatenate([np.zeros_like(probs[:, :1]), np.cumsum(probs, axis=-1)[:, :-1]], axis=-1)
            keep = (prev < top_p) | (np.arange(scores.shape[-1])[None, :] == 0)
            scores = np.where(keep, scores, -np.inf)
        if key is None:
            raise ValueError("sampling with temperature > 0 needs a key")
        sel = JR.categorical(key, scores.astype(np.float32))
        token = sel if order is None else np.take_along_axis(order, sel[:, None], axis=-1)[:, 0].astype(np.int32)
    logp = np.take_along_axis(full, token[:, None].astype(np.int64), axis=-1)[:, 0]
    return token, logp


def generate(params, cfg, prompt_ids, prompt_mask, *, sampler_config: SamplerConfig, dtype: str = F32,
             key=None, step_hook=None) -> RolloutBatch:
    """sampler.py:204-322: prefill, then up to N sample/append steps with early exit once every
    row emitted EOS. ``key`` (uint32 [2], default ``PRNGKey(seed)``) is split once per step
    (sampler.py:265); ``step_hook(step, logits, cache)`` observes the per-step state."""

    sc = sampler_config
    if prompt_ids.shape[1] != sc.max_prompt_len:
        raise ValueError("prompt width does not match max_prompt_len")
    if sc.max_prompt_len <= 0 or sc.max_new_tokens <= 0:
        raise ValueError("max_prompt_len and max_new_tokens must both be positive")
    if sc.top_k > cfg.vocab_size:  # sampler.py:219-220
        raise ValueError(f"top_k={sc.top_k} exceeds vocab_size={cfg.vocab_size}")
    if not math.isfinite(sc.temperature):  # sampler.py:221-222
        raise ValueError("temperature must be finite")
    if not math.isfinite(sc.top_p) or not 0 < sc.top_p <= 1:
        raise ValueError("top_p must be finite and in (0, 1]")
    prompt_mask = prompt_mask.astype(bool)
    logits, _, cache = prefill(params, cfg, prompt_ids, prompt_mask, max_new_tokens=sc.max_new_tokens, dtype=dtype)
    B = prompt_ids.shape[0]
    N = sc.max_new_tokens
    prompt_len = prompt_mask.sum(axis=-1).astype(np.int32)
    active = np.ones(B, bool)
    ids = np.full((B, N), cfg.pad_token_id, np.int32)
    cmask = np.zeros((B, N), bool)
    logps = np.zeros((B, N), np.float32)
    cur = logits[:, -1].astype(np.float32)
    key = JR.prng_key(sc.seed) if key is None else np.asarray(key, np.uint32)
    step = 0
    while step < N and active.any():
        if step_hook is not None:
            step_hook(step, cur, cache)
        key, sample_key = JR.split(key)
        tok, lp = sample_token(cur, temperature=sc.temperature, top_k=sc.top_k, top_p=sc.top_p, key=sample_key)
        tok = np.where(active, tok, cfg.pad_token_id).astype(np.int32)
        lp = np.where(active, lp, 0.0).astype(np.float32)
        ids[:, step], cmask[:, step], logps[:, step] = tok, active, lp
        nxt = active & ~np.isin(tok, np.asarray(sc.eos_ids, np.int32))
        if step + 1 < N and nxt.any():
            out, _, cache = decode_step(params, cfg, tok, prompt_len + step, cache, attention_mask=active, dtype=dtype)
            cur = out[:, -1].astype(np.float32)
        active = nxt
        step += 1
    return RolloutBatch(prompt_ids, ids, cmask, logps, cmask.sum(axis=-1).astype(np.int32))
