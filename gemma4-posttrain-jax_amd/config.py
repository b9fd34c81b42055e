"""Static Gemma 4 text-decoder configuration and per-layer derivations.

Same fields and semantics as the reference's ``Gemma4TextConfig`` (model.py:32-58) and
``config_from_hf`` (model.py:100-147), so a config built for the reference builds here too.
The KV-sharing map is computed by the native library (``g4_kv_source_layers``), the single
implementation the host and the tests use.
"""

from __future__ import annotations

from collections.abc import Mapping
from typing import Any, NamedTuple

from . import _lib

SLIDING = "sliding_attention"
FULL = "full_attention"


class Gemma4TextConfig(NamedTuple):
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    global_head_dim: int
    num_global_key_value_heads: int | None
    layer_types: tuple[str, ...]
    sliding_window: int
    num_kv_shared_layers: int
    use_double_wide_mlp: bool
    attention_k_eq_v: bool
    hidden_size_per_layer_input: int
    vocab_size_per_layer_input: int
    rms_norm_eps: float
    rope_theta_sliding: float
    rope_theta_full: float
    full_partial_rotary_factor: float
    final_logit_softcapping: float | None
    bos_token_id: int
    eos_token_id: int
    pad_token_id: int


def _attention_dims(text: Mapping[str, Any], layer_types: list[str]) -> tuple[int, int, int, int | None]:
    """(sliding head dim, global head dim, kv heads, global kv heads) of an HF text config
    (model.py:61-97).

    Without ``per_layer_config`` the legacy fields are read as they are. With it (transformers
    writes the field and drops ``global_head_dim``), every layer starts from ``head_dim`` /
    ``num_key_value_heads`` and takes its sparse override; each attention type must then resolve
    to one (dim, kv heads) pair, and a separate global kv-head count only exists for K=V
    global layers. Anything else cannot be represented by this parameter structure and raises
    ``ValueError``, as the reference does.
    """

    head_dim = int(text.get("head_dim", 256))
    kv_heads = int(text["num_key_value_heads"])
    if "per_layer_config" not in text:
        return head_dim, int(text.get("global_head_dim", 512)), kv_heads, text.get("num_global_key_value_heads")
    raw = text["per_layer_config"]
    if raw is not None and not isinstance(raw, Mapping):
        raise ValueError("per_layer_config must map layer indices to overrides")
    overrides: dict[int, Mapping[str, Any]] = {}
    for key, value in (raw or {}).items():
        index = int(key)
        if str(index) != str(key) or not 0 <= index < len(layer_types) or index in overrides:
            raise ValueError(f"invalid or repeated per_layer_config layer index: {key!r}")
        if not isinstance(value, Mapping) or not set(value) <= {"head_dim", "num_key_value_heads"}:
            raise ValueError(f"unsupported per_layer_config override for layer {index}: {value!r}")
        overrides[index] = value
    q_heads = int(text["num_attention_heads"])
    per_type: dict[str, set[tuple[int, int]]] = {SLIDING: set(), FULL: set()}
    for index, layer_type in enumerate(layer_types):
        override = overrides.get(index, {})
        dims = (int(override.get("head_dim", head_dim)), int(override.get("num_key_value_heads", kv_heads)))
        if dims[0] <= 0 or dims[1] <= 0 or q_heads % dims[1]:
            raise ValueError(f"layer {index}: head dim and kv heads must be positive, kv heads dividing {q_heads}")
        per_type[layer_type].add(dims)
    if len(per_type[SLIDING]) > 1 or len(per_type[FULL]) > 1:
        raise ValueError("layers of one attention type have different dimensions, which these parameters cannot hold")
    sliding_dim, sliding_kv = min(per_type[SLIDING], default=(head_dim, kv_heads))
    global_dim, global_kv = min(per_type[FULL], default=(head_dim, kv_heads))
    if global_kv != sliding_kv and not text.get("attention_k_eq_v", False):
        raise ValueError("a separate global kv-head count needs K=V global attention (attention_k_eq_v)")
    return sliding_dim, global_dim, sliding_kv, (global_kv if global_kv != sliding_kv else None)


def config_from_hf(hf: Mapping[str, Any]) -> Gemma4TextConfig:
    """model.py:100-147: a composite or text-only HF ``config.json`` dict, legacy global-attention
    fields or the sparse ``per_layer_config`` of transformers' serialization (model.py:61-97);
    the last layer is forced FULL (line 112)."""

    text = hf.get("text_config", hf)
    num_layers = int(text["num_hidden_layers"])
    layer_types = list(text["layer_types"])
    if len(layer_types) != num_layers:
        raise ValueError(f"layer_types has {len(layer_types)} entries for {num_layers} layers")
    layer_types[-1] = FULL
    head_dim, global_head_dim, kv_heads, global_kv_heads = _attention_dims(text, layer_types)
    rope = text.get("rope_parameters") or {}
    sliding_rope = rope.get(SLIDING) or {}
    full_rope = rope.get(FULL) or {}
    if sliding_rope.get("rope_type", "default") != "default" or full_rope.get("rope_type", "proportional") != "proportional":
        raise ValueError(f"unsupported rope_parameters: {rope}")
    return Gemma4TextConfig(
        vocab_size=int(text["vocab_size"]),
        hidden_size=int(text["hidden_size"]),
        intermediate_size=int(text["intermediate_size"]),
        num_hidden_layers=num_layers,
        num_attention_heads=int(text["num_attention_heads"]),
        num_key_value_heads=kv_heads,
        head_dim=head_dim,
        global_head_dim=global_head_dim,
        num_global_key_value_heads=global_kv_heads,
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


def is_kv_shared(config: Gemma4TextConfig, layer_index: int) -> bool:
    """model.py:153-155."""

    first_shared = config.num_hidden_layers - config.num_kv_shared_layers
    return config.num_kv_shared_layers > 0 and layer_index >= first_shared


def kv_source_layers(config: Gemma4TextConfig) -> list[int]:
    """model.py:158-168 for every layer, from the native ``g4_kv_source_layers``."""

    types = [1 if t == FULL else 0 for t in config.layer_types]
    return _lib.kv_source_layers(types, config.num_kv_shared_layers)


def kv_source_layer(config: Gemma4TextConfig, layer_index: int) -> int:
    """model.py:158-168: index of the last non-shared layer of the same type."""

    return kv_source_layers(config)[layer_index]


def layer_head_dim(config: Gemma4TextConfig, layer_index: int) -> int:
    """model.py:171-172."""

    return config.global_head_dim if config.layer_types[layer_index] == FULL else config.head_dim


def layer_kv_heads(config: Gemma4TextConfig, layer_index: int) -> int:
    """model.py:175-178."""

    if config.layer_types[layer_index] == FULL and config.attention_k_eq_v and config.num_global_key_value_heads:
        return int(config.num_global_key_value_heads)
    return config.num_key_value_heads


def layer_has_v_proj(config: Gemma4TextConfig, layer_index: int) -> bool:
    """model.py:181-182."""

    return not (config.attention_k_eq_v and config.layer_types[layer_index] == FULL)


def layer_intermediate_size(config: Gemma4TextConfig, layer_index: int) -> int:
    """model.py:185-187."""

    double = config.use_double_wide_mlp and is_kv_shared(config, layer_index)
    return config.intermediate_size * (2 if double else 1)
