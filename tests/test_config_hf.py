"""``config_from_hf`` on configs as Hugging Face serializes them (CPU only).

The reference's own cases (tests/test_hf_config_roundtrip.py:17-80 of the reference) restated on
the installed transformers' ``Gemma4TextConfig``: its ``to_dict()`` / ``config.json`` carries the
sparse ``per_layer_config`` and drops ``global_head_dim``, which model.py:61-97 turns back into the
two attention types' dimensions.
"""

from __future__ import annotations

import copy
import json

import pytest

from hf_util import TINY_A, TINY_B

from gemma4_posttrain_jax_amd import config as C

transformers = pytest.importorskip("transformers")


def _serialized(kwargs: dict) -> dict:
    return transformers.Gemma4TextConfig(**kwargs).to_dict()


@pytest.mark.parametrize("kwargs", [TINY_A, TINY_B], ids=["tiny_a", "tiny_b"])
def test_hf_serialized_config_parses_like_the_constructor_arguments(kwargs, tmp_path):
    """test_hf_config_roundtrip.py:17-34: a saved config.json (per_layer_config, no
    global_head_dim) gives the config of the dict it was built from, per-layer dims included."""

    transformers.Gemma4TextConfig(**kwargs).save_pretrained(tmp_path)
    saved = json.loads((tmp_path / "config.json").read_text())
    assert "global_head_dim" not in saved and "per_layer_config" in saved
    expected = C.config_from_hf(kwargs)
    parsed = C.config_from_hf(saved)
    assert parsed == expected
    for i in range(parsed.num_hidden_layers):
        assert C.layer_head_dim(parsed, i) == C.layer_head_dim(expected, i)
        assert C.layer_kv_heads(parsed, i) == C.layer_kv_heads(expected, i)
        assert C.layer_has_v_proj(parsed, i) == C.layer_has_v_proj(expected, i)


def test_tiny_configs_resolve_to_the_reference_dimensions():
    """The two fixtures' known per-type dimensions (conftest.py:23-64 of the reference): sliding
    head dim 8, global 16; TINY_B's K=V global layers keep one kv head of their own."""

    a = C.config_from_hf(_serialized(TINY_A))
    assert (a.head_dim, a.global_head_dim, a.num_key_value_heads, a.num_global_key_value_heads) == (8, 16, 2, None)
    b = C.config_from_hf(_serialized(TINY_B))
    assert (b.head_dim, b.global_head_dim, b.num_key_value_heads, b.num_global_key_value_heads) == (8, 16, 2, 1)
    assert [C.layer_kv_heads(b, i) for i in range(6)] == [2, 1, 2, 2, 2, 1]


def test_explicit_layer_configuration_overrides_legacy_global_field():
    """test_hf_config_roundtrip.py:37-43: per_layer_config wins over a stale global_head_dim,
    also inside a composite config's text_config."""

    saved = _serialized(TINY_A)
    saved["global_head_dim"] = 999
    expected = C.config_from_hf(TINY_A)
    assert C.config_from_hf(saved) == expected
    assert C.config_from_hf({"text_config": saved}) == expected


@pytest.mark.parametrize("empty", [{}, None])
def test_explicit_empty_layer_configuration_uses_head_dim_not_legacy_alias(empty):
    """test_hf_config_roundtrip.py:46-52: with an empty override map every layer has head_dim."""

    saved = _serialized(TINY_A)
    saved["per_layer_config"] = empty
    saved["global_head_dim"] = 999
    parsed = C.config_from_hf(saved)
    assert parsed.global_head_dim == parsed.head_dim == saved["head_dim"]
    assert parsed.num_global_key_value_heads is None


@pytest.mark.parametrize("case", ["different_full_width", "unsupported_norm", "index_out_of_range",
                                  "kv_override_without_k_eq_v", "non_canonical_index", "not_a_mapping",
                                  "kv_heads_not_dividing"])
def test_unrepresentable_layer_overrides_fail_closed(case):
    """test_hf_config_roundtrip.py:55-73 (first four cases) and the index / value checks of
    model.py:72-85."""

    saved = copy.deepcopy(_serialized(TINY_A))
    overrides = {str(k): v for k, v in saved["per_layer_config"].items()}
    saved["per_layer_config"] = overrides
    if case == "different_full_width":
        overrides["5"]["head_dim"] = 32
    elif case == "unsupported_norm":
        overrides["1"]["rms_norm_eps"] = 1e-3
    elif case == "index_out_of_range":
        overrides["6"] = {"head_dim": 16}
    elif case == "kv_override_without_k_eq_v":
        for value in overrides.values():
            value["num_key_value_heads"] = 1
    elif case == "non_canonical_index":
        overrides["01"] = overrides.pop("1")
    elif case == "not_a_mapping":
        saved["per_layer_config"] = [overrides["1"]]
    else:
        overrides["1"]["num_key_value_heads"] = 3
    with pytest.raises(ValueError):
        C.config_from_hf(saved)


def test_equal_explicit_global_kv_count_survives_hf_serialization():
    """test_hf_config_roundtrip.py:76-90: a global kv count equal to the sliding one is dropped by
    the sparse serialization; the per-layer dimensions stay the same."""

    legacy = {k: v for k, v in TINY_B.items()}
    legacy["global_head_dim"] = 16
    legacy["num_global_key_value_heads"] = legacy["num_key_value_heads"]
    serialized = _serialized(legacy)
    parsed, expected = C.config_from_hf(serialized), C.config_from_hf(legacy)
    assert parsed == expected._replace(num_global_key_value_heads=None)
    for i in range(parsed.num_hidden_layers):
        assert C.layer_head_dim(parsed, i) == C.layer_head_dim(expected, i)
        assert C.layer_kv_heads(parsed, i) == C.layer_kv_heads(expected, i)
