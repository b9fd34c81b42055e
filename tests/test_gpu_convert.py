"""GPU parity of the rollout weight handoff (g4_convert_f32_to_bf16 / g4_convert_bf16_to_f32 and
sharding.reshard_for_rollout / reshard_after_rollout / device_converter) with the oracle's
bitwise cast, pinned in tests/test_oracle_convert.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import hf_util as H
from oracle import g4_oracle as O
from test_oracle_convert import boundary_vectors

from gemma4_posttrain_jax_amd import config as C
from gemma4_posttrain_jax_amd import kernels
from gemma4_posttrain_jax_amd import model as M
from gemma4_posttrain_jax_amd import sampler as SMP
from gemma4_posttrain_jax_amd import sharding as SH

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def test_convert_every_encoding_and_boundary(device):
    value = boundary_vectors()
    conv = SH.device_converter("identity", value.shape)
    out, finite = conv(torch.from_numpy(value).to(device))
    np.testing.assert_array_equal(_bits(out), O.bf16_bits(value))
    assert not bool(finite)  # the top boundary overflows to inf, as the reference's test expects
    ok = value[np.abs(value) < 3.0e38]
    out, finite = SH.device_converter("reshape", (ok.size,))(torch.from_numpy(ok).to(device))
    np.testing.assert_array_equal(_bits(out), O.bf16_bits(ok))
    assert bool(finite)


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf, np.finfo(np.float32).max])
@pytest.mark.parametrize("n,at", [(1, 0), (13, 12), (4096, 1000)])
def test_nonfinite_input_or_overflow_is_reported(device, bad, n, at):
    """tests/test_inference_device.py:55-62: inf / NaN inputs and f32 max (overflows bf16)."""

    x = np.random.default_rng(n).standard_normal(n).astype(np.float32)
    x[at] = bad
    _, finite = SH.device_converter("identity", (n,))(torch.from_numpy(x).to(device))
    assert not bool(finite)


@pytest.mark.parametrize("n", [1, 7, 8, 9, 1000, 65543])
def test_ragged_sizes_and_unaligned_views(device, n):
    x = torch.randn(n + 3, device=device) * 100
    for view in (x[:n], x[3:3 + n]):  # the second is not 16-byte aligned (copied by the wrapper)
        out = kernels.convert_f32_to_bf16(view)
        np.testing.assert_array_equal(_bits(out), O.bf16_bits(view.cpu().numpy()))
        back = kernels.convert_bf16_to_f32(out)
        np.testing.assert_array_equal(back.cpu().numpy(), O.from_bf16_bits(_bits(out)))


def test_reshard_round_trip_keeps_master_and_rollout_matches(device):
    """tests/test_rollout_layout.py:19-38 and test_sharding_tpu.py:287-305: the rollout copy is the
    bf16 cast of every leaf, the f32 master is unchanged, the round trip equals bf16 -> f32, and a
    greedy rollout on the resharded tree equals one on a tree built directly in bf16."""

    kw = H.TINY_A
    ocfg = O.config_from_hf(kw)
    host = H.hf_to_params(H.build_hf_model(kw, seed=0), ocfg)
    cfg = C.config_from_hf(kw)
    master = M.params_from_numpy(host, cfg, dtype=torch.float32, device=device)
    before = [t.clone() for t in SH.tree_leaves(master)]
    rollout = SH.reshard_for_rollout(master, cfg, layout="fsdp")
    for leaf, orig in zip(SH.tree_leaves(rollout), before):
        assert leaf.dtype == torch.bfloat16
        np.testing.assert_array_equal(_bits(leaf), O.bf16_bits(orig.cpu().numpy()))
    for leaf, orig in zip(SH.tree_leaves(master), before):
        assert torch.equal(leaf, orig)
    back = SH.reshard_after_rollout(rollout, cfg)
    for leaf, orig in zip(SH.tree_leaves(back), before):
        assert torch.equal(leaf, orig.to(torch.bfloat16).to(torch.float32))
    with pytest.raises(ValueError, match="layout"):
        SH.reshard_for_rollout(master, cfg, layout="unknown")

    # a bf16 rollout (bf16 attention needs head dims >= 32: a small config of the bf16 model tests)
    kw = dict(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=3, num_attention_heads=8,
              num_key_value_heads=2, head_dim=64, global_head_dim=64,
              layer_types=["sliding_attention", "sliding_attention", "full_attention"], sliding_window=8,
              num_kv_shared_layers=0, hidden_size_per_layer_input=0, final_logit_softcapping=30.0)
    ocfg, cfg = O.config_from_hf(kw), C.config_from_hf(kw)
    host = O.init_params(ocfg, seed=5, dtype=O.F32, std=0.03, norm_std=0.05)
    master = M.params_from_numpy(host, cfg, dtype=torch.float32, device=device)
    rollout = SH.reshard_for_rollout(master, cfg)
    direct = M.params_from_numpy(host, cfg, dtype=torch.bfloat16, device=device)
    ids = torch.tensor([[5, 6, 7, 8], [0, 0, 9, 10]], dtype=torch.int32, device=device)
    pm = ids != 0
    sc = SMP.SamplerConfig(4, 6, temperature=0.0)
    a = SMP.generate(rollout, cfg, ids, pm, sampler_config=sc)
    b = SMP.generate(direct, cfg, ids, pm, sampler_config=sc)
    assert torch.equal(a.completion_ids, b.completion_ids) and torch.equal(a.rollout_logps, b.rollout_logps)
