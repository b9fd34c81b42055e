"""BASELINE configs 3 and 4 at their full sizes against the oracle (the kernels run at full size;
the oracle checks every row of config 3 and a subset of (b, kv head) pairs of config 4).

configs[2] (config 3): global-layer decode over a linear cache of capacity 32768, B16, Hq8/Hkv2,
D256 bf16, per-row lengths U[1024, 32768], each step appending one token (the fused append) and
attending over the whole valid prefix (model.py:338-365, 368-390, 496-499): the split-K path.

configs[3] (config 4): chunked prefill of B8 x S4096, Hq8/Hkv2, D256 bf16: the 4096 prompt tokens
appended into a 512-slot ring (only the last 512 stay) and a 4096-slot linear cache, bit-exact
(model.py:368-390), and causal attention for a global and a sliding(512) layer on MFMA
(model.py:320-335, 496-499).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import TOL, attention_rows, cache_to_ref, np_bits, to_np
from oracle import g4_oracle as O

from gemma4_posttrain_jax_amd import kernels
from gemma4_posttrain_jax_amd.kvcache import group_keys, group_values, new_layer_cache, ungroup_keys, ungroup_values

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[full] {msg}", flush=True)


def _bf16_randn(shape, g, device):
    return torch.randn(shape, device=device, generator=g).to(torch.bfloat16)


def test_config3_long_context_decode_full_size(device):
    """B16, C32768, ragged lengths U[1024, 32768]; two steps of append + attend (split-K over
    up to 64 key splits per row). Row 3 is left-padded by 700 tokens; row 9 finished at position
    20000 (later positions are pads). Outputs within 2e-2 of the oracle on every row; the cache
    after the appends equals the oracle's bit for bit."""

    B, H, R, D, C = 16, 2, 4, 256, 32768
    g = torch.Generator(device=device).manual_seed(31)
    rng = np.random.default_rng(31)
    layer = new_layer_cache(B, H, D, C, False, torch.bfloat16, device)
    layer.key.normal_(generator=g)
    layer.value_t.normal_(generator=g)
    steps = 2
    lens = rng.integers(1024, C - steps + 1, B)
    lens[0] = C - steps  # one row reaches the last slot
    key_mask = np.ones((B, C), bool)
    key_mask[3, :700] = False
    key_mask[9, 20000:] = False
    km = torch.from_numpy(key_mask).to(device)
    k_ref, v_ref = cache_to_ref(layer)
    kv = O.LayerKV(k_ref, v_ref)
    with O.inplace_cache_updates():
        for step in range(steps):
            q_pos = (lens + step).astype(np.int32)
            q = _bf16_randn((B, H, R, D), g, device)
            nk, nv = _bf16_randn((B, H, D), g, device), _bf16_randn((B, H, D), g, device)
            out = kernels.decode_attention(layer, q, km, q_pos=torch.from_numpy(q_pos).to(device), window=0,
                                           new_k=nk, new_v=nv)
            kv = O.update_layer_cache(kv, to_np(nk)[:, None], to_np(nv)[:, None], q_pos, False, O.BF16)
            mask = O.make_cached_qk_masks(key_mask, 1 << 30, q_pos, 1)[O.FULL]
            qr = to_np(q).transpose(0, 2, 1, 3)[:, None]
            o32 = O.attention_core(qr, kv.key, kv.value, mask, O.BF16)[:, 0].transpose(0, 2, 1, 3)
            with O.accumulate_f64():
                o64 = O.attention_core(qr, kv.key, kv.value, mask, O.BF16)[:, 0].transpose(0, 2, 1, 3)
            err, n64, bad = attention_rows(to_np(out), o32, o64, TOL[O.BF16])
            _say(f"config 3 step {step}: max |out - oracle| {err:.3g}; rows matching only the f64 oracle {n64}")
            assert bad == 0 and n64 <= 1, f"step {step}: {err} ({n64} rows only near the f64 oracle, {bad} neither)"
    gk, gv = cache_to_ref(layer)  # bf16 values as f32: equal f32 bits = equal bf16 bits
    np.testing.assert_array_equal(gk.view(np.uint32), kv.key.view(np.uint32))
    np.testing.assert_array_equal(gv.view(np.uint32), kv.value.view(np.uint32))


@pytest.fixture(scope="module")
def config4(device):
    B, S, H, R, D = 8, 4096, 2, 4, 256
    g = torch.Generator(device=device).manual_seed(41)
    q = _bf16_randn((B, S, H, R, D), g, device)
    k = _bf16_randn((B, S, H, D), g, device)
    v = _bf16_randn((B, S, H, D), g, device)
    key_mask = np.ones((B, S), bool)
    key_mask[5, :100] = False  # a left-padded prompt
    return dict(B=B, S=S, H=H, R=R, D=D, q=q, k=k, v=v, key_mask=key_mask)


def test_config4_prompt_append_is_bit_exact(config4, device):
    """The 4096-token prompt of every row appended in one call (model.py:368-390): the 512-slot
    ring keeps positions 3584..4095 at slots p mod 512, the linear cache all 4096; the chunk's
    own K / V^T (the prefill attention's input) equal the prompt."""

    c = config4
    B, S, H, D = c["B"], c["S"], c["H"], c["D"]
    ring = new_layer_cache(B, H, D, 512, True, torch.bfloat16, device)
    lin = new_layer_cache(B, H, D, S, False, torch.bfloat16, device)
    k_out = torch.empty((B, H, S // 32, D // 32, 2, 16, 32), dtype=torch.bfloat16, device=device)
    vt_out = torch.empty((B, H, S // 8, D, 8), dtype=torch.bfloat16, device=device)
    kernels.kv_append(ring, c["k"], c["v"], write_pos=0, k_out=k_out, vt_out=vt_out)
    kernels.kv_append(lin, c["k"], c["v"], write_pos=0)
    k, v = to_np(c["k"]), to_np(c["v"])
    zeros = np.zeros((B, 512, H, D), np.float32)
    want_ring = O.update_layer_cache(O.LayerKV(zeros, zeros.copy()), k, v, 0, True, O.BF16)
    gk, gv = cache_to_ref(ring)
    np.testing.assert_array_equal(np_bits(gk, O.BF16), np_bits(want_ring.key, O.BF16))
    np.testing.assert_array_equal(np_bits(gv, O.BF16), np_bits(want_ring.value, O.BF16))
    np.testing.assert_array_equal(np_bits(gk[:, 17], O.BF16), np_bits(k[:, S - 512 + 17], O.BF16))
    zeros = np.zeros((B, S, H, D), np.float32)
    want_lin = O.update_layer_cache(O.LayerKV(zeros, zeros.copy()), k, v, 0, False, O.BF16)
    gk, gv = cache_to_ref(lin)
    np.testing.assert_array_equal(np_bits(gk, O.BF16), np_bits(want_lin.key, O.BF16))
    np.testing.assert_array_equal(np_bits(gv, O.BF16), np_bits(want_lin.value, O.BF16))
    np.testing.assert_array_equal(np_bits(to_np(ungroup_keys(k_out)).transpose(0, 2, 1, 3), O.BF16), np_bits(k, O.BF16))
    np.testing.assert_array_equal(np_bits(to_np(ungroup_values(vt_out)).transpose(0, 2, 1, 3), O.BF16),
                                  np_bits(v, O.BF16))


MAX_F64_ROWS = 4  # of the 16,384 (query, head) rows of a pair


@pytest.mark.parametrize("window", [0, 512])
def test_config4_prefill_attention_full_size(config4, device, window):
    """Causal (global) and sliding(512) attention over the 4096-token prompts of all 8 rows on
    MFMA; the oracle recomputes three (b, kv head) pairs in full (every query row), one of them the
    left-padded row whose first 100 queries have no valid key. N(0, 1) q and k of dimension 256 give
    scores up to ~50, where one bf16 ulp is 0.25: each output row must match the oracle within 2e-2,
    or, where a score sits within f32 rounding of a bf16 boundary, the f64-accumulated oracle
    (gpu_util.attention_rows; at most MAX_F64_ROWS rows per pair)."""

    c = config4
    B, S, H, R, D = c["B"], c["S"], c["H"], c["R"], c["D"]
    kd = group_keys(c["k"].permute(0, 2, 1, 3))  # operand-ordered keys (S is a multiple of 64)
    vtd = group_values(c["v"].permute(0, 2, 1, 3))  # [B, H, S / 8, D, 8]
    km = torch.from_numpy(c["key_mask"]).to(device)
    out = kernels.prefill_attention(c["q"], kd, vtd, km, window=window)
    torch.cuda.synchronize()
    masks = O.make_qk_masks(c["key_mask"], window if window else 1 << 30, 0, S)[O.SLIDING]
    for b, h in ((0, 0), (5, 1), (7, 1)):
        q = to_np(c["q"][b:b + 1, :, h:h + 1]).transpose(0, 1, 3, 2, 4)  # [1, S, R, 1, D]
        k = to_np(c["k"][b:b + 1, :, h:h + 1])
        v = to_np(c["v"][b:b + 1, :, h:h + 1])
        o32 = O.attention_core(q, k, v, masks[b:b + 1], O.BF16)  # [1, S, R, 1, D]
        with O.accumulate_f64():
            o64 = O.attention_core(q, k, v, masks[b:b + 1], O.BF16)
        got = to_np(out[b:b + 1, :, h:h + 1]).transpose(0, 1, 3, 2, 4)
        err, n64, bad = attention_rows(got, o32, o64, TOL[O.BF16])
        _say(f"config 4 window {window} pair ({b}, {h}): max |out - oracle| {err:.3g}; rows matching only the "
             f"f64-accumulated oracle {n64} of {S * R}; rows matching neither {bad}")
        assert bad == 0, f"pair ({b}, {h}): {bad} rows outside 2e-2 of both oracle evaluations"
        assert n64 <= MAX_F64_ROWS, f"pair ({b}, {h}): {n64} rows differ from the f32 oracle"
