"""GPU parity of the three kernels against the oracle, through the C ABI.

Bars: cache contents after append are bit-exact (pure data movement, and RoPE with the oracle's
op order); attention outputs are within max-abs 2e-2 (bf16) / 1e-5 (fp32).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_util import TOL, bits, cache_to_ref, np_bits, ref_to_cache, to_dev, to_np
from oracle import g4_oracle as O

from gemma4_posttrain_jax_amd import _lib, kernels
from gemma4_posttrain_jax_amd.kvcache import group_keys, group_values, new_layer_cache, ungroup_keys, ungroup_values

pytestmark = pytest.mark.gpu


def _rand(rng, shape, dtype):
    return O.cast(rng.standard_normal(shape, dtype=np.float32), dtype)


# --- append ---------------------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
@pytest.mark.parametrize("ring", [True, False])
@pytest.mark.parametrize("S", [1, 5, 40])
def test_append_is_bit_exact(device, dtype, ring, S):
    """_update_layer_cache (model.py:368-390): per-row start positions, chunks longer than the ring."""

    rng = np.random.default_rng(S + 10 * ring)
    B, H, D = 3, 2, 64
    cap = 16 if ring else 64
    layer = new_layer_cache(B, H, D, cap, ring, __import__("gpu_util").TORCH_DTYPE[dtype], device)
    k0, v0 = _rand(rng, (B, cap, H, D), dtype), _rand(rng, (B, cap, H, D), dtype)
    ref_to_cache(layer, k0, v0, dtype)
    k, v = _rand(rng, (B, S, H, D), dtype), _rand(rng, (B, S, H, D), dtype)
    starts = rng.integers(0, 50 if ring else cap - S + 1, B).astype(np.int32)
    kernels.kv_append(layer, to_dev(k, dtype, device), to_dev(v, dtype, device),
                      write_pos=torch.from_numpy(starts).to(device))
    ref = O.update_layer_cache(O.LayerKV(k0, v0), k, v, starts, ring, dtype)
    gk, gv = cache_to_ref(layer)
    np.testing.assert_array_equal(np_bits(gk, dtype), np_bits(ref.key, dtype))
    np.testing.assert_array_equal(np_bits(gv, dtype), np_bits(ref.value, dtype))
    # scalar start (the reference's single `length`)
    kernels.kv_append(layer, to_dev(k, dtype, device), to_dev(v, dtype, device), write_pos=int(starts[0]))
    ref = O.update_layer_cache(ref, k, v, int(starts[0]), ring, dtype)
    gk, gv = cache_to_ref(layer)
    np.testing.assert_array_equal(np_bits(gk, dtype), np_bits(ref.key, dtype))
    np.testing.assert_array_equal(np_bits(gv, dtype), np_bits(ref.value, dtype))


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
@pytest.mark.parametrize("D", [64, 256])
def test_append_fused_rope_is_bit_exact(device, dtype, D):
    """RoPE'd K append (model.py:309-317 + 368-390) with the oracle's rounding order."""

    rng = np.random.default_rng(D)
    B, S, H, cap = 2, 7, 2, 32
    layer = new_layer_cache(B, H, D, cap, False, __import__("gpu_util").TORCH_DTYPE[dtype], device)
    k, v = _rand(rng, (B, S, H, D), dtype), _rand(rng, (B, S, H, D), dtype)
    pos = rng.integers(0, 5000, (B, S)).astype(np.int32)
    inv = O.rope_inv_freq(O.config_from_hf(dict(
        vocab_size=8, hidden_size=8, intermediate_size=8, num_hidden_layers=1, num_attention_heads=2,
        num_key_value_heads=1, head_dim=D, global_head_dim=D, layer_types=["sliding_attention"])))[O.FULL]
    cos, sin = O.rotary_values(inv, pos)
    kernels.kv_append(layer, to_dev(k, dtype, device), to_dev(v, dtype, device), write_pos=3,
                      flags=_lib.G4_APPEND_ROPE_K, rope_cos=torch.from_numpy(cos).to(device),
                      rope_sin=torch.from_numpy(sin).to(device))
    ref = O.update_layer_cache(O.LayerKV(np.zeros((B, cap, H, D), np.float32), np.zeros((B, cap, H, D), np.float32)),
                               O.rope(k, cos, sin, dtype), v, 3, False, dtype)
    gk, gv = cache_to_ref(layer)
    np.testing.assert_array_equal(np_bits(gk, dtype), np_bits(ref.key, dtype))
    np.testing.assert_array_equal(np_bits(gv, dtype), np_bits(ref.value, dtype))


@pytest.mark.parametrize("dtype,D", [(O.BF16, 128), (O.F32, 128), (O.BF16, 512)])
def test_append_with_norms_and_q_matches_oracle(device, dtype, D):
    """q/k norm + RoPE, unscaled v norm, prefill chunk outputs (model.py:463-482); also at head dim
    512 (the reference's default global head dim)."""

    rng = np.random.default_rng(3)
    B, S, H, R, cap = 2, 9, 2, 4, 64
    width = (H * R + 2 * H) * D
    rows = _rand(rng, (B, S, width), dtype)
    qn, kn = O.cast(1 + 0.3 * rng.standard_normal(D), dtype), O.cast(1 + 0.3 * rng.standard_normal(D), dtype)
    pos = np.tile(np.arange(S, dtype=np.int32), (B, 1))
    cos, sin = O.rotary_values(np.float32(1) / np.power(np.float32(1e4), np.arange(0, D, 2, dtype=np.float32) / D), pos)
    layer = new_layer_cache(B, H, D, cap, True, __import__("gpu_util").TORCH_DTYPE[dtype], device)
    rows_d = to_dev(rows, dtype, device)
    q = rows_d[:, :, : H * R * D].view(B, S, H, R, D)
    k = rows_d[:, :, H * R * D: (H * R + H) * D].view(B, S, H, D)
    v = rows_d[:, :, (H * R + H) * D:].view(B, S, H, D)
    q_out = torch.empty((B, S, H, R, D), dtype=q.dtype, device=device)
    k_out = torch.empty((B, H, 2, D // 32, 2, 16, 32), dtype=q.dtype, device=device)
    vt_out = torch.empty((B, H, 8, D, 8), dtype=q.dtype, device=device)
    flags = (_lib.G4_APPEND_NORM_Q | _lib.G4_APPEND_ROPE_Q | _lib.G4_APPEND_NORM_K | _lib.G4_APPEND_ROPE_K
             | _lib.G4_APPEND_NORM_V)
    kernels.kv_append(layer, k, v, write_pos=0, flags=flags, eps=1e-6, q=q, q_out=q_out,
                      q_norm_weight=to_dev(qn, dtype, device), k_norm_weight=to_dev(kn, dtype, device),
                      rope_cos=torch.from_numpy(cos).to(device), rope_sin=torch.from_numpy(sin).to(device),
                      k_out=k_out, vt_out=vt_out)
    qr = rows[:, :, : H * R * D].reshape(B, S, H, R, D)
    kr = rows[:, :, H * R * D: (H * R + H) * D].reshape(B, S, H, D)
    vr = rows[:, :, (H * R + H) * D:].reshape(B, S, H, D)
    q_ref = O.rope(O.rms_norm(qn, qr, 1e-6, dtype), cos, sin, dtype)
    k_ref = O.rope(O.rms_norm(kn, kr, 1e-6, dtype), cos, sin, dtype)
    v_ref = O.rms_norm(None, vr, 1e-6, dtype)
    tol = TOL[dtype]
    np.testing.assert_allclose(to_np(q_out), q_ref, atol=tol, rtol=0)
    np.testing.assert_allclose(to_np(ungroup_keys(k_out)[:, :, :S]).transpose(0, 2, 1, 3), k_ref, atol=tol, rtol=0)
    np.testing.assert_allclose(to_np(ungroup_values(vt_out)[:, :, :S]).transpose(0, 2, 1, 3), v_ref, atol=tol, rtol=0)
    ref = O.update_layer_cache(O.LayerKV(np.zeros((B, cap, H, D), np.float32), np.zeros((B, cap, H, D), np.float32)),
                               k_ref, v_ref, 0, True, dtype)
    gk, gv = cache_to_ref(layer)
    np.testing.assert_allclose(gk, ref.key, atol=tol, rtol=0)
    np.testing.assert_allclose(gv, ref.value, atol=tol, rtol=0)


@pytest.mark.parametrize("D", [128, 256, 512])
@pytest.mark.parametrize("ring", [True, False])
def test_append_tiles_match_token_by_token_appends(device, D, ring):
    """Prefill-sized bf16 appends (8 tokens per workgroup, V staged in LDS and stored as whole 16-byte
    pieces where the 8 slots form one aligned group) against the same chunk appended one token at a
    time (the one-token kernel): every cache element, chunk output and prepared q bit for bit. Rows
    start on and off an 8-slot boundary; the ring's chunk is longer than the ring; S = 37 leaves a
    partial last tile."""

    rng = np.random.default_rng(D + ring)
    dtype = O.BF16
    B, S, H, R = 4, 37, 2, 4
    cap = 32 if ring else 96
    starts = np.array([0, 8, 5, 43] if ring else [0, 8, 3, 40], np.int32)
    width = (H * R + 2 * H) * D
    rows = to_dev(_rand(rng, (B, S, width), dtype), dtype, device)
    qn = to_dev(O.cast(1 + 0.3 * rng.standard_normal(D), dtype), dtype, device)
    kn = to_dev(O.cast(1 + 0.3 * rng.standard_normal(D), dtype), dtype, device)
    pos = starts[:, None] + np.arange(S, dtype=np.int32)[None, :]
    cos, sin = O.rotary_values(np.float32(1) / np.power(np.float32(1e4), np.arange(0, D, 2, dtype=np.float32) / D), pos)
    cos_d, sin_d = torch.from_numpy(cos).to(device), torch.from_numpy(sin).to(device)
    flags = (_lib.G4_APPEND_NORM_Q | _lib.G4_APPEND_ROPE_Q | _lib.G4_APPEND_NORM_K | _lib.G4_APPEND_ROPE_K
             | _lib.G4_APPEND_NORM_V)
    q = rows[:, :, : H * R * D].view(B, S, H, R, D)
    k = rows[:, :, H * R * D: (H * R + H) * D].view(B, S, H, D)
    v = rows[:, :, (H * R + H) * D:].view(B, S, H, D)
    td = torch.bfloat16
    wp = torch.from_numpy(starts).to(device)

    tiled = new_layer_cache(B, H, D, cap, ring, td, device)
    q_out = torch.empty((B, S, H, R, D), dtype=td, device=device)
    k_out = torch.empty((B, H, 2, D // 32, 2, 16, 32), dtype=td, device=device)  # 64 chunk slots
    vt_out = torch.zeros((B, H, 8, D, 8), dtype=td, device=device)
    kernels.kv_append(tiled, k, v, write_pos=wp, flags=flags, eps=1e-6, q=q, q_out=q_out, q_norm_weight=qn,
                      k_norm_weight=kn, rope_cos=cos_d, rope_sin=sin_d, k_out=k_out, vt_out=vt_out)

    single = new_layer_cache(B, H, D, cap, ring, td, device)
    chunk = new_layer_cache(B, H, D, 64, False, td, device)  # token s at slot s: the chunk outputs' layout
    q_one = torch.empty((B, S, H, R, D), dtype=td, device=device)
    for s in range(S):
        qs = torch.empty((B, 1, H, R, D), dtype=td, device=device)
        args = dict(flags=flags, eps=1e-6, q=q[:, s:s + 1], q_out=qs, q_norm_weight=qn, k_norm_weight=kn,
                    rope_cos=cos_d[:, s:s + 1].contiguous(), rope_sin=sin_d[:, s:s + 1].contiguous())
        if not ring or s >= S - cap:  # a ring keeps the chunk's last `cap` tokens
            kernels.kv_append(single, k[:, s:s + 1], v[:, s:s + 1], write_pos=wp + s, **args)
        kernels.kv_append(chunk, k[:, s:s + 1], v[:, s:s + 1], write_pos=s, **args)
        q_one[:, s:s + 1] = qs
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(q_out), bits(q_one))
    np.testing.assert_array_equal(bits(tiled.key), bits(single.key))
    np.testing.assert_array_equal(bits(tiled.value_t), bits(single.value_t))
    np.testing.assert_array_equal(bits(ungroup_keys(k_out)[:, :, :S]), bits(ungroup_keys(chunk.key)[:, :, :S]))
    np.testing.assert_array_equal(bits(ungroup_values(vt_out)[:, :, :S]), bits(ungroup_values(chunk.value_t)[:, :, :S]))


# --- decode attention -----------------------------------------------------------------------------


def _attention_ref(q, k, v, mask, dtype):
    """The oracle's attention core (model.py:496-499). fp32: with f64-accumulated products, as the
    f32 kernels compute them (the exactly rounded dot products); bf16: f32 accumulation."""

    if dtype == O.F32:
        with O.accumulate_f64():
            return O.attention_core(q, k, v, mask, dtype)
    return O.attention_core(q, k, v, mask, dtype)


def _decode_case(device, dtype, *, B, H, R, D, cap, ring, window, q_pos, key_mask, fused, seed, num_splits=0):
    rng = np.random.default_rng(seed)
    td = __import__("gpu_util").TORCH_DTYPE[dtype]
    layer = new_layer_cache(B, H, D, cap, ring, td, device)
    k0, v0 = _rand(rng, (B, cap, H, D), dtype), _rand(rng, (B, cap, H, D), dtype)
    ref_to_cache(layer, k0, v0, dtype)
    q = _rand(rng, (B, H, R, D), dtype)
    nk, nv = _rand(rng, (B, H, D), dtype), _rand(rng, (B, H, D), dtype)
    qp = torch.from_numpy(q_pos.astype(np.int32)).to(device)
    km = torch.from_numpy(key_mask).to(device)
    if fused:
        out = kernels.decode_attention(layer, to_dev(q, dtype, device), km, q_pos=qp, window=window,
                                       new_k=to_dev(nk, dtype, device), new_v=to_dev(nv, dtype, device),
                                       num_splits=num_splits)
        ref_kv = O.update_layer_cache(O.LayerKV(k0, v0), nk[:, None], nv[:, None], q_pos, ring, dtype)
    else:
        out = kernels.decode_attention(layer, to_dev(q, dtype, device), km, q_pos=qp, window=window,
                                       num_splits=num_splits)
        ref_kv = O.LayerKV(k0, v0)
    masks = O.make_cached_qk_masks(key_mask, window if ring else 1 << 30, q_pos, 1)
    mask = masks[O.SLIDING] if ring else masks[O.FULL]
    q_ref = q.transpose(0, 2, 1, 3)[:, None]  # [B, 1, R, H, D]
    o_ref = _attention_ref(q_ref, ref_kv.key, ref_kv.value, mask, dtype)[:, 0].transpose(0, 2, 1, 3)
    got = to_np(out)
    err = np.abs(got - o_ref).max()
    assert err <= TOL[dtype], f"max |out - oracle| = {err}"
    if fused:
        gk, gv = cache_to_ref(layer)
        np.testing.assert_array_equal(np_bits(gk, dtype), np_bits(ref_kv.key, dtype))
        np.testing.assert_array_equal(np_bits(gv, dtype), np_bits(ref_kv.value, dtype))
    return err


@pytest.mark.parametrize("fused,num_splits", [(False, 0), (True, 0), (True, 1), (True, 2),
                                               (False, _lib.G4_DECODE_TWO_PASS), (True, _lib.G4_DECODE_TWO_PASS)])
def test_decode_ring_config2_shape(device, fused, num_splits):
    """B64, Hq8/Hkv2, D256, W512 ring that has wrapped several times;
    per-row write positions U[1536, 2048). num_splits 1/2: one or two workgroups per (b, kv head);
    G4_DECODE_TWO_PASS: scores and values in two launches."""

    rng = np.random.default_rng(2)
    B, H, R, D, W = 64, 2, 4, 256, 512
    q_pos = rng.integers(1536, 2048, B)
    key_mask = np.ones((B, 2048), bool)
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=W, ring=True, window=W, q_pos=q_pos, key_mask=key_mask,
                 fused=fused, seed=20, num_splits=num_splits)


@pytest.mark.parametrize("D,num_splits", [(128, 1), (256, 1), (256, 2)])
def test_decode_linear_long_rows(device, D, num_splits):
    """Rows longer than one round of chunks (capacity 768, the E2B global-layer cache): the
    appended slot falls in the first round for some rows and in later rounds for others;
    batch*heads not a multiple of 8 (padding workgroups of the two-split grid); a fully masked
    row; rows shorter than one round."""

    rng = np.random.default_rng(7)
    B, H, R, C = 5, 3, 4, 768
    q_pos = np.array([767, 600, 100, 20, 700])
    key_mask = np.ones((B, C), bool)
    key_mask[1, :40] = False
    key_mask[4, :] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=C, ring=False, window=0, q_pos=q_pos, key_mask=key_mask,
                 fused=True, seed=23, num_splits=num_splits)


@pytest.mark.parametrize("ring,cap,num_splits", [(True, 512, 0), (False, 768, 0), (True, 512, 2), (False, 768, 2)])
def test_decode_e2b_batch(device, ring, cap, num_splits):
    """The E2B decode shape the rollout runs: B256 x Hkv2 = 512 pairs, ring 512 (sliding layers)
    and linear 768 (global layers), ragged write positions, a left-padded row, a finished row.
    num_splits 0: the library's choice (two launches at this many pairs); 2: one launch."""

    rng = np.random.default_rng(11)
    B, H, R, D = 256, 2, 4, 256
    C = 768
    q_pos = rng.integers(300, 767, B)
    key_mask = np.ones((B, C), bool)
    key_mask[3, :50] = False
    key_mask[7, 400:] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=cap, ring=ring, window=512 if ring else 0, q_pos=q_pos,
                 key_mask=key_mask, fused=True, seed=26, num_splits=num_splits)


@pytest.mark.parametrize("D", [128, 256, 512])
@pytest.mark.parametrize("ring,cap", [(True, 48), (False, 48), (False, 768), (False, 1000), (True, 1024)])
def test_decode_two_pass_edge_rows(device, D, ring, cap):
    """G4_DECODE_TWO_PASS on rows shorter than the capacity (16, 24 and 32 chunks of V^T in
    registers): ring not yet full, left padding, a finished row, a fully masked row (uniform
    average over the capacity, including never-scanned slots), a row whose only valid key is the
    appended one."""

    B, H, R = 5, 2, 4
    sc = cap // 48
    q_pos = np.array([5, 20, 40, 33, 9]) * sc
    key_mask = np.ones((B, cap), bool)
    key_mask[1, :3 * sc] = False
    key_mask[2, 30 * sc:] = False
    key_mask[3, :] = False
    key_mask[4, :9 * sc] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=cap, ring=ring, window=cap if ring else 0, q_pos=q_pos,
                 key_mask=key_mask, fused=True, seed=27, num_splits=_lib.G4_DECODE_TWO_PASS)


@pytest.mark.parametrize("D", [256, 512])
def test_decode_two_pass_ring_end_group(device, D):
    """G4_DECODE_TWO_PASS appends into a 100-slot ring at its last 8-slot value group (slots 96..103
    of a 128-slot stride: the launch rewrites the appended value's group whole, including the slots
    past the capacity), after wrapping, and at slot 3; the cache stays bit-exact."""

    B, H, R, cap = 4, 2, 4, 100
    q_pos = np.array([96, 99, 197, 303])
    key_mask = np.ones((B, 320), bool)
    key_mask[2, :20] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=cap, ring=True, window=cap, q_pos=q_pos,
                 key_mask=key_mask, fused=True, seed=31, num_splits=_lib.G4_DECODE_TWO_PASS)


@pytest.mark.parametrize("R,W", [(1, 512), (2, 512), (8, 512), (16, 512), (4, 768), (16, 1024)])
def test_decode_two_pass_group_sizes(device, R, W):
    """G4_DECODE_TWO_PASS with 1..16 query heads per KV head: values waves with no head of their
    own (R < 4) and waves with several (R > 4); a wrapped ring of 512..1024 slots, one row fully
    masked."""

    rng = np.random.default_rng(12)
    B, H, D = 6, 2, 256
    q_pos = rng.integers(600, 1400, B)
    key_mask = np.ones((B, 1400), bool)
    key_mask[2, :] = False
    key_mask[4, 700:] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=W, ring=True, window=W, q_pos=q_pos, key_mask=key_mask,
                 fused=True, seed=28, num_splits=_lib.G4_DECODE_TWO_PASS)


@pytest.mark.parametrize("R,ring,cap", [(1, True, 512), (4, True, 512), (8, False, 1000), (16, True, 96)])
def test_decode_head_dim_512_automatic(device, R, ring, cap):
    """bf16 head dim 512 (the reference's default global head dim, model.py:66) with the library's
    own choice of path (num_splits 0): the two-launch path at any pair count for rows of up to 1024
    slots (values workgroups of 8 or 4 waves: 4 or 8 per pair); 1..16 query heads per KV head, a
    wrapped ring, a left-padded row, a fully masked row."""

    rng = np.random.default_rng(R + cap)
    B, H, D = 3, 2, 512
    q_pos = rng.integers(cap, 2 * cap, B) if ring else np.array([999, 400, 37])
    key_mask = np.ones((B, 2 * cap if ring else cap), bool)  # a linear cache's mask spans its capacity
    key_mask[1, :20] = False
    key_mask[2, :] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=cap, ring=ring, window=cap if ring else 0, q_pos=q_pos,
                 key_mask=key_mask, fused=True, seed=29)


@pytest.mark.parametrize("D", [128, 256, 512])
def test_decode_split_keys_long_context(device, D):
    """BASELINE config 3 shape at reduced capacity: global-layer linear cache with ragged
    lengths over few (b, kv head) pairs, so the library splits the key range (scores / values /
    combine launches). Rows end mid-split, one row is shorter than a split, one is fully masked,
    one is left-padded; the appended slot lands in different splits."""

    rng = np.random.default_rng(9)
    B, H, R, C = 4, 2, 4, 4096
    q_pos = np.array([4095, 2600, 300, 1500])
    key_mask = np.ones((B, C), bool)
    key_mask[2, :] = False
    key_mask[3, :700] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=C, ring=False, window=0, q_pos=q_pos, key_mask=key_mask,
                 fused=True, seed=24)


def test_decode_split_keys_beyond_one_combine_batch(device):
    """Split-K over more than 64 key splits (capacity 40000: 79 splits of 512 slots), so the combine
    adds a row's partials in two batches of loads: a row over every split, a fully masked row (the
    uniform average over all 79 splits) and a left-padded one; 6 pairs x 79 splits, not a multiple
    of 8 items."""

    B, H, R, D, C = 3, 2, 4, 256, 40000
    q_pos = np.array([39999, 35000, 20000])
    key_mask = np.ones((B, C), bool)
    key_mask[1, :] = False
    key_mask[2, :5000] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=C, ring=False, window=0, q_pos=q_pos, key_mask=key_mask,
                 fused=True, seed=31)


@pytest.mark.parametrize("D", [128, 256, 512])
def test_decode_split_keys_forced_matches_one_pass(device, D):
    """num_splits = G4_DECODE_SPLIT_KEYS on a 768-slot cache (where the one-pass kernel also
    applies) against the oracle; unfused (no append)."""

    rng = np.random.default_rng(10)
    B, H, R, C = 3, 2, 4, 768
    q_pos = np.array([767, 513, 100])
    key_mask = np.ones((B, C), bool)
    key_mask[1, 500:520] = False
    _decode_case(device, O.BF16, B=B, H=H, R=R, D=D, cap=C, ring=False, window=0, q_pos=q_pos, key_mask=key_mask,
                 fused=False, seed=25, num_splits=_lib.G4_DECODE_SPLIT_KEYS)


@pytest.mark.parametrize("dtype,D", [(O.BF16, 64), (O.BF16, 256), (O.F32, 64)])
def test_decode_ring_partial_and_masked_rows(device, dtype, D):
    """Ring not yet full, left padding, a finished row and a fully masked row (uniform average)."""

    B, H, R, W = 4, 2, 4, 16
    q_pos = np.array([5, 20, 40, 33])
    key_mask = np.ones((B, 48), bool)
    key_mask[1, :3] = False
    key_mask[2, 30:] = False  # finished row: positions after 29 are pads
    key_mask[3, :] = False  # every key masked
    _decode_case(device, dtype, B=B, H=H, R=R, D=D, cap=W, ring=True, window=W, q_pos=q_pos, key_mask=key_mask,
                 fused=True, seed=21)


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
def test_decode_linear_ragged(device, dtype):
    """Global-layer linear cache, ragged lengths, left padding, a fully masked row."""

    rng = np.random.default_rng(4)
    B, H, R, D, C = 5, 2, 4, 128 if dtype == O.BF16 else 64, 1000
    q_pos = rng.integers(0, C, B)
    q_pos[0] = C - 1
    key_mask = np.ones((B, C), bool)
    key_mask[1, :17] = False
    key_mask[2, :] = False
    _decode_case(device, dtype, B=B, H=H, R=R, D=D, cap=C, ring=False, window=0, q_pos=q_pos, key_mask=key_mask,
                 fused=True, seed=22)


def test_decode_is_deterministic(device):
    rng = np.random.default_rng(9)
    B, H, R, D, W = 8, 2, 4, 256, 512
    layer = new_layer_cache(B, H, D, W, True, torch.bfloat16, device)
    layer.key.normal_()
    layer.value_t.normal_()
    q = torch.randn((B, H, R, D), device=device).to(torch.bfloat16)
    km = torch.ones((B, 4096), dtype=torch.bool, device=device)
    qp = torch.from_numpy(rng.integers(600, 4000, B).astype(np.int32)).to(device)
    a = kernels.decode_attention(layer, q, km, q_pos=qp, window=W)
    b = kernels.decode_attention(layer, q, km, q_pos=qp, window=W)
    assert torch.equal(a, b)


# --- prefill attention ----------------------------------------------------------------------------


@pytest.mark.parametrize("dtype,D", [(O.BF16, 512), (O.BF16, 256), (O.BF16, 128), (O.BF16, 64), (O.F32, 64)])
@pytest.mark.parametrize("window", [0, 48])
def test_prefill_matches_oracle(device, dtype, D, window):
    """Causal + sliding-window prefill with left padding (fully masked pad queries); S not a
    multiple of the 32-key chunk nor of a workgroup's 32 positions."""

    rng = np.random.default_rng(D + window)
    B, S, H, R = 2, 150, 2, 4
    Sp = (S + 63) // 64 * 64
    q = _rand(rng, (B, S, H, R, D), dtype)
    k = _rand(rng, (B, S, H, D), dtype)
    v = _rand(rng, (B, S, H, D), dtype)
    key_mask = np.ones((B, S), bool)
    key_mask[1, :11] = False
    td = __import__("gpu_util").TORCH_DTYPE[dtype]
    kd = torch.zeros((B, H, Sp, D), dtype=td, device=device)
    vs = torch.zeros((B, H, Sp, D), dtype=td, device=device)
    kd[:, :, :S] = to_dev(k, dtype, device).permute(0, 2, 1, 3)
    vs[:, :, :S] = to_dev(v, dtype, device).permute(0, 2, 1, 3)
    vtd = group_values(vs)
    out = kernels.prefill_attention(to_dev(q, dtype, device), group_keys(kd), vtd, torch.from_numpy(key_mask).to(device),
                                    window=window)
    masks = O.make_qk_masks(key_mask, window if window else 1 << 30, 0, S)
    q_ref = q.transpose(0, 1, 3, 2, 4)  # [B, S, R, H, D]
    o_ref = _attention_ref(q_ref, k, v, masks[O.SLIDING], dtype).transpose(0, 1, 3, 2, 4)
    err = np.abs(to_np(out) - o_ref).max()
    assert err <= TOL[dtype], f"max |out - oracle| = {err}"


@pytest.mark.parametrize("R", [1, 2, 8])
def test_prefill_group_sizes(device, R):
    """Other GQA group sizes (16/R positions per wave) on the LDS-staged bf16 kernel, a longer row
    (several workgroups of positions, heaviest launched first) and a sliding window."""

    rng = np.random.default_rng(30 + R)
    B, S, H, D, window = 1, 300, 2, 128, 100
    q = _rand(rng, (B, S, H, R, D), O.BF16)
    k = _rand(rng, (B, S, H, D), O.BF16)
    v = _rand(rng, (B, S, H, D), O.BF16)
    key_mask = np.ones((B, S), bool)
    key_mask[0, 120:125] = False
    Sp = (S + 63) // 64 * 64
    kd = torch.zeros((B, H, Sp, D), dtype=torch.bfloat16, device=device)
    vs = torch.zeros((B, H, Sp, D), dtype=torch.bfloat16, device=device)
    kd[:, :, :S] = to_dev(k, O.BF16, device).permute(0, 2, 1, 3)
    vs[:, :, :S] = to_dev(v, O.BF16, device).permute(0, 2, 1, 3)
    vtd = group_values(vs)
    out = kernels.prefill_attention(to_dev(q, O.BF16, device), group_keys(kd), vtd, torch.from_numpy(key_mask).to(device),
                                    window=window)
    masks = O.make_qk_masks(key_mask, window, 0, S)
    o_ref = O.attention_core(q.transpose(0, 1, 3, 2, 4), k, v, masks[O.SLIDING], O.BF16).transpose(0, 1, 3, 2, 4)
    err = np.abs(to_np(out) - o_ref).max()
    assert err <= TOL[O.BF16], f"max |out - oracle| = {err}"


# --- fused decoder-layer glue ---------------------------------------------------------------------

# one rounding of the activation dtype on either side (the kernels and the oracle sum the mean of
# squares in different orders, which can move a result across a rounding boundary)
GLUE_RTOL = {O.BF16: 2.0 ** -7, O.F32: 1e-5}
# absolute floor for results that cancel to near zero (a residual plus a normed branch; gelu of a
# very negative gate, where 1 + tanh cancels and tanh implementations differ in the last bits)
GLUE_ATOL = {O.BF16: 1e-5, O.F32: 1e-6}


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
@pytest.mark.parametrize("cols", [2048, 4096, 200, 100])
def test_rms_norm_matches_oracle(device, dtype, cols):
    """g4_rms_norm against the oracle's rms_norm (model.py:278-285): bf16 rows of a multiple of 8
    take the one-wave-per-row kernel (full and partial 512-column rounds), others the general one."""

    rng = np.random.default_rng(cols)
    x = _rand(rng, (5, 3, cols), dtype) * 3
    w = O.cast(1 + 0.3 * rng.standard_normal(cols).astype(np.float32), dtype)
    got = to_np(kernels.rms_norm(to_dev(x, dtype, device), to_dev(w, dtype, device), 1e-6))
    ref = O.rms_norm(w, x, 1e-6, dtype)
    np.testing.assert_allclose(got, ref, rtol=GLUE_RTOL[dtype], atol=GLUE_ATOL[dtype])
    got = to_np(kernels.rms_norm(to_dev(x, dtype, device), None, 1e-6))  # no scale (v_norm)
    np.testing.assert_allclose(got, O.rms_norm(None, x, 1e-6, dtype), rtol=GLUE_RTOL[dtype], atol=GLUE_ATOL[dtype])


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
@pytest.mark.parametrize("M", [2048, 4096, 1004])
def test_residual_norm_matches_oracle_layer_tail(device, dtype, M):
    """g4_residual_norm = the oracle's post-norm, residual add, layer scalar and the next norm
    (forward_decoder_layer, model.py:505-554), each rounded where the oracle rounds."""

    rng = np.random.default_rng(5)
    a = _rand(rng, (4, 1, M), dtype)
    x = _rand(rng, (4, 1, M), dtype)
    wa = O.cast(1 + 0.3 * rng.standard_normal(M).astype(np.float32), dtype)
    wn = O.cast(1 + 0.3 * rng.standard_normal(M).astype(np.float32), dtype)
    scalar = np.float32(0.8125)
    xo, ho = kernels.residual_norm(to_dev(a, dtype, device), to_dev(wa, dtype, device), to_dev(x, dtype, device),
                                   scalar=torch.tensor([scalar], device=device), next_weight=to_dev(wn, dtype, device),
                                   eps=1e-6)
    x_ref = O.cast(O.cast(x + O.rms_norm(wa, a, 1e-6, dtype), dtype) * scalar, dtype)
    np.testing.assert_allclose(to_np(xo), x_ref, rtol=GLUE_RTOL[dtype], atol=GLUE_ATOL[dtype])
    np.testing.assert_allclose(to_np(ho), O.rms_norm(wn, to_np(xo), 1e-6, dtype), rtol=GLUE_RTOL[dtype], atol=GLUE_ATOL[dtype])
    xo2, h2 = kernels.residual_norm(to_dev(a, dtype, device), to_dev(wa, dtype, device), to_dev(x, dtype, device),
                                    scalar=None, next_weight=None, eps=1e-6, with_next=False)
    assert h2 is None
    np.testing.assert_allclose(to_np(xo2), O.cast(x + O.rms_norm(wa, a, 1e-6, dtype), dtype),
                               rtol=GLUE_RTOL[dtype], atol=GLUE_ATOL[dtype])


@pytest.mark.parametrize("dtype", [O.BF16, O.F32])
def test_gelu_mul_matches_oracle(device, dtype):
    """g4_gelu_mul = the oracle's gelu_tanh(gate) * up rounded once (forward_mlp, model.py:393-396)."""

    rng = np.random.default_rng(6)
    F = 1000  # a multiple of 8: the 16-byte bf16 path; F + 4 below: the general one
    gu = _rand(rng, (3, 2, 2 * F), dtype) * 2
    got = to_np(kernels.gelu_mul(to_dev(gu, dtype, device)))
    ref = O.cast(O.gelu_tanh(gu[..., :F]) * gu[..., F:], dtype)
    np.testing.assert_allclose(got, ref, rtol=GLUE_RTOL[dtype], atol=GLUE_ATOL[dtype])
    gu = _rand(rng, (3, 2, 2 * (F + 4)), dtype) * 2
    got = to_np(kernels.gelu_mul(to_dev(gu, dtype, device)))
    ref = O.cast(O.gelu_tanh(gu[..., :F + 4]) * gu[..., F + 4:], dtype)
    np.testing.assert_allclose(got, ref, rtol=GLUE_RTOL[dtype], atol=GLUE_ATOL[dtype])
