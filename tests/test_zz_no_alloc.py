"""g4_decode_attention_noalloc (the entry point for callers that cannot allocate) against
g4_decode_attention with a caller workspace: bitwise the same outputs and caches, through the C
ABI, on two calls in a row with the second smaller, for each path that uses scratch (the two-launch
path and split-K), and the host-side rejection of a call needing more than the library's scratch."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gemma4_posttrain_jax_amd import _lib, kernels
from gemma4_posttrain_jax_amd.kvcache import new_layer_cache

pytestmark = pytest.mark.gpu


def _case(device, *, B, H, R, D, cap, ring, seed, num_splits):
    g = torch.Generator(device=device).manual_seed(seed)
    rng = np.random.default_rng(seed)
    layer = new_layer_cache(B, H, D, cap, ring, torch.bfloat16, device)
    layer.key.normal_(generator=g)
    layer.value_t.normal_(generator=g)
    twin = new_layer_cache(B, H, D, cap, ring, torch.bfloat16, device)
    twin.key.copy_(layer.key)
    twin.value_t.copy_(layer.value_t)
    q = torch.randn((B, H, R, D), device=device, generator=g).to(torch.bfloat16)
    nk = torch.randn((B, H, D), device=device, generator=g).to(torch.bfloat16)
    nv = torch.randn((B, H, D), device=device, generator=g).to(torch.bfloat16)
    hi = 3 * cap if ring else cap
    q_pos = torch.from_numpy(rng.integers(cap // 2, hi, B).astype(np.int32)).to(device)
    km = torch.ones((B, hi + 1), dtype=torch.bool, device=device)
    km[0, :7] = False
    want = kernels.decode_attention(twin, q, km, q_pos=q_pos, window=cap if ring else 0, new_k=nk, new_v=nv,
                                    num_splits=num_splits)
    out = torch.empty_like(q)
    got = kernels.decode_attention(layer, q, km, q_pos=q_pos, window=cap if ring else 0, new_k=nk, new_v=nv,
                                   num_splits=num_splits, out=out, no_alloc=True)
    torch.cuda.synchronize()
    assert got is out
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert torch.equal(layer.key.view(torch.int16), twin.key.view(torch.int16))
    assert torch.equal(layer.value_t.view(torch.int16), twin.value_t.view(torch.int16))


def test_noalloc_two_pass_matches_workspace_call(device):
    """Two-launch path: 256 pairs on a 512-slot ring, then 64 pairs (forced) on a 768-slot linear
    cache; the second call reuses the scratch the first one filled."""

    _case(device, B=128, H=2, R=4, D=256, cap=512, ring=True, seed=1, num_splits=0)
    _case(device, B=32, H=2, R=4, D=128, cap=768, ring=False, seed=2, num_splits=_lib.G4_DECODE_TWO_PASS)


def test_noalloc_split_keys_matches_workspace_call(device):
    """Split-K path (long rows over few pairs): 32 pairs over 32768 slots (16 MiB of scratch), then
    8 pairs over 4096 slots."""

    _case(device, B=16, H=2, R=4, D=256, cap=32768, ring=False, seed=3, num_splits=0)
    _case(device, B=4, H=2, R=4, D=128, cap=4096, ring=False, seed=4, num_splits=0)


def test_noalloc_rejects_oversized_and_workspace_calls(device):
    """Host-side errors, before any launch: a call needing more scratch than the library holds, and a
    call that brings its own workspace."""

    B, H, R, D, C = 64, 2, 4, 256, 32768  # split-K over 128 pairs x 64 splits: 64 MiB
    a = _lib.G4DecodeArgs(dtype=_lib.G4_DTYPE_BF16, kind=_lib.G4_CACHE_LINEAR, batch=B, kv_heads=H, group=R,
                          head_dim=D, capacity=C, slot_stride=C, window=0, q_pos_scalar=0, q_pos=None, key_mask=1,
                          key_mask_stride=C, q=1, cache_k=1, cache_vt=1, cache_k_w=1, new_k=None, new_v=None, out=1,
                          workspace=None, workspace_bytes=0, prep=None, num_splits=_lib.G4_DECODE_SPLIT_KEYS)
    assert _lib.lib().g4_decode_workspace_size(ctypes.byref(a)) > 32 << 20
    assert _lib.lib().g4_decode_attention_noalloc(ctypes.byref(a), None) == _lib.G4_ERR_WORKSPACE
    assert b"more than the" in _lib.lib().g4_last_error()
    a.workspace, a.workspace_bytes = 1, 1 << 20
    assert _lib.lib().g4_decode_attention_noalloc(ctypes.byref(a), None) == _lib.G4_ERR_INVALID
