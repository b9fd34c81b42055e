"""g4_decode_prologue against the framework ops it replaces in the graphed decode step (the
embedding lookup and scale, the key-mask scatter at the write slot, the rotary tables of
model.rotary_tables): the embedding rows and the key mask bit for bit, the f32 cos / sin within
one ulp of torch's device cos / sin on the same f32 angles."""

from __future__ import annotations

import math

import pytest
import torch

from gemma4_posttrain_jax_amd import kernels
from gemma4_posttrain_jax_amd.model import rotary_tables

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,M,V,C,dims", [(256, 2048, 4096, 768, (256, 256)), (3, 64, 50, 40, (64, 16)),
                                          (5, 128, 1000, 20, (32,))])
def test_decode_prologue_matches_framework_ops(device, B, M, V, C, dims):
    g = torch.Generator(device="cuda").manual_seed(B + M)
    embed = (torch.randn((V, M), device="cuda", generator=g) * 0.5).to(torch.bfloat16)
    tokens = torch.randint(-2, V + 2, (B,), device="cuda", generator=g, dtype=torch.int32)  # a few off-table ids
    positions = torch.randint(0, 40000, (B,), device="cuda", generator=g, dtype=torch.int32)
    active = torch.rand((B,), device="cuda", generator=g) > 0.3
    slot = torch.randint(-1, C + 1, (B,), device="cuda", generator=g, dtype=torch.int32)  # some outside the row
    km = torch.rand((B, C), device="cuda", generator=g) > 0.5
    inv = [(1.0 / (10000.0 ** (torch.arange(0, d, 2, device="cuda", dtype=torch.float32) / d))).contiguous()
           for d in dims]
    scale = float(torch.tensor(math.sqrt(M), dtype=torch.bfloat16).float())

    km_ref = km.clone()
    inside = (slot >= 0) & (slot < C)
    rows = torch.arange(B, device="cuda")[inside]
    km_ref[rows, slot[inside].long()] = active[inside]
    x_ref = (embed[tokens.clamp(0, V - 1).long()].float() * scale).to(torch.bfloat16)

    x, tables = kernels.decode_prologue(embed, tokens, positions, active, slot, km, embed_scale=scale, inv_freq=inv)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int16), x_ref.view(torch.int16))
    assert torch.equal(km, km_ref)
    for f, (c, s) in zip(inv, tables):
        c_ref, s_ref = rotary_tables(f, positions[:, None])
        for got, ref in ((c, c_ref[:, 0]), (s, s_ref[:, 0])):
            ulp = (got.view(torch.int32).long() - ref.view(torch.int32).long()).abs()
            assert int(ulp.max()) <= 1, f"cos/sin differ by {int(ulp.max())} ulp"
