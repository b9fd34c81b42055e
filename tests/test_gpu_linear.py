"""g4_linear_bf16 (the decode-step projection GEMM) against an fp32 reference of the same product.

The bar: |y - x.w^T| <= 2^-8 |x.w^T| + 1e-5 elementwise, i.e. the bf16 rounding of an f32-accumulated
dot product (half an ulp is 2^-9 relative) plus summation-order slack."""

from __future__ import annotations

import pytest
import torch

from gemma4_posttrain_jax_amd import kernels

pytestmark = pytest.mark.gpu


def _check(m, n, k, ksplit, seed, ldy=None):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn((n, k), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    out = None
    if ldy is not None:
        out = torch.full((m, ldy), float("nan"), device="cuda", dtype=torch.bfloat16)[:, :n]
    y = kernels.linear(x, w, out=out, ksplit=ksplit)
    ref = x.double().cpu() @ w.double().cpu().T
    err = (y.double().cpu() - ref).abs()
    bar = ref.abs() * 2.0 ** -8 + 1e-5
    assert torch.all(err <= bar), f"max excess {(err - bar).max().item():.3g} (max err {err.max().item():.3g})"
    if ldy is not None:  # columns past n untouched
        assert torch.isnan(out.as_strided((m, ldy), (ldy, 1))[:, n:].float()).all()


@pytest.mark.parametrize("n,k,ksplit", [(16384, 2048, 1), (2048, 8192, 8), (3072, 2048, 4), (2048, 2048, 1),
                                        (2048, 8192, 1)])
def test_linear_e2b_projection_shapes(device, n, k, ksplit):
    """The E2B decode projections at B=256: gate/up, down (split 8), q/k/v, o; down unsplit."""

    _check(256, n, k, ksplit, seed=n + k + ksplit)


@pytest.mark.parametrize("m,n", [(1, 192), (17, 192), (64, 192), (200, 192), (200, 256), (129, 384), (255, 128),
                                 (200, 1024)])
def test_linear_partial_row_blocks(device, m, n):
    """Fewer rows than the tile (rows past m read as zero, never stored): the 256 x 64 tiles, and the
    128 x 128 tiles (m > 128, n a multiple of 128) whose second row half is partly filled; split-K;
    a strided output with columns past n left untouched."""

    _check(m, n, 640, 5 if m != 64 else 1, seed=m + n, ldy=n + 64)


@pytest.mark.parametrize("rows,cols,k,ksplit,with_scalar", [(256, 2048, 8192, 8, True), (37, 4096, 1536, 3, False),
                                                            (5, 64, 512, 2, True)])
def test_residual_norm_splitk_equals_unfused(device, rows, cols, k, ksplit, with_scalar):
    """The down projection's partial sums fed straight into the residual norm give the same bits
    as g4_linear_bf16's own split-K sum followed by g4_residual_norm (same split order, same
    rounding points)."""

    g = torch.Generator(device="cuda").manual_seed(rows + cols)
    act = torch.randn((rows, k), device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn((cols, k), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    res = torch.randn((rows, cols), device="cuda", generator=g).to(torch.bfloat16)
    bw = (1 + 0.1 * torch.randn(cols, device="cuda", generator=g)).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(cols, device="cuda", generator=g)).to(torch.bfloat16)
    scalar = torch.tensor([0.75], device="cuda") if with_scalar else None
    part = kernels.linear_partials(act, w, ksplit=ksplit)
    x1, h1 = kernels.residual_norm_splitk(part, bw, res, scalar=scalar, next_weight=nw, eps=1e-6)
    y = kernels.linear(act, w, ksplit=ksplit)
    x2, h2 = kernels.residual_norm(y, bw, res, scalar=scalar, next_weight=nw, eps=1e-6)
    assert torch.equal(x1.view(torch.int16), x2.view(torch.int16))
    assert torch.equal(h1.view(torch.int16), h2.view(torch.int16))


@pytest.mark.parametrize("m,f,k", [(256, 8192, 2048), (19, 96, 320), (200, 192, 512)])
def test_linear_gelu_epilogue(device, m, f, k):
    """The gated-GELU epilogue equals g4_linear_bf16's own gate/up product followed by
    g4_gelu_mul bit for bit, and the fp32 reference within the bf16 bar."""

    g = torch.Generator(device="cuda").manual_seed(m + f)
    x = torch.randn((m, k), device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn((2 * f, k), device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    act = kernels.linear_gelu(x, w)
    ref = kernels.gelu_mul(kernels.linear(x, w))
    assert torch.equal(act.view(torch.int16), ref.view(torch.int16))
    gu = (x.double().cpu() @ w.double().cpu().T).to(torch.bfloat16).double()
    gg, uu = gu[:, :f], gu[:, f:]
    want = 0.5 * gg * (1 + torch.tanh(0.7978845608028654 * (gg + 0.044715 * gg ** 3))) * uu
    # g and u may round one bf16 ulp (2^-8 relative) away from the f64 products' rounding, which
    # moves gelu(g) * u by up to about 2^-7 |g u|: the bar is 2^-6 (|want| + |g u|)
    err = (act.double().cpu() - want).abs()
    bar = (want.abs() + (gg * uu).abs()) * 2.0 ** -6 + 1e-5
    assert torch.all(err <= bar), float((err - bar).max())
