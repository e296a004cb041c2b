"""GPU: the differentiable LayerNorm (``kernels.LayerNormFunction``: pf_layernorm_fwd and
pf_layernorm_bwd), against torch's LayerNorm differentiated in fp64 (a library routine), at
the widths the training paths use; fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref|; bf16
within 2x the error of torch's own bf16 LayerNorm gradient (computed on the CPU). The affine
gradients are summed in a fixed order: bitwise-reproducible."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from tests._helpers import assert_fp32_close, mod, rel_l2

pytestmark = pytest.mark.gpu
kernels = mod("kernels")


def _case(M, C, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, C, generator=g) * 2 + 0.5
    w, b = 1 + 0.2 * torch.randn(C, generator=g), 0.3 * torch.randn(C, generator=g)
    dy = torch.randn(M, C, generator=g)
    return x, w, b, dy


def _ref(x, w, b, dy, dtype):
    leaves = [t.to(dtype).requires_grad_(True) for t in (x, w, b)]
    out = F.layer_norm(leaves[0], (x.shape[-1],), leaves[1], leaves[2], 1e-5)
    return [g.double() for g in torch.autograd.grad(out, leaves, grad_outputs=dy.to(dtype))]


@pytest.mark.parametrize("C", [64, 128, 384])
def test_layernorm_backward_fp32(dev, C):
    M = 1000
    x, w, b, dy = _case(M, C, C)
    leaves = [t.to(dev).requires_grad_(True) for t in (x, w, b)]
    out = kernels.LayerNormFunction.apply(*leaves, 1e-5)
    got = torch.autograd.grad(out, leaves, grad_outputs=dy.to(dev))
    want = _ref(x, w, b, dy, torch.float64)
    for a, r, name in zip(got, want, ("dx", "dw", "db")):
        assert_fp32_close(a.cpu(), r.float(), what=f"LayerNorm {name} C={C}")
    again = torch.autograd.grad(kernels.LayerNormFunction.apply(*leaves, 1e-5), leaves, grad_outputs=dy.to(dev))
    for a, r in zip(got, again):
        assert torch.equal(a, r)


def test_layernorm_backward_bf16(dev):
    M, C = 4096, 128
    x, w, b, dy = _case(M, C, 5)
    xb, dyb = x.to(torch.bfloat16), dy.to(torch.bfloat16)
    leaves = [xb.to(dev).requires_grad_(True), w.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)]
    out = kernels.LayerNormFunction.apply(*leaves, 1e-5)
    got = torch.autograd.grad(out, leaves, grad_outputs=dyb.to(dev))
    want = _ref(xb.float(), w, b, dyb.float(), torch.float64)
    eager = _ref(xb.float(), w, b, dyb.float(), torch.float32)
    eager_dx = eager[0].to(torch.bfloat16).double()  # torch's bf16 LayerNorm returns dx in bf16
    assert rel_l2(got[0].double().cpu(), want[0]) <= 2 * rel_l2(eager_dx, want[0]) + 1e-6
    for a, r in zip(got[1:], want[1:]):
        assert rel_l2(a.double().cpu(), r) < 1e-3
