"""GPU: the differentiable LayerNorm (``kernels.LayerNormFunction``: pf_layernorm_fwd and
pf_layernorm_bwd), against torch's LayerNorm differentiated in fp64 (a library routine), at
the widths the training paths use; fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref|; bf16
within 2x the error of torch's own bf16 LayerNorm gradient (computed on the CPU). The affine
gradients are summed in a fixed order: bitwise-reproducible. The mixed-dtype entry points
(fp32 input, bf16 output and cotangent: the autocast training path) against the fp32 kernels
with the cast done by torch, bit for bit. The kernel-level fused ops under grad (built on it
and on the HIP SwiGLU backward) against torch's formulas in fp64."""

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


def _grads(fn, leaves, cot):
    out = fn(*leaves)
    return out, torch.autograd.grad(out, leaves, grad_outputs=cot)


@pytest.mark.parametrize("C", [128, 384, 96])
def test_layernorm_mixed_dtypes_are_the_casts(dev, C):
    """bf16 output from fp32 x = the fp32 LayerNorm rounded by torch; the backward with a bf16
    cotangent = the fp32 backward with that cotangent upcast (the same arithmetic, bit for
    bit). C=96 runs the generic row kernel forward (the backward is built for 64..512)."""
    M = 777
    x, w, b, dy = _case(M, C, 11 + C)
    x32 = x.to(dev).requires_grad_(True)
    w1, b1 = w.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    out16 = kernels.LayerNormFunction.apply(x32, w1, b1, 1e-5, torch.bfloat16)
    assert out16.dtype == torch.bfloat16
    with torch.no_grad():
        ref32 = kernels.LayerNormFunction.apply(x32.detach(), w1.detach(), b1.detach(), 1e-5)
    assert torch.equal(out16, ref32.to(torch.bfloat16))
    if C == 96:
        return
    dy16 = dy.to(dev, torch.bfloat16)
    got = torch.autograd.grad(out16, [x32, w1, b1], grad_outputs=dy16)
    x2 = x.to(dev).requires_grad_(True)
    w2, b2 = w.to(dev).requires_grad_(True), b.to(dev).requires_grad_(True)
    out32 = kernels.LayerNormFunction.apply(x2, w2, b2, 1e-5)
    want = torch.autograd.grad(out32, [x2, w2, b2], grad_outputs=dy16.float())
    print(f"[layernorm mixed] C={C}", flush=True)
    for g_, r_ in zip(got, want):
        assert g_.dtype == r_.dtype and torch.equal(g_, r_)


def test_fused_ops_are_differentiable_fp32(dev):
    """FusedSwiGLU, FusedLayerNormLinear, FusedPairBias and FusedLayerNormTranspose under grad
    (swiglu.py:60-95, layernorm_linear.py:164-322, fused_pair_bias.py, layernorm_transpose.py:95-161)
    against torch's formulas differentiated in fp64."""
    fused = mod("fused")
    g = torch.Generator().manual_seed(7)
    # SwiGLU
    x = torch.randn(300, 2 * 96, generator=g)
    cot = torch.randn(300, 96, generator=g)
    _, got = _grads(fused.FusedSwiGLU(), [x.to(dev).requires_grad_(True)], cot.to(dev))
    _, want = _grads(lambda t: F.silu(t[:, :96]) * t[:, 96:], [x.double().requires_grad_(True)], cot.double())
    assert_fp32_close(got[0].cpu(), want[0].float(), what="FusedSwiGLU dx")
    # LayerNorm + linear with bias, W as [K, N]
    K, N = 128, 64
    X = torch.randn(4, 50, K, generator=g)
    lw, lb = 1 + 0.1 * torch.randn(K, generator=g), 0.1 * torch.randn(K, generator=g)
    Wt, bias = torch.randn(K, N, generator=g) / K**0.5, torch.randn(N, generator=g)
    cot = torch.randn(4, 50, N, generator=g)
    op = fused.FusedLayerNormLinear(K, N, has_linear_bias=True)
    _, got = _grads(op, [t.to(dev).requires_grad_(True) for t in (X, lw, lb, Wt, bias)], cot.to(dev))
    _, want = _grads(lambda a, w, b, W_, bb: F.layer_norm(a, (K,), w, b, 1e-5) @ W_ + bb,
                     [t.double().requires_grad_(True) for t in (X, lw, lb, Wt, bias)], cot.double())  # fmt: skip
    for a, r, name in zip(got, want, ("X", "ln_w", "ln_b", "W", "b")):
        assert_fp32_close(a.cpu(), r.float(), what=f"FusedLayerNormLinear d{name}")
    # pair bias with a mask, and LayerNorm + transpose
    B, Nr, C, H = 1, 20, 128, 4
    z = torch.randn(B, Nr, Nr, C, generator=g)
    pw = torch.randn(H, C, generator=g) / C**0.5
    mask = (torch.rand(B, Nr, generator=g) > 0.2).float()
    cot = torch.randn(B, H, Nr, Nr, generator=g)
    _, got = _grads(lambda a, w, b, p: fused.FusedPairBias(C, H)(a, w, b, p, mask.to(dev)),
                    [t.to(dev).requires_grad_(True) for t in (z, lw, lb, pw)], cot.to(dev))  # fmt: skip
    _, want = _grads(lambda a, w, b, p: F.linear(F.layer_norm(a, (C,), w, b, 1e-5), p).permute(0, 3, 1, 2),
                     [t.double().requires_grad_(True) for t in (z, lw, lb, pw)], cot.double())  # fmt: skip
    for a, r, name in zip(got, want, ("z", "ln_w", "ln_b", "proj_w")):
        assert_fp32_close(a.cpu(), r.float(), what=f"FusedPairBias d{name}")
    cot = torch.randn(B, Nr, Nr, C, generator=g)
    _, got = _grads(fused.FusedLayerNormTranspose(C, True), [t.to(dev).requires_grad_(True) for t in (z, lw, lb)],
                    cot.to(dev))  # fmt: skip
    _, want = _grads(lambda a, w, b: F.layer_norm(a, (C,), w, b, 1e-5).permute(0, 2, 1, 3),
                     [t.double().requires_grad_(True) for t in (z, lw, lb)], cot.double())  # fmt: skip
    for a, r, name in zip(got, want, ("x", "w", "b")):
        assert_fp32_close(a.cpu(), r.float(), what=f"FusedLayerNormTranspose d{name}")
