"""GPU: the triangle multiply's training path (``FusedTriMulFunction``, fused_trimul.py:285-330).

- ``kernels.FusedTriMulFunction`` with fp32 GEMM operands against the oracle's
  ``tri_mul_core`` differentiated in fp64 (its composition with the LayerNorm is pinned to
  ``tri_mul`` and its gradient by finite differences in test_oracle.py): the update and the
  gradients of x, w_gate, w_proj, the LN_out affine, w_out and w_out_gate at relL2 <= 1e-5 and
  max-abs <= 1e-5 max|ref|; C = 64, 128, 256, both directions, ragged N, masked pairs.
- The modules under grad in the reference's training regime, as its
  test_fused_backward_matches_stock (tests/triton/test_fused_trimul.py:87-106): z fp32 under
  bf16 autocast, N = 133, C = 128 / 256, B = 1 / 2; every gradient (z and all parameters)
  within 3x the relL2 of the stock path under bf16 autocast (+1e-3) of the fp32 stock path.
  The stock references run on the CPU (fp32 and CPU bf16 autocast).
- The module in fp32 end to end against the oracle's stock ``tri_mul`` in fp64.
- Bitwise-reproducible gradients.
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_fp32_close, mod, rel_l2, sub

pytestmark = pytest.mark.gpu
W = mod("weights")
ops = mod("ops")
kernels = mod("kernels")
BF = torch.bfloat16


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _core_inputs(B, N, C, seed):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)  # noqa: E731
    x = r(B, N, N, C)
    mask = (torch.rand(B, N, N, generator=g) > 0.15).float()
    mask[:, N - 2 :, :] = 0.0
    mask[:, :, N - 2 :] = 0.0
    ws = [r(2 * C, C) / C**0.5, r(2 * C, C) / C**0.5, 1 + 0.1 * r(C), 0.1 * r(C), r(C, C) / C**0.5, r(C, C) / C**0.5]
    cot = r(B, N, N, C)
    return x, mask, ws, cot


NAMES = ("x", "w_gate", "w_proj", "ln_out_w", "ln_out_b", "w_out", "w_out_gate")


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
@pytest.mark.parametrize("C,N", [(128, 37), (128, 130), (64, 50), (256, 33)])
def test_fused_trimul_function_fp32(dev, C, N, outgoing):
    print(f"[trimul vjp fp32] C={C} N={N} outgoing={outgoing}", flush=True)
    x, mask, ws, cot = _core_inputs(1 if N > 100 else 2, N, C, seed=C + N)
    leaves = [t.to(dev).requires_grad_(True) for t in [x] + ws]
    out = kernels.FusedTriMulFunction.apply(leaves[0], mask.to(dev), *leaves[1:], 1e-5, outgoing)
    got = torch.autograd.grad(out, leaves, grad_outputs=cot.to(dev))
    ref_leaves = [t.double().requires_grad_(True) for t in [x] + ws]
    ref = R.tri_mul_core(ref_leaves[0], mask.double(), *ref_leaves[1:], 1e-5, outgoing)
    want = torch.autograd.grad(ref, ref_leaves, grad_outputs=cot.double())
    assert_fp32_close(out.detach().cpu(), ref.detach().float(), what="update")
    for a, b, name in zip(got, want, NAMES):
        assert a.shape == b.shape, name
        assert_fp32_close(a.cpu(), b.float(), what=f"d{name} C={C} N={N}")


def _modules(cls, C, seed=0):
    """The reference test's construction: weights N(0, 1/C) on every matrix (test_fused_trimul.py:24-31)."""
    g = torch.Generator().manual_seed(seed)
    m = cls(C)
    for p in m.parameters():
        if p.dim() == 2:
            with torch.no_grad():
                p.copy_(torch.randn(p.shape, generator=g) / C**0.5)
    return m


def _oracle_params(m) -> dict:
    return {k: v.detach().clone() for k, v in m.state_dict().items()}


def _oracle_grads(p, z, mask, weight, outgoing, autocast):
    leaves = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    zz = z.clone().requires_grad_(True)
    with torch.autocast("cpu", dtype=BF, enabled=autocast):
        out = R.tri_mul(zz, mask, leaves, outgoing)
    (out.float() * weight).sum().backward()
    return {"z": zz.grad.float(), **{k: t.grad.float() for k, t in leaves.items()}}


@pytest.mark.parametrize("cls", ["TriangleMulOutgoing", "TriangleMulIncoming"])
@pytest.mark.parametrize("C,B", [(128, 1), (256, 1), (128, 2)])
def test_module_backward_matches_stock_bf16(dev, cls, C, B):
    print(f"[trimul module bwd bf16] {cls} C={C} B={B}", flush=True)
    outgoing = cls == "TriangleMulOutgoing"
    m = _modules(getattr(ops, cls), C)
    p = _oracle_params(m)
    g = torch.Generator().manual_seed(1)
    z = torch.randn(B, 133, 133, C, generator=g)
    mask = (torch.rand(B, 133, 133, generator=g) > 0.1).float()
    weight = torch.randn(z.shape, generator=g)
    ref32 = _oracle_grads(p, z, mask, weight, outgoing, False)
    ref16 = _oracle_grads(p, z, mask, weight, outgoing, True)
    m = m.to(dev)
    x = z.to(dev).requires_grad_(True)
    with torch.autocast("cuda", dtype=BF):
        out = m(x, mask.to(dev))
    (out.float() * weight.to(dev)).sum().backward()
    got = {"z": x.grad.float().cpu(), **{k: t.grad.float().cpu() for k, t in m.named_parameters()}}
    for k, ref in ref32.items():
        e_hip, e_stock = rel_l2(got[k], ref), rel_l2(ref16[k], ref)
        print(f"  {k}: hip {e_hip:.2e} stock-bf16 {e_stock:.2e}", flush=True)
        assert e_hip < 3 * e_stock + 1e-3, k


@pytest.mark.parametrize("cls", ["TriangleMulOutgoing", "TriangleMulIncoming"])
def test_module_backward_fp32(dev, cls):
    outgoing = cls == "TriangleMulOutgoing"
    prefix = "tri_mul_out." if outgoing else "tri_mul_in."
    p = sub(W.make_block_weights(31, perturb_affine=True), prefix)
    m = getattr(ops, cls)(128)
    m.load_state_dict(p)
    inp = W.make_inputs(41, seed=32, pad_last=3)
    g = torch.Generator().manual_seed(33)
    weight = torch.randn(1, 41, 41, 128, generator=g)
    want = _oracle_grads({k: v.double() for k, v in p.items()}, inp["pair"].double(), inp["pair_mask"].double(),
                         weight.double(), outgoing, False)  # fmt: skip
    m = m.to(dev)
    x = inp["pair"].to(dev).requires_grad_(True)
    out = m(x, inp["pair_mask"].to(dev))
    (out * weight.to(dev)).sum().backward()
    got = {"z": x.grad.cpu(), **{k: t.grad.cpu() for k, t in m.named_parameters()}}
    for k, ref in want.items():
        assert_fp32_close(got[k], ref.float(), what=f"module d{k}")


def test_trimul_backward_is_deterministic(dev):
    m = _modules(ops.TriangleMulOutgoing, 128).to(dev)
    g = torch.Generator().manual_seed(2)
    z = torch.randn(1, 149, 149, 128, generator=g).to(dev)
    mask = (torch.rand(1, 149, 149, generator=g) > 0.1).float().to(dev)
    grads = []
    for _ in range(2):
        m.zero_grad(set_to_none=True)
        x = z.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=BF):
            m(x, mask).float().pow(2).sum().backward()
        grads.append([x.grad.clone()] + [p.grad.clone() for p in m.parameters()])
    for a, b in zip(*grads):
        assert torch.equal(a, b)
