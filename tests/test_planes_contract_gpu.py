"""GPU: pf_planes_contract, X[g] = A[g] B[g]^T over G planes (the forward's contraction
kernels, also serving the triangle multiply's VJP cotangents dP = dX Q, dQ = dX^T P).

bf16 at Np = 768 (the 384-wide persistent tiling), 1024 (256-wide) and 384 (the generic
128-wide kernel) by the reference's bf16 rule against the fp32 product
(tests/triton/test_fused_trimul.py:66-83; the eager bf16 product is torch's bf16 batched
matmul with a contiguous right operand); fp32 at Np = 256 against float64 at relL2 <= 1e-5.
"""

from __future__ import annotations

import pytest
import torch

from tests._helpers import assert_bf16_rule, assert_fp32_close, mod

pytestmark = pytest.mark.gpu
_lib = mod("_lib")


def _contract(a, b):
    x = torch.empty_like(a)
    G, Np, _ = a.shape
    _lib.call("pf_planes_contract", a.data_ptr(), b.data_ptr(), x.data_ptr(), G, Np, _lib.dtype_code(a.dtype),
              _lib.stream_of(a))  # fmt: skip
    return x


@pytest.mark.parametrize("G,Np", [(16, 768), (8, 1024), (12, 384)])
def test_planes_contract_bf16_rule(dev, G, Np):
    g = torch.Generator().manual_seed(G + Np)
    a = torch.randn(G, Np, Np, generator=g)
    b = torch.randn(G, Np, Np, generator=g)
    print(f"[planes contract bf16] G={G} Np={Np}", flush=True)
    with torch.no_grad():
        got = _contract(a.to(dev, torch.bfloat16), b.to(dev, torch.bfloat16))
        bt = b.to(dev, torch.bfloat16).transpose(1, 2).contiguous()
        eager = torch.bmm(a.to(dev, torch.bfloat16), bt)
        ref = torch.bmm(a.to(dev), b.to(dev).transpose(1, 2).contiguous())
    assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), f"planes contract G={G} Np={Np}")


def test_planes_contract_fp32(dev):
    torch.set_float32_matmul_precision("highest")
    g = torch.Generator().manual_seed(5)
    a = torch.randn(6, 256, 256, generator=g)
    b = torch.randn(6, 256, 256, generator=g)
    print("[planes contract fp32] G=6 Np=256", flush=True)
    with torch.no_grad():
        got = _contract(a.to(dev), b.to(dev))
    ref = torch.bmm(a.double(), b.double().transpose(1, 2))
    assert_fp32_close(got.cpu(), ref, what="planes contract fp32")
