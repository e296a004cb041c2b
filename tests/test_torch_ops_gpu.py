"""GPU: the registered ``deepfold3_amd::*`` operators run the same HIP kernels as the
functional wrappers (bit for bit), trace whole under ``torch.compile`` (``aot_eager``: the
graph keeps each op as one node, no generated kernels), and the attention op's registered
autograd formula (the HIP backward) gives the gradients of ``_EvoAttnFunction``."""

from __future__ import annotations

import pytest
import torch

from tests._helpers import mod

pytestmark = pytest.mark.gpu
T = mod("torch_ops")
kernels = mod("kernels")
fused = mod("fused")


def _evo_inputs(dev, dtype, N=72, S=6, seed=0):
    g = torch.Generator().manual_seed(seed)
    q, k, v = ((torch.randn(1, S, 4, N, 32, generator=g) * 32**-0.5).to(dev, dtype) for _ in range(3))
    keep = torch.rand(1, S, N, generator=g) > 0.1
    rm = torch.where(keep, 0.0, float("-inf")).to(dev)
    pb = torch.randn(1, 4, N, N, generator=g).to(dev)
    return q, k, v, rm, pb


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ops_equal_wrappers(dev, dtype):
    print(f"[torch ops == wrappers {dtype}]", flush=True)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 40, 40, 128, generator=g).to(dev, dtype)
    w, b = torch.randn(128, generator=g).to(dev), torch.randn(128, generator=g).to(dev)
    with torch.no_grad():
        assert torch.equal(T.layer_norm(x, w, b, 1e-5), kernels.layer_norm(x, w, b, 1e-5))
        assert torch.equal(T.ln_transpose(x, w, b, 1e-5, True), kernels.ln_transpose(x, w, b, 1e-5, True))
        h = torch.randn(2, 50, 1024, generator=g).to(dev, dtype)
        assert torch.equal(T.swiglu(h), kernels.SwiGLUFunction.apply(h))
        cdt = dtype
        wp, wg = (torch.randn(256, 128, generator=g).to(dev) * 0.05 for _ in range(2))
        packed = kernels.pack_trimul_weights(wp, wg, cdt)
        wo, wog = ((torch.randn(128, 128, generator=g) * 0.05).to(dev, cdt) for _ in range(2))
        mask = (torch.rand(1, 40, 40, generator=g) > 0.1).float().to(dev)
        for outgoing in (True, False):
            args = (x, mask, w, b, 1e-5, packed, w, b, 1e-5, wo, wog, outgoing)
            assert torch.equal(T.trimul(*args), kernels.trimul_forward(*args))
        q, k, v, rm, pb = _evo_inputs(dev, dtype)
        assert torch.equal(T.evo_attention(q, k, v, rm, pb, True), fused._evo_fwd(q, k, v, rm, pb, True))


def test_compile_traces_whole_graph(dev):
    print("[torch ops under torch.compile aot_eager]", flush=True)
    q, k, v, rm, pb = _evo_inputs(dev, torch.bfloat16, seed=2)
    w, b = torch.ones(128, device=dev), torch.zeros(128, device=dev)
    z = torch.randn(1, 24, 24, 128, generator=torch.Generator().manual_seed(3)).to(dev, torch.bfloat16)

    def fn(q, k, v, rm, pb, z):
        o = T.evo_attention(q * 1.0, k, v, rm, pb, True)
        return o.float().sum(-1), T.ln_transpose(z, w, b, 1e-5, True) + 1.0

    with torch.no_grad():
        ref = fn(q, k, v, rm, pb, z)
        got = torch.compile(fn, backend="aot_eager", fullgraph=True)(q, k, v, rm, pb, z)
    for a, r in zip(got, ref):
        assert torch.equal(a, r)


def test_evo_attention_autograd(dev):
    print("[torch op evo_attention backward]", flush=True)
    q, k, v, rm, pb = _evo_inputs(dev, torch.bfloat16, seed=4)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(5)).to(dev, q.dtype)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v)] + [pb.clone().requires_grad_(True)]
    T.evo_attention(leaves[0], leaves[1], leaves[2], rm, leaves[3], True).backward(do)
    ref = [t.clone().requires_grad_(True) for t in (q, k, v)] + [pb.clone().requires_grad_(True)]
    fused._EvoAttnFunction.apply(ref[0], ref[1], ref[2], rm, ref[3]).backward(do)
    for a, r, name in zip(leaves, ref, ("dq", "dk", "dv", "dpb")):
        assert torch.equal(a.grad, r.grad), name
