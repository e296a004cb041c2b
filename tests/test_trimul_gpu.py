"""GPU: HIP triangle multiplication against the oracle.

fp32 GEMM regime: relL2 <= 1e-5 and max-abs <= 1e-5 * max|ref| against the fp32
oracle. bf16 regime: relL2(HIP - fp32 oracle) <= 2 x relL2(eager bf16 - fp32 oracle),
the reference's own rule (tests/triton/test_fused_trimul.py:66-83).
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
ops = mod("ops")
kernels = mod("kernels")


def _module(outgoing, p, dev, dtype=torch.float32):
    m = (ops.TriangleMulOutgoing if outgoing else ops.TriangleMulIncoming)(128).to(dev)
    m.load_state_dict(p)
    return m.to(dtype)


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("n,pad", [(24, 3), (64, 0), (130, 7)])
def test_trimul_fp32_matches_oracle(dev, outgoing, n, pad):
    sd = W.make_block_weights(11, perturb_affine=True)
    p = sub(sd, "tri_mul_out." if outgoing else "tri_mul_in.")
    inp = W.make_inputs(n, seed=n, pad_last=pad)
    m = _module(outgoing, p, dev)
    torch.set_float32_matmul_precision("highest")
    with torch.no_grad():
        got = m(inp["pair"].to(dev), inp["pair_mask"].to(dev))
        ref = R.tri_mul(inp["pair"], inp["pair_mask"], p, outgoing)
    print(f"[trimul fp32 out={outgoing} n={n}]", flush=True)
    assert_fp32_close(got.cpu(), ref, what=f"trimul fp32 outgoing={outgoing} N={n}")


@pytest.mark.parametrize("outgoing", [True, False])
# padded 128 / 256 / 512 / 768: every contraction tiling (generic, 256 x 256, 256 x 384)
@pytest.mark.parametrize("n", [96, 200, 500, 700])
def test_trimul_bf16_tolerance_rule(dev, outgoing, n):
    sd = W.make_block_weights(12, perturb_affine=True)
    p = sub(sd, "tri_mul_out." if outgoing else "tri_mul_in.")
    inp = W.make_inputs(n, seed=5, pad_random=6)
    m = _module(outgoing, p, dev, torch.bfloat16)
    zb = inp["pair"].to(dev, torch.bfloat16)
    mb = inp["pair_mask"].to(dev, torch.bfloat16)
    with torch.no_grad():
        got = m(zb, mb)
        eager = R.tri_mul(zb, mb, to(p, dev, torch.bfloat16), outgoing)
        ref = R.tri_mul(zb.float().cpu(), inp["pair_mask"], p, outgoing)
    assert got.dtype == torch.bfloat16
    print("[trimul bf16]", assert_bf16_rule(got.cpu(), eager.cpu(), ref, "trimul bf16"), flush=True)


def test_trimul_autocast_regime_fp32_stream(dev):
    """fp32 z with bf16 GEMMs (the reference inference regime) under autocast."""
    n = 80
    sd = W.make_block_weights(13)
    p = sub(sd, "tri_mul_out.")
    inp = W.make_inputs(n, seed=8)
    m = _module(True, p, dev)
    z = inp["pair"].to(dev)
    mk = inp["pair_mask"].to(dev)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        got = m(z, mk)
        eager = R.tri_mul(z, mk, to(p, dev), True)
    ref = R.tri_mul(inp["pair"], inp["pair_mask"], p, True)
    assert got.dtype == torch.float32
    assert_bf16_rule(got.cpu(), eager.cpu(), ref, "trimul autocast")


def test_trimul_fused_residual_and_batch(dev):
    n = 40
    sd = W.make_block_weights(14, perturb_affine=True)
    p = sub(sd, "tri_mul_in.")
    inp = W.make_inputs(n, seed=9, batch=2, pad_random=3)
    m = _module(False, p, dev)
    z = inp["pair"].to(dev).contiguous()
    mk = inp["pair_mask"].to(dev)
    with torch.no_grad():
        upd = m(z, mk)
        z2 = z.clone()
        m.forward_residual_(z2, mk)
        single = m(z[1], mk[1])
    ref = R.tri_mul(inp["pair"], inp["pair_mask"], p, False)
    assert_fp32_close(upd.cpu(), ref, what="batched")
    assert_fp32_close(single.cpu(), ref[1], what="unbatched")
    assert_fp32_close(z2.cpu(), inp["pair"] + ref, what="fused residual")


def test_fused_trimul_functional_api(dev):
    """kernels.fused_trimul has the reference signature (triton/fused_trimul.py:332-366)."""
    n = 32
    sd = W.make_block_weights(15, perturb_affine=True)
    p = sub(sd, "tri_mul_out.")
    m = _module(True, p, dev)
    inp = W.make_inputs(n, seed=10)
    order = m._block_order.to(dev)
    with torch.no_grad():
        got = kernels.fused_trimul(
            inp["pair"].to(dev), inp["pair_mask"].to(dev), True, m.norm_left, m.gate.weight[order],
            m.proj.weight[order], m.norm_center, m.out_proj.weight, m.out_gate.weight,
        )  # fmt: skip
    ref = R.tri_mul(inp["pair"], inp["pair_mask"], p, True)
    assert_fp32_close(got.cpu(), ref, what="fused_trimul API")


def test_grad_enabled_is_refused(dev):
    """The inference entries refuse grad (fused_trimul.py:332 is inference-only); the module's
    forward under grad takes the differentiable path instead (tests/test_trimul_bwd_gpu.py)."""
    m = _module(True, sub(W.make_block_weights(1), "tri_mul_out."), dev)
    err = mod("inference_guard").InferenceOnlyKernelError
    z, mask = torch.randn(1, 8, 8, 128, device=dev), torch.ones(1, 8, 8, device=dev)
    with pytest.raises(err):
        m.forward_residual_(z, mask)
    with pytest.raises(err):
        kernels.fused_trimul(z, mask, True, m.norm_left, m.gate.weight, m.proj.weight, m.norm_center,
                             m.out_proj.weight, m.out_gate.weight)  # fmt: skip
