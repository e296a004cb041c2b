"""GPU: a whole PairFormer block (and a two-block stack) differentiated on the HIP kernels.

Under grad, ``PairFormerBlock.forward`` runs every branch's training path: triangle
multiplications (``FusedTriMulFunction``), row and column attention and single attention on
the fused attention op with its backward, transitions with the HIP LayerNorm and SwiGLU,
residual scales folded into the output projections. Checked against the oracle block
(``pairformer_block``, pinned to the reference's golden outputs) differentiated in fp64: fp32
at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref| for the gradients of both inputs and every
parameter; and in the reference's regime (fp32 streams under bf16 autocast) each gradient
within 3x the stock path's bf16-autocast error + 1e-3 (the reference's
test_fused_backward_matches_stock rule, tests/triton/test_fused_trimul.py:87-106), the stock
references on the CPU. Pair masks without fully masked lines: there the fused attention
kernel's rule (output 0) and the stock rule (mean of V) differ by design. The gradient of
``single_to_pair_norm.bias`` is zero in exact arithmetic (that bias adds one constant per head
to every pair logit, and the softmax is invariant to it): there both sides are rounding noise,
compared on the scale of the largest gradient instead.
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_fp32_close, mod, rel_l2

pytestmark = pytest.mark.gpu
W = mod("weights")
evoformer = mod("evoformer")
BF = torch.bfloat16
STRUCTURAL_ZERO = ("single_to_pair_norm.bias",)


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _inputs(N, seed):
    g = torch.Generator().manual_seed(seed)
    pair = torch.randn(1, N, N, 128, generator=g)
    single = torch.randn(1, N, 384, generator=g)
    pm = (torch.rand(1, N, N, generator=g) > 0.1).float()
    pm[:, :, 0] = 1.0
    pm[:, 0, :] = 1.0
    sm = torch.ones(1, N)
    sm[:, N - 2 :] = 0.0  # padded residues: masked keys of the single attention
    gp = torch.randn(1, N, N, 128, generator=g)
    gs = torch.randn(1, N, 384, generator=g)
    return pair, single, pm, sm, gp, gs


def _oracle_grads(sd, pair, single, pm, sm, gp, gs, dtype, autocast=False, scales=None):
    leaves = {k: v.to(dtype).clone().requires_grad_(True) for k, v in sd.items()}
    p0, s0 = pair.to(dtype).clone().requires_grad_(True), single.to(dtype).clone().requires_grad_(True)
    with torch.autocast("cpu", dtype=BF, enabled=autocast):
        p, s = R.pairformer_block(p0, s0, pm.to(dtype), sm.to(dtype), leaves, scales=scales)
    ((p.to(dtype) * gp.to(dtype)).sum() + (s.to(dtype) * gs.to(dtype)).sum()).backward()
    return {"pair": p0.grad.float(), "single": s0.grad.float(), **{k: t.grad.float() for k, t in leaves.items()}}


def _hip_grads(blk, pair, single, pm, sm, gp, gs, dev, autocast=False):
    blk.zero_grad(set_to_none=True)
    p0, s0 = pair.to(dev).requires_grad_(True), single.to(dev).requires_grad_(True)
    with torch.autocast("cuda", dtype=BF, enabled=autocast):
        p, s = blk(p0, s0, pm.to(dev), sm.to(dev))
    ((p.float() * gp.to(dev)).sum() + (s.float() * gs.to(dev)).sum()).backward()
    return {"pair": p0.grad.float().cpu(), "single": s0.grad.float().cpu(),
            **{k: t.grad.float().cpu() for k, t in blk.named_parameters()}}  # fmt: skip


@pytest.mark.parametrize("scaled", [False, True], ids=["unscaled", "scaled"])
def test_block_backward_fp32(dev, scaled):
    sd = W.make_block_weights(61, perturb_affine=True)
    kw = dict(residual_out_scale=0.7, pair_transition_residual_gain=0.5) if scaled else {}
    blk = evoformer.PairFormerBlock(128, 384, **kw)
    blk.load_state_dict(sd)
    blk = blk.to(dev).eval()  # eval mode: no dropout (training mode: tests/test_train_mode_gpu.py)
    args = _inputs(30, 62)
    print(f"[block backward fp32] N=30 scaled={scaled}", flush=True)
    scales = {"residual_out_scale": 0.7, "pair_transition_residual_gain": 0.5} if scaled else None
    want = _oracle_grads(sd, *args, torch.float64, scales=scales)
    got = _hip_grads(blk, *args, dev)
    assert set(got) == set(want)
    scale = max(float(r.abs().max()) for r in want.values())
    for k, ref in want.items():
        if k in STRUCTURAL_ZERO:
            assert float(ref.abs().max()) <= 1e-5 * scale and float(got[k].abs().max()) <= 1e-5 * scale, k
            continue
        assert_fp32_close(got[k], ref, what=f"block d{k}")


def test_block_backward_bf16_autocast(dev):
    sd = W.make_block_weights(63, perturb_affine=True)
    blk = evoformer.PairFormerBlock(128, 384)
    blk.load_state_dict(sd)
    blk = blk.to(dev).eval()
    args = _inputs(64, 64)
    print("[block backward bf16 autocast] N=64", flush=True)
    ref32 = _oracle_grads(sd, *args, torch.float32)
    ref16 = _oracle_grads(sd, *args, torch.float32, autocast=True)
    got = _hip_grads(blk, *args, dev, autocast=True)
    worst = []
    scale = max(float(r.abs().max()) for r in ref32.values())
    for k, ref in ref32.items():
        if k in STRUCTURAL_ZERO:
            assert float(got[k].abs().max()) <= 1e-3 * scale, k
            continue
        e_hip, e_stock = rel_l2(got[k], ref), rel_l2(ref16[k], ref)
        worst.append((e_hip / max(e_stock, 1e-12), k, e_hip, e_stock))
        assert e_hip < 3 * e_stock + 1e-3, (k, e_hip, e_stock)
    r, k, e_hip, e_stock = max(worst)
    print(f"  worst ratio {r:.2f} at {k}: hip {e_hip:.2e} stock-bf16 {e_stock:.2e}", flush=True)


def test_stack_backward_is_blocks_in_order(dev):
    sds = W.make_trunk_weights(65, 2, perturb_affine=True)
    stack = evoformer.PairFormerStack(2, 128, 384)
    for blk, sd in zip(stack.blocks, sds):
        blk.load_state_dict(sd)
    stack = stack.to(dev).eval()
    pair, single, pm, sm, gp, gs = _inputs(24, 66)
    p0, s0 = pair.to(dev).requires_grad_(True), single.to(dev).requires_grad_(True)
    p, s = stack(p0, s0, pm.to(dev), sm.to(dev))
    ((p * gp.to(dev)).sum() + (s * gs.to(dev)).sum()).backward()
    leaves = [[{k: v.double().clone().requires_grad_(True) for k, v in sd.items()} for sd in sds]][0]
    rp0, rs0 = pair.double().requires_grad_(True), single.double().requires_grad_(True)
    rp, rs = R.pairformer_trunk(rp0, rs0, pm.double(), sm.double(), leaves)
    ((rp * gp.double()).sum() + (rs * gs.double()).sum()).backward()
    assert_fp32_close(p0.grad.cpu(), rp0.grad.float(), what="stack dpair")
    assert_fp32_close(s0.grad.cpu(), rs0.grad.float(), what="stack dsingle")
    for i, blk in enumerate(stack.blocks):
        for k, t in blk.named_parameters():
            if k in STRUCTURAL_ZERO:
                continue
            assert_fp32_close(t.grad.cpu(), leaves[i][k].grad.float(), what=f"stack block {i} d{k}")
