"""GPU: the RMSNorm branch scaler (branch_scaler="rmsnorm", branch_scaler.py:38-50, applied to
every residual branch at evoformer.py:289-335) and its kernel.

- ``kernels.rms_residual_add`` (pf_rms_residual_add) against float64 torch: res + s x /
  sqrt(mean x^2 + 1e-6) and the scaled branch alone, fp32 (relL2 <= 1e-6) and bf16 (the fp32
  result rounded once: max-abs <= one bf16 ulp of the result), in place, C = 128 and 384.
- A PairFormer block with the scaler against the oracle block (pinned in test_oracle.py):
  eval fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref| with a residual scale of 0.7, with
  and without the single track; bf16 by the reference's rule
  (tests/triton/test_fused_trimul.py:66-83); every gradient under grad against the oracle
  differentiated in fp64 at the fp32 bar.
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, rel_l2, to

pytestmark = pytest.mark.gpu
W = mod("weights")
kernels = mod("kernels")
evoformer = mod("evoformer")
BF = torch.bfloat16


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


@pytest.mark.parametrize("C", [128, 384])
def test_rms_residual_add_kernel(dev, C):
    g = torch.Generator().manual_seed(C)
    res = torch.randn(1000, C, generator=g)
    x = torch.randn(1000, C, generator=g) * (0.1 + 3 * torch.rand(1000, 1, generator=g))
    s = 0.7
    ref = res.double() + s * x.double() / (x.double().pow(2).mean(-1, keepdim=True) + 1e-6).sqrt()
    alone = ref - res.double()
    print(f"[rms residual add] C={C}", flush=True)
    with torch.no_grad():
        got = kernels.rms_residual_add(res.to(dev), x.to(dev), s)
        assert rel_l2(got.cpu(), ref) < 1e-6
        assert rel_l2(kernels.rms_residual_add(None, x.to(dev), s).cpu(), alone) < 1e-6
        inplace = res.to(dev).clone()
        kernels.rms_residual_add(inplace, x.to(dev), s, out=inplace)
        assert torch.equal(inplace, got)
        gb = kernels.rms_residual_add(res.to(dev, BF), x.to(dev, BF), s).float().cpu()
        refb = res.to(BF).double() + s * x.to(BF).double() / (x.to(BF).double().pow(2).mean(-1, keepdim=True)
                                                              + 1e-6).sqrt()  # fmt: skip
    ulp = refb.abs().float() * 2.0**-7 + 1e-30  # one bf16 ulp of the result (8 significant bits)
    assert ((gb.double() - refb).abs() <= ulp.double()).all()


def _block(dev, seed, dtype=torch.float32, single=True):
    sd = W.make_block_weights(seed, perturb_affine=True, use_single_track=single)
    blk = evoformer.PairFormerBlock(128, 384, branch_scaler="rmsnorm", residual_out_scale=0.7, use_single_track=single)
    blk.load_state_dict(sd)
    return blk.to(dev).to(dtype).eval(), sd


@pytest.mark.parametrize("single", [True, False], ids=["single", "no-single"])
def test_rmsnorm_block_eval_fp32(dev, single):
    blk, sd = _block(dev, 81, single=single)
    x = W.make_inputs(36, seed=11, pad_last=3)
    print(f"[rmsnorm block eval fp32] N=36 single={single}", flush=True)
    with torch.no_grad():
        p, s = blk(*(x[k].to(dev) for k in ("pair", "single", "pair_mask", "seq_mask")))
        rp, rs = R.pairformer_block(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], sd,
                                    scales={"residual_out_scale": 0.7}, use_single_track=single,
                                    branch_scaler="rmsnorm")  # fmt: skip
    assert_fp32_close(p.cpu(), rp, what="pair")
    assert_fp32_close(s.cpu(), rs, what="single")


def test_rmsnorm_block_bf16_rule(dev):
    blk, sd = _block(dev, 82, BF)
    x = W.make_inputs(96, seed=12, pad_random=5)
    a = [x[k].to(dev) for k in ("pair", "single", "pair_mask", "seq_mask")]
    kw = dict(scales={"residual_out_scale": 0.7}, branch_scaler="rmsnorm")
    print("[rmsnorm block bf16] N=96", flush=True)
    with torch.no_grad():
        p, s = blk(a[0].to(BF), a[1].to(BF), a[2], a[3])
        with torch.autocast("cuda", dtype=BF):
            ep, es = R.pairformer_block(a[0].to(BF), a[1].to(BF), a[2], a[3], to(sd, dev, BF), **kw)
        rp, rs = R.pairformer_block(a[0], a[1], a[2], a[3], to(sd, dev), **kw)
    assert_bf16_rule(p.cpu(), ep.cpu(), rp.cpu(), "pair")
    assert_bf16_rule(s.cpu(), es.cpu(), rs.cpu(), "single")


def test_rmsnorm_block_backward_fp32(dev):
    blk, sd = _block(dev, 83)
    n = 24
    g = torch.Generator().manual_seed(84)
    pair, single = torch.randn(1, n, n, 128, generator=g), torch.randn(1, n, 384, generator=g)
    pm, sm = torch.ones(1, n, n), torch.ones(1, n)
    sm[:, n - 2 :] = 0.0
    gp, gs = torch.randn(1, n, n, 128, generator=g), torch.randn(1, n, 384, generator=g)
    print("[rmsnorm block backward fp32] N=24", flush=True)
    p0, s0 = pair.to(dev).requires_grad_(True), single.to(dev).requires_grad_(True)
    p, s = blk(p0, s0, pm.to(dev), sm.to(dev))
    ((p * gp.to(dev)).sum() + (s * gs.to(dev)).sum()).backward()
    got = {"pair": p0.grad.cpu(), "single": s0.grad.cpu(), **{k: t.grad.cpu() for k, t in blk.named_parameters()}}
    leaves = {k: v.double().requires_grad_(True) for k, v in sd.items()}
    q0, t0 = pair.double().requires_grad_(True), single.double().requires_grad_(True)
    rp, rs = R.pairformer_block(q0, t0, pm.double(), sm.double(), leaves, scales={"residual_out_scale": 0.7},
                                branch_scaler="rmsnorm")  # fmt: skip
    ((rp * gp.double()).sum() + (rs * gs.double()).sum()).backward()
    ref = {"pair": q0.grad, "single": t0.grad, **{k: t.grad for k, t in leaves.items()}}
    for k in got:
        if k == "single_to_pair_norm.bias":  # zero in exact arithmetic (a per-head logit shift)
            continue
        assert_fp32_close(got[k], ref[k], what=k)
