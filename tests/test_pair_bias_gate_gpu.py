"""GPU: the single attention's per-head pair-bias gate (attention.py:392-398, :422-424) inside a
PairFormer block: tau_h = exp(a_h) scales head h's pair logits. Against the oracle block
(whose gate is pinned in test_oracle.py): fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref|
in eval (the in-place path) and under grad (every gradient, the gate's a included, against
the oracle differentiated in fp64); bf16 by the reference's rule against eager bf16
(tests/triton/test_fused_trimul.py:66-83)."""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, to

pytestmark = pytest.mark.gpu
W = mod("weights")
evoformer = mod("evoformer")
BF = torch.bfloat16


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _block(dev, seed, dtype=torch.float32):
    sd = W.make_block_weights(seed, perturb_affine=True, pair_bias_gate=True)
    blk = evoformer.PairFormerBlock(128, 384, pair_bias_gate=True)
    blk.load_state_dict(sd)
    return blk.to(dev).to(dtype).eval(), sd


def test_gated_block_eval_fp32(dev):
    blk, sd = _block(dev, 71)
    x = W.make_inputs(40, seed=8, pad_last=3)
    print("[pair-bias gate block eval fp32] N=40", flush=True)
    with torch.no_grad():
        p, s = blk(*(x[k].to(dev) for k in ("pair", "single", "pair_mask", "seq_mask")))
        rp, rs = R.pairformer_block(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], sd)
    assert_fp32_close(p.cpu(), rp, what="pair")
    assert_fp32_close(s.cpu(), rs, what="single")


def test_gated_block_bf16_rule(dev):
    blk, sd = _block(dev, 72, BF)
    x = W.make_inputs(96, seed=9, pad_random=5)
    args = [x[k].to(dev) for k in ("pair", "single", "pair_mask", "seq_mask")]
    print("[pair-bias gate block bf16] N=96", flush=True)
    with torch.no_grad():
        p, s = blk(args[0].to(BF), args[1].to(BF), args[2], args[3])
        with torch.autocast("cuda", dtype=BF):
            ep, es = R.pairformer_block(args[0].to(BF), args[1].to(BF), args[2], args[3], to(sd, dev, BF))
        rp, rs = R.pairformer_block(args[0], args[1], args[2], args[3], to(sd, dev))
    assert_bf16_rule(p.cpu(), ep.cpu(), rp.cpu(), "pair")
    assert_bf16_rule(s.cpu(), es.cpu(), rs.cpu(), "single")


def test_gated_block_backward_fp32(dev):
    blk, sd = _block(dev, 73)
    n = 24
    g = torch.Generator().manual_seed(74)
    pair, single = torch.randn(1, n, n, 128, generator=g), torch.randn(1, n, 384, generator=g)
    pm, sm = torch.ones(1, n, n), torch.ones(1, n)
    sm[:, n - 2 :] = 0.0
    gp, gs = torch.randn(1, n, n, 128, generator=g), torch.randn(1, n, 384, generator=g)
    print("[pair-bias gate block backward fp32] N=24", flush=True)
    p0, s0 = pair.to(dev).requires_grad_(True), single.to(dev).requires_grad_(True)
    p, s = blk(p0, s0, pm.to(dev), sm.to(dev))
    ((p * gp.to(dev)).sum() + (s * gs.to(dev)).sum()).backward()
    got = {"pair": p0.grad.cpu(), "single": s0.grad.cpu(), **{k: t.grad.cpu() for k, t in blk.named_parameters()}}
    leaves = {k: v.double().requires_grad_(True) for k, v in sd.items()}
    q0, t0 = pair.double().requires_grad_(True), single.double().requires_grad_(True)
    rp, rs = R.pairformer_block(q0, t0, pm.double(), sm.double(), leaves)
    ((rp * gp.double()).sum() + (rs * gs.double()).sum()).backward()
    ref = {"pair": q0.grad, "single": t0.grad, **{k: t.grad for k, t in leaves.items()}}
    for k in ("pair", "single", "single_attn.pair_bias_gate_a", "single_to_pair.weight", "single_attn.to_q.weight"):
        assert_fp32_close(got[k], ref[k], what=k)
