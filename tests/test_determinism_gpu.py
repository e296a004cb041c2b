"""GPU: bitwise reproducibility, after the reference's rerun test
(tests/triton/test_evo_attn_robustness.py:1401-1447: same inputs, reruns bitwise equal).

The kernels use no atomics and a static tile-to-workgroup map, so every output element is
accumulated in a fixed order: reruns must agree bit for bit -- the trunk through its
two-stream path, and each hot-path op on its own (the kernel-level attention op is covered
in test_attn_edge_gpu.py)."""

from __future__ import annotations

import pytest
import torch

from tests._helpers import mod, sub

pytestmark = pytest.mark.gpu
W = mod("weights")
evoformer = mod("evoformer")
ops = mod("ops")
attention = mod("attention")
primitives = mod("primitives")
BF = torch.bfloat16


def _same(fn, runs: int = 5):
    with torch.no_grad():
        first = fn()
        first = tuple(t.clone() for t in first) if isinstance(first, tuple) else first.clone()
        for i in range(1, runs):
            again = fn()
            pairs = zip(first, again) if isinstance(first, tuple) else [(first, again)]
            for a, b in pairs:
                assert torch.equal(a, b), f"rerun {i} differs (max {(a.float() - b.float()).abs().max().item():.3e})"


@pytest.mark.parametrize("stream_dtype", [BF, torch.float32])
def test_trunk_reruns_bitwise(dev, stream_dtype):
    """An 8-block stack (two-stream path) at N=200, 10 tokens padded, bf16 GEMM operands."""
    stack = evoformer.PairFormerStack(8).eval()
    for blk, sd in zip(stack.blocks, W.make_trunk_weights(21, 8)):
        blk.load_state_dict(sd)
    stack = stack.to(dev).to(stream_dtype)
    x = {k: v.to(dev) for k, v in W.make_inputs(200, seed=21, pad_random=10).items()}
    pair, single = x["pair"].to(stream_dtype), x["single"].to(stream_dtype)

    def run():
        with torch.autocast("cuda", dtype=BF, enabled=stream_dtype == torch.float32):
            return stack(pair, single, x["pair_mask"], x["seq_mask"])

    _same(run, runs=3)


def test_ops_rerun_bitwise(dev):
    sd = W.make_block_weights(22, perturb_affine=True)
    x = {k: v.to(dev) for k, v in W.make_inputs(300, seed=22, pad_random=12).items()}
    z, pm = x["pair"].to(BF), x["pair_mask"]
    s, sm = x["single"].to(BF), x["seq_mask"]
    for name, cls in (("tri_mul_out.", ops.TriangleMulOutgoing), ("tri_mul_in.", ops.TriangleMulIncoming)):
        m = cls(128).to(dev)
        m.load_state_dict(sub(sd, name))
        m = m.to(BF)
        _same(lambda: m(z, pm))
    for transpose, name in ((False, "pair_attn_row."), (True, "pair_attn_col.")):
        a = attention.GridSelfAttention(128, 4, transpose=transpose).to(dev)
        a.load_state_dict(sub(sd, name))
        a = a.to(BF)
        _same(lambda: a(z, pm))
    t = primitives.TransitionBlock(128, 4).to(dev)
    t.load_state_dict(sub(sd, "pair_transition."))
    t = t.to(BF)
    _same(lambda: t(z))
    sa = attention.SingleAttention(384).to(dev)
    sa.load_state_dict(sub(sd, "single_attn."))
    sa = sa.to(BF)
    pl = torch.randn((1, 16, 300, 300), generator=torch.Generator().manual_seed(3)).to(dev)
    _same(lambda: sa(s, sm, pl))
