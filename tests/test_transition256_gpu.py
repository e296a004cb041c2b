"""GPU: the pair transition at 256 channels (factor 4) with bf16 z and GEMM operands
(reference ``primitives.py:193-251``, ``triton/fused_transition.py:34-83`` at the production
width of ``configs/stage0.yaml:54-56``).

This regime runs the fused weight-streaming kernel (hidden activations on chip, 128-position
tiles, 32 hidden chunks of 32 units). Checked against the fp32 oracle by the bf16 rule
(relL2(HIP - fp32) <= 2 relL2(eager bf16 - fp32)) for M a multiple of the tile and ragged
(M = 1369, 4000, 16384), stored and added into an existing output (the in-place residual of
the block), and the module in a C=256 block against the composed kernels' path (fp32
stream under autocast, which keeps the composed kernels) by the same rule.
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, mod, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
primitives = mod("primitives")

BF = torch.bfloat16
C = 256


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _block(dev, seed):
    p = sub(W.make_block_weights(seed, perturb_affine=True, c_pair=C, num_pair_heads=8), "pair_transition.")
    m = primitives.TransitionBlock(C, 4).eval()
    m.load_state_dict(p)
    return m.to(dev).to(BF), p


@pytest.mark.parametrize("m_rows", [1369, 4000, 16384])
def test_transition256_bf16_rule(dev, m_rows):
    m, p = _block(dev, 110 + m_rows % 7)
    g = torch.Generator().manual_seed(m_rows)
    x = torch.randn(m_rows, C, generator=g).to(dev, BF)
    print(f"[transition256] M={m_rows}", flush=True)
    with torch.no_grad():
        got, _ = m.run(x)
        with torch.autocast("cuda", dtype=BF):
            eager = R.transition(x, to(p, dev, BF))
        ref = R.transition(x.float(), to(p, dev))
    assert bool(torch.isfinite(got).all())
    print(f"[transition256 M={m_rows}]",
          assert_bf16_rule(got.float().cpu(), eager.float().cpu(), ref.cpu(), f"transition256 M={m_rows}"), flush=True)  # fmt: skip


def test_transition256_accumulate(dev):
    """out += transition(x) in place (out is x): equal to x + transition(x) up to the rounding
    of the separately stored update."""
    m, _ = _block(dev, 117)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(5000, C, generator=g).to(dev, BF)
    with torch.no_grad():
        upd, _ = m.run(x)
        got, _ = m.run(x, out=x.clone(), accumulate=True)
        inplace = x.clone()
        m.run(inplace, out=inplace, accumulate=True)
    want = x.float() + upd.float()
    tol = 2.0**-7 * want.abs().max().item()
    assert (got.float() - want).abs().max().item() <= tol
    assert torch.equal(inplace, got)


def test_transition256_matches_composed_path(dev):
    """The fused kernel against the composed LN + GEMM path the fp32 stream takes under
    autocast (same bf16 GEMM operands), both against the oracle by the bf16 rule."""
    m, p = _block(dev, 118)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(3000, C, generator=g).to(dev)
    with torch.no_grad():
        fused_out, _ = m.run(x.to(BF))
        with torch.autocast("cuda", dtype=BF):
            composed = m.float().run(x)[0]
            eager = R.transition(x.to(BF), to(p, dev, BF))
        ref = R.transition(x, to(p, dev))
    for got, what in ((fused_out, "fused"), (composed, "composed")):
        print(f"[transition256 {what}]",
              assert_bf16_rule(got.float().cpu(), eager.float().cpu(), ref.cpu(), what), flush=True)  # fmt: skip
