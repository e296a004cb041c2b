"""GPU: the other pair stacks that call the same primitives.

- The confidence head's PairFormer layers (confidence.py:88-117, run at :304-308): 4 blocks
  of the trunk's shape under the keys layers.{i}.*, against the oracle trunk of 4 blocks.
- TemplatePairFormerBlock (template_embedding.py:180-241): the pair-only block with a
  factor-2 transition, against the oracle's template block (pinned in test_oracle.py to
  the pair half of the golden-pinned PairFormer block).

fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref|; bf16 by the reference's rule
relL2(HIP - fp32) <= 2 relL2(eager bf16 - fp32) (tests/triton/test_fused_trimul.py:66-83).
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, to

pytestmark = pytest.mark.gpu
W = mod("weights")
evoformer = mod("evoformer")
BF = torch.bfloat16
PAIR_KEYS = ("tri_mul_out.", "tri_mul_in.", "pair_attn_row.", "pair_attn_col.", "pair_transition.")


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _confidence(dev, seed, dtype):
    sds = W.make_trunk_weights(seed, 4, perturb_affine=True)
    m = evoformer.ConfidencePairFormer().eval()
    m.load_state_dict({f"layers.{i}.{k}": v for i, sd in enumerate(sds) for k, v in sd.items()})
    return m.to(dev).to(dtype), sds


def test_confidence_layers_fp32(dev):
    m, sds = _confidence(dev, 17, torch.float32)
    x = W.make_inputs(40, seed=5, pad_last=3)
    with torch.no_grad():
        p, s = m(x["pair"].to(dev), x["single"].to(dev), x["pair_mask"].to(dev), x["seq_mask"].to(dev))
        rp, rs = R.pairformer_trunk(x["pair"], x["single"], x["pair_mask"], x["seq_mask"], sds)
    assert_fp32_close(p.cpu(), rp, what="confidence pair")
    assert_fp32_close(s.cpu(), rs, what="confidence single")


def test_confidence_layers_bf16_rule(dev):
    m, sds = _confidence(dev, 18, BF)
    x = {k: v.to(dev) for k, v in W.make_inputs(96, seed=6, pad_random=7).items()}
    pm, sm = x["pair_mask"], x["seq_mask"]
    with torch.no_grad():
        p, s = m(x["pair"].to(BF), x["single"].to(BF), pm, sm)
        with torch.autocast("cuda", dtype=BF):
            ep, es = R.pairformer_trunk(x["pair"].to(BF), x["single"].to(BF), pm, sm, [to(sd, dev, BF) for sd in sds])
        rp, rs = R.pairformer_trunk(x["pair"].to(BF).float(), x["single"].to(BF).float(), pm, sm,
                                    [to(sd, dev) for sd in sds])  # fmt: skip
    print("[confidence bf16]", assert_bf16_rule(p.cpu(), ep.cpu(), rp.cpu(), "confidence pair"),
          assert_bf16_rule(s.cpu(), es.cpu(), rs.cpu(), "confidence single"), flush=True)  # fmt: skip


def _template(dev, seed, dtype):
    sd = W.make_block_weights(seed, perturb_affine=True, factor=2)
    p = {k: v for k, v in sd.items() if k.startswith(PAIR_KEYS)}
    m = evoformer.TemplatePairFormerBlock(128).eval()
    m.load_state_dict(p)
    return m.to(dev).to(dtype), p


@pytest.mark.parametrize("n,pad", [(33, 2), (70, 5)])
def test_template_block_fp32(dev, n, pad):
    m, p = _template(dev, 19, torch.float32)
    x = W.make_inputs(n, seed=n, pad_last=pad)
    with torch.no_grad():
        got = m(x["pair"].to(dev), x["pair_mask"].to(dev))
        ref = R.template_pairformer_block(x["pair"], x["pair_mask"], p)
    assert_fp32_close(got.cpu(), ref, what=f"template block N={n}")


def test_template_block_bf16_rule(dev):
    m, p = _template(dev, 20, BF)
    x = {k: v.to(dev) for k, v in W.make_inputs(100, seed=7, pad_random=6).items()}
    z, pm = x["pair"].to(BF), x["pair_mask"]
    with torch.no_grad():
        got = m(z, pm)
        with torch.autocast("cuda", dtype=BF):
            eager = R.template_pairformer_block(z, pm, to(p, dev, BF))
        ref = R.template_pairformer_block(z.float(), pm, to(p, dev))
    print("[template bf16]", assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), "template block"), flush=True)
