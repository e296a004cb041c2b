"""GPU: the pair kernels at channel counts other than 128.

- Triangle multiplication at 64 channels (the template stack) and 256 (the 256-channel
  trunk), both directions: the generic tile kernels around the same contraction.
- Grid attention at 64 channels in 4 heads of 16 and 256 channels in 8 heads of 32, rows and
  columns: LN and projection row GEMMs, the flash kernel on four-head groups with the head
  dimension zero-padded to 32, gate and output GEMM.
- TemplatePairFormerBlock at its reference width, 64 (template_embedding.py:180-241).
- A PairFormerBlock at 256 pair channels with 8 pair heads (the generic transition and the
  standalone single_to_pair).

Against the oracle (pinned in test_oracle.py, the grid attention by explicit loops at 64
channels in 4 heads as well): fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref|; bf16 by the
reference's rule relL2(HIP - fp32) <= 2 relL2(eager bf16 - fp32)
(tests/triton/test_fused_trimul.py:66-83).
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
ops = mod("ops")
attention = mod("attention")
evoformer = mod("evoformer")
kernels = mod("kernels")
BF = torch.bfloat16


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _z(n: int, c: int, seed: int) -> torch.Tensor:
    return torch.randn(1, n, n, c, generator=torch.Generator().manual_seed(seed))


def _trimul(dev, c, outgoing, seed, dtype):
    prefix = "tri_mul_out." if outgoing else "tri_mul_in."
    p = sub(W.make_block_weights(seed, perturb_affine=True, c_pair=c), prefix)
    m = (ops.TriangleMulOutgoing if outgoing else ops.TriangleMulIncoming)(c).eval()
    m.load_state_dict(p)
    return m.to(dev).to(dtype), p


@pytest.mark.parametrize("outgoing", [True, False], ids=["out", "in"])
@pytest.mark.parametrize("c", [64, 256])
def test_trimul_widths_fp32(dev, c, outgoing):
    m, p = _trimul(dev, c, outgoing, 41, torch.float32)
    x = W.make_inputs(37, seed=3, pad_last=3)
    z = _z(37, c, c)
    print(f"[trimul width fp32] C={c} outgoing={outgoing}", flush=True)
    with torch.no_grad():
        got = m(z.to(dev), x["pair_mask"].to(dev))
        ref = R.tri_mul(z, x["pair_mask"], p, outgoing)
    assert_fp32_close(got.cpu(), ref, what=f"trimul C={c}")


@pytest.mark.parametrize("c", [64, 256])
def test_trimul_widths_bf16_rule(dev, c):
    m, p = _trimul(dev, c, True, 42, BF)
    mask = W.make_inputs(96, seed=4, pad_random=6)["pair_mask"].to(dev)
    z = _z(96, c, 7).to(dev).to(BF)
    with torch.no_grad():
        got = m(z, mask)
        with torch.autocast("cuda", dtype=BF):
            eager = R.tri_mul(z, mask, to(p, dev, BF), True)
        ref = R.tri_mul(z.float(), mask, to(p, dev), True)
    print(f"[trimul width bf16] C={c}", assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), f"trimul C={c}"), flush=True)


def _attn(dev, c, heads, transpose, seed, dtype):
    prefix = "pair_attn_col." if transpose else "pair_attn_row."
    p = sub(W.make_block_weights(seed, perturb_affine=True, c_pair=c, num_pair_heads=heads), prefix)
    m = attention.GridSelfAttention(c, heads, transpose=transpose).eval()
    m.load_state_dict(p)
    return m.to(dev).to(dtype), p


@pytest.mark.parametrize("transpose", [False, True], ids=["rows", "cols"])
@pytest.mark.parametrize("c,heads", [(64, 4), (256, 8)])
def test_grid_attention_widths_fp32(dev, c, heads, transpose):
    m, p = _attn(dev, c, heads, transpose, 43, torch.float32)
    x = W.make_inputs(45, seed=5, pad_last=4)
    z = _z(45, c, c + 1)
    print(f"[grid attention width fp32] C={c} H={heads} transpose={transpose}", flush=True)
    with torch.no_grad():
        got = m(z.to(dev), x["pair_mask"].to(dev))
        ref = R.grid_attention(z, x["pair_mask"], p, transpose)
    assert_fp32_close(got.cpu(), ref, what=f"grid attention C={c} H={heads}")


@pytest.mark.parametrize("c,heads", [(64, 4), (256, 8)])
def test_grid_attention_widths_bf16_rule(dev, c, heads):
    m, p = _attn(dev, c, heads, False, 44, BF)
    mask = W.make_inputs(80, seed=6, pad_random=5)["pair_mask"].to(dev)
    z = _z(80, c, 9).to(dev).to(BF)
    with torch.no_grad():
        got = m(z, mask)
        with torch.autocast("cuda", dtype=BF):
            eager = R.grid_attention(z, mask, to(p, dev, BF), False)
        ref = R.grid_attention(z.float(), mask, to(p, dev), False)
    print(f"[grid attention width bf16] C={c} H={heads}",
          assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), f"grid attention C={c}"), flush=True)  # fmt: skip


def _template64(dev, seed, dtype):
    sd = W.make_block_weights(seed, perturb_affine=True, c_pair=64, factor=2)
    p = {k: v for k, v in sd.items() if k.startswith(("tri_mul_", "pair_attn_", "pair_transition."))}
    m = evoformer.TemplatePairFormerBlock(64).eval()
    m.load_state_dict(p)
    return m.to(dev).to(dtype), p


def test_template_block_c64_fp32(dev):
    m, p = _template64(dev, 45, torch.float32)
    x = W.make_inputs(38, seed=8, pad_last=2)
    z = _z(38, 64, 11)
    print("[template block C=64 fp32] N=38", flush=True)
    with torch.no_grad():
        got = m(z.to(dev), x["pair_mask"].to(dev))
        ref = R.template_pairformer_block(z, x["pair_mask"], p)
    assert_fp32_close(got.cpu(), ref, what="template block C=64")


def test_template_block_c64_bf16_rule(dev):
    m, p = _template64(dev, 46, BF)
    mask = W.make_inputs(72, seed=9, pad_random=4)["pair_mask"].to(dev)
    z = _z(72, 64, 12).to(dev).to(BF)
    with torch.no_grad():
        got = m(z, mask)
        with torch.autocast("cuda", dtype=BF):
            eager = R.template_pairformer_block(z, mask, to(p, dev, BF))
        ref = R.template_pairformer_block(z.float(), mask, to(p, dev))
    print("[template block C=64 bf16]", assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), "template C=64"),
          flush=True)  # fmt: skip


def _block256(dev, seed, dtype):
    sd = W.make_block_weights(seed, perturb_affine=True, c_pair=256, num_pair_heads=8)
    m = evoformer.PairFormerBlock(256, 384, num_pair_heads=8).eval()
    m.load_state_dict(sd)
    return m.to(dev).to(dtype), sd


def test_pairformer_block_c256_fp32(dev):
    m, sd = _block256(dev, 47, torch.float32)
    x = W.make_inputs(30, seed=10, pad_last=2)
    z = _z(30, 256, 13)
    print("[PairFormer block C=256 fp32] N=30", flush=True)
    with torch.no_grad():
        p, s = m(z.to(dev), x["single"].to(dev), x["pair_mask"].to(dev), x["seq_mask"].to(dev))
        rp, rs = R.pairformer_block(z, x["single"], x["pair_mask"], x["seq_mask"], sd)
    assert_fp32_close(p.cpu(), rp, what="block C=256 pair")
    assert_fp32_close(s.cpu(), rs, what="block C=256 single")


def test_pairformer_block_c256_bf16_rule(dev):
    m, sd = _block256(dev, 48, BF)
    x = {k: v.to(dev) for k, v in W.make_inputs(64, seed=11, pad_random=4).items()}
    z = _z(64, 256, 14).to(dev).to(BF)
    single = x["single"].to(BF)
    pm, sm = x["pair_mask"], x["seq_mask"]
    with torch.no_grad():
        p, s = m(z, single, pm, sm)
        with torch.autocast("cuda", dtype=BF):
            ep, es = R.pairformer_block(z, single, pm, sm, to(sd, dev, BF))
        rp, rs = R.pairformer_block(z.float(), single.float(), pm, sm, to(sd, dev))
    print("[PairFormer block C=256 bf16]", assert_bf16_rule(p.cpu(), ep.cpu(), rp.cpu(), "pair"),
          assert_bf16_rule(s.cpu(), es.cpu(), rs.cpu(), "single"), flush=True)  # fmt: skip


@pytest.mark.parametrize("stream_dtype", [torch.float32, BF], ids=["fp32-stream", "bf16-stream"])
@pytest.mark.parametrize("c", [64, 256])
def test_single_to_pair_widths_bf16_rule(dev, c, stream_dtype):
    """The standalone single_to_pair at 64 and 256 channels with bf16 GEMM operands (16
    positions per wave on MFMAs), 70 tokens (a ragged last group of positions)."""
    n = 70
    sd = W.make_block_weights(47, perturb_affine=True, c_pair=c)
    p = {k: v for k, v in sd.items() if k.startswith("single_to_pair")}
    z = _z(n, c, 11)
    with torch.no_grad():
        got = kernels.single_to_pair(z.to(dev, stream_dtype), p["single_to_pair_norm.weight"].to(dev),
                                     p["single_to_pair_norm.bias"].to(dev), 1e-5,
                                     p["single_to_pair.weight"].to(dev, BF))  # fmt: skip
        with torch.autocast("cuda", dtype=BF):
            eager = R.single_to_pair(z.to(dev, stream_dtype), to(p, dev, stream_dtype))
        ref = R.single_to_pair(z, p)
    print(f"[single_to_pair width] C={c} stream={stream_dtype}",
          assert_bf16_rule(got.cpu(), eager.float().cpu(), ref, f"single_to_pair C={c}"), flush=True)  # fmt: skip
