"""GPU: the Evoformer MSA-stack block (evoformer.py:100-175) and its two MSA operators.

- OuterProductMean (ops.py:683-785): LN + projections, the sequence contraction and the
  out_w contraction on the batched GEMM, the mask-count normalisation.
- MSAAttention (attention.py:272-341): pair-weighted averaging, shared weights per batch
  item and head, values averaged on the batched GEMM.
- EvoformerBlock: OPM -> MSA attention -> MSA transition -> the PairFormer pair half, with
  and without a residual scale; a two-block stack equals the blocks in order.

Against the oracle (its OPM and MSA attention pinned by explicit loops, the block by
composition, in test_oracle.py): fp32 at relL2 <= 1e-5 and max-abs <= 1e-5 max|ref|; bf16
by the reference's rule relL2(HIP - fp32) <= 2 relL2(eager bf16 - fp32).
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
BF = torch.bfloat16


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _msa_inputs(S: int, N: int, seed: int, cm: int = 64, cz: int = 128):
    g = torch.Generator().manual_seed(seed)
    msa = torch.randn(1, S, N, cm, generator=g)
    pair = torch.randn(1, N, N, cz, generator=g)
    mask = (torch.rand(1, S, N, generator=g) > 0.15).float()
    mask[:, :, N - 2 :] = 0.0  # two padded residues, absent from every sequence
    seq = (mask.max(dim=1).values > 0).float()
    pair_mask = seq[:, :, None] * seq[:, None, :]
    return msa, pair, mask, pair_mask


def _opm(dev, seed, dtype):
    p = sub(W.make_evoformer_block_weights(seed, perturb_affine=True), "outer_product.")
    m = ops.OuterProductMean(64, 128).eval()
    m.load_state_dict(p)
    return m.to(dev).to(dtype), p


@pytest.mark.parametrize("S,N", [(5, 19), (70, 33)])
def test_outer_product_mean_fp32(dev, S, N):
    m, p = _opm(dev, 61, torch.float32)
    msa, _, mask, _ = _msa_inputs(S, N, S + N)
    print(f"[OPM fp32] S={S} N={N}", flush=True)
    with torch.no_grad():
        got = m(msa.to(dev), mask.to(dev))
        ref = R.outer_product_mean(msa, mask, p)
    assert_fp32_close(got.cpu(), ref, what=f"OPM S={S} N={N}")


def test_outer_product_mean_bf16_rule(dev):
    m, p = _opm(dev, 62, BF)
    msa, _, mask, _ = (t.to(dev) for t in _msa_inputs(64, 96, 3))
    msa = msa.to(BF)
    with torch.no_grad():
        got = m(msa, mask)
        with torch.autocast("cuda", dtype=BF):
            eager = R.outer_product_mean(msa, mask, to(p, dev, BF))
        ref = R.outer_product_mean(msa.float(), mask, to(p, dev))
    print("[OPM bf16]", assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), "OPM"), flush=True)


def _pav(dev, seed, dtype):
    p = sub(W.make_evoformer_block_weights(seed, perturb_affine=True), "row_attn.")
    m = attention.MSAAttention(64, 128, num_heads=8).eval()
    m.load_state_dict(p)
    return m.to(dev).to(dtype), p


@pytest.mark.parametrize("S,N", [(3, 21), (40, 70)])
def test_msa_attention_fp32(dev, S, N):
    m, p = _pav(dev, 63, torch.float32)
    msa, pair, mask, _ = _msa_inputs(S, N, S * N)
    print(f"[MSA attention fp32] S={S} N={N}", flush=True)
    with torch.no_grad():
        got = m(msa.to(dev), mask.to(dev), pair.to(dev))
        ref = R.msa_attention(msa, mask, pair, p, 8)
    assert_fp32_close(got.cpu(), ref, what=f"MSA attention S={S} N={N}")


def test_msa_attention_bf16_rule(dev):
    m, p = _pav(dev, 64, BF)
    msa, pair, mask, _ = (t.to(dev) for t in _msa_inputs(48, 80, 4))
    msa, pair = msa.to(BF), pair.to(BF)
    with torch.no_grad():
        got = m(msa, mask, pair)
        with torch.autocast("cuda", dtype=BF):
            eager = R.msa_attention(msa, mask, pair, to(p, dev, BF), 8)
        ref = R.msa_attention(msa.float(), mask, pair.float(), to(p, dev), 8)
    print("[MSA attention bf16]", assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), "MSA attention"), flush=True)


def _block(dev, seed, dtype, s=1.0):
    sd = W.make_evoformer_block_weights(seed, perturb_affine=True)
    m = evoformer.EvoformerBlock(64, 128, residual_out_scale=s).eval()
    m.load_state_dict(sd)
    return m.to(dev).to(dtype), sd


@pytest.mark.parametrize("scale", [1.0, 0.5])
def test_evoformer_block_fp32(dev, scale):
    m, sd = _block(dev, 65, torch.float32, scale)
    msa, pair, mask, pm = _msa_inputs(6, 29, 7)
    print(f"[Evoformer block fp32] s={scale}", flush=True)
    with torch.no_grad():
        gm, gp = m(msa.to(dev), pair.to(dev), mask.to(dev), pm.to(dev))
        rm, rp = R.evoformer_block(msa, pair, mask, pm, sd, residual_out_scale=scale)
    assert_fp32_close(gm.cpu(), rm, what="Evoformer block msa")
    assert_fp32_close(gp.cpu(), rp, what="Evoformer block pair")


def test_evoformer_block_bf16_rule(dev):
    m, sd = _block(dev, 66, BF)
    msa, pair, mask, pm = (t.to(dev) for t in _msa_inputs(32, 64, 8))
    msa, pair = msa.to(BF), pair.to(BF)
    with torch.no_grad():
        gm, gp = m(msa, pair, mask, pm)
        with torch.autocast("cuda", dtype=BF):
            em, ep = R.evoformer_block(msa, pair, mask, pm, to(sd, dev, BF))
        rm, rp = R.evoformer_block(msa.float(), pair.float(), mask, pm, to(sd, dev))
    print("[Evoformer block bf16]", assert_bf16_rule(gm.cpu(), em.cpu(), rm.cpu(), "msa"),
          assert_bf16_rule(gp.cpu(), ep.cpu(), rp.cpu(), "pair"), flush=True)  # fmt: skip


def test_evoformer_stack_is_blocks_in_order(dev):
    st = evoformer.EvoformerStack(2).eval()
    for i, blk in enumerate(st.msa_stack):
        blk.load_state_dict(W.make_evoformer_block_weights(70 + i, perturb_affine=True))
    st = st.to(dev).to(BF)
    msa, pair, mask, pm = (t.to(dev) for t in _msa_inputs(16, 48, 9))
    msa, pair = msa.to(BF), pair.to(BF)
    with torch.no_grad():
        sm, sp = st(msa, pair, mask, pm)
        m1, p1 = st.msa_stack[0](msa, pair, mask, pm)
        m2, p2 = st.msa_stack[1](m1, p1, mask, pm)
    assert torch.equal(sm, m2) and torch.equal(sp, p2)
