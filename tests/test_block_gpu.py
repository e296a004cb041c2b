"""GPU: HIP triangle attention, transitions, single track and the whole PairFormer block.

fp32 GEMM regime: relL2 <= 1e-5 and max-abs <= 1e-5 * max|ref| against the fp32 oracle
(the CPU restatement of the reference, pinned to reference golden vectors in
tests/test_oracle.py). bf16 regime: relL2(HIP - fp32 oracle) <= 2 x relL2(eager bf16 -
fp32 oracle), the reference's own rule (tests/triton/test_fused_trimul.py:66-83).
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, rel_l2, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
attention = mod("attention")
primitives = mod("primitives")
evoformer = mod("evoformer")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _grid(transpose, p, dev, dtype=torch.float32):
    m = attention.GridSelfAttention(128, 4, transpose=transpose).to(dev)
    m.load_state_dict(p)
    return m.to(dtype)


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("n,pad", [(24, 3), (64, 0), (130, 7)])
def test_grid_attention_fp32(dev, transpose, n, pad):
    print(f"[grid attn fp32 transpose={transpose} n={n} pad={pad}]", flush=True)
    sd = W.make_block_weights(21, perturb_affine=True)
    p = sub(sd, "pair_attn_col." if transpose else "pair_attn_row.")
    inp = W.make_inputs(n, seed=n + 1, pad_last=pad)
    m = _grid(transpose, p, dev)
    with torch.no_grad():
        got = m(inp["pair"].to(dev), inp["pair_mask"].to(dev))
        ref = R.grid_attention(inp["pair"], inp["pair_mask"], p, transpose)
    assert_fp32_close(got.cpu(), ref, what=f"grid attention transpose={transpose} N={n}")


def test_grid_attention_fully_masked_line_is_mean_of_v(dev):
    """A fully masked line attends uniformly over all N keys (eager rule, attention.py:157-160)."""
    n = 40
    sd = W.make_block_weights(22, perturb_affine=True)
    p = sub(sd, "pair_attn_row.")
    inp = W.make_inputs(n, seed=3)
    mask = inp["pair_mask"].clone()
    mask[0, 5, :] = 0.0  # line 5: every key masked
    mask[0, :, 9] = 0.0  # key 9 masked on every line
    m = _grid(False, p, dev)
    with torch.no_grad():
        got = m(inp["pair"].to(dev), mask.to(dev))
        ref = R.grid_attention(inp["pair"], mask, p, False)
    assert_fp32_close(got.cpu(), ref, what="masked lines")


@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("n", [96, 130])
def test_grid_attention_bf16_rule(dev, transpose, n):
    print(f"[grid attn bf16 transpose={transpose} n={n}]", flush=True)
    sd = W.make_block_weights(23, perturb_affine=True)
    p = sub(sd, "pair_attn_col." if transpose else "pair_attn_row.")
    inp = W.make_inputs(n, seed=4, pad_random=6)
    m = _grid(transpose, p, dev, torch.bfloat16)
    zb = inp["pair"].to(dev, torch.bfloat16)
    mb = inp["pair_mask"].to(dev, torch.bfloat16)
    with torch.no_grad():
        got = m(zb, mb)
        eager = R.grid_attention(zb, mb, to(p, dev, torch.bfloat16), transpose)
        ref = R.grid_attention(zb.float().cpu(), inp["pair_mask"], p, transpose)
    print("[grid bf16]", assert_bf16_rule(got.cpu(), eager.cpu(), ref, "grid attention bf16"), flush=True)


def test_grid_attention_residual_in_place(dev):
    n = 48
    sd = W.make_block_weights(24, perturb_affine=True)
    p = sub(sd, "pair_attn_col.")
    inp = W.make_inputs(n, seed=5, batch=2, pad_random=4)
    m = _grid(True, p, dev)
    z = inp["pair"].to(dev).contiguous()
    with torch.no_grad():
        m.forward_residual_(z, inp["pair_mask"].to(dev))
    ref = inp["pair"] + R.grid_attention(inp["pair"], inp["pair_mask"], p, True)
    assert_fp32_close(z.cpu(), ref, what="fused residual, batch 2")


@pytest.mark.parametrize("transpose", [False, True])
def test_grid_attention_bf16_accumulate_into_other_stream(dev, transpose):
    """bf16 path, out != z with accumulate: the output kernel adds the update to out's rows
    (not z's), with the gate still taken from z; in place it adds to z. Both against the
    plain update (accumulate off) plus the stream, within one bf16 rounding of the sum."""
    n = 70
    sd = W.make_block_weights(25, perturb_affine=True)
    p = sub(sd, "pair_attn_col." if transpose else "pair_attn_row.")
    inp = W.make_inputs(n, seed=8, batch=2, pad_random=5)
    m = _grid(transpose, p, dev, torch.bfloat16)
    z = inp["pair"].to(dev, torch.bfloat16).contiguous()
    mask = inp["pair_mask"].to(dev)
    gen = torch.Generator().manual_seed(9)
    stream = torch.randn(z.shape, generator=gen).to(dev, torch.bfloat16)
    print(f"[grid bf16 accumulate transpose={transpose}]", flush=True)
    with torch.no_grad():
        upd = m(z, mask).float()
        other = stream.clone()
        m._run(z, mask, other, True)
        inplace = z.clone()
        m.forward_residual_(inplace, mask)
    for got, base, what in ((other, stream, "other stream"), (inplace, z, "in place")):
        want = base.float() + upd
        err = (got.float() - want).abs()
        tol = 2.0 ** -7 * want.abs() + 2.0 ** -7 * upd.abs() + 1e-6
        assert bool((err <= tol).all()), f"{what}: max err {err.max().item():.3e}"


@pytest.mark.parametrize("stream_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [24, 70, 130])
def test_pair_transition_and_fused_single_to_pair_bf16_rule(dev, n, stream_dtype):
    """bf16 GEMM kernel (persistent, 256-position tiles; N^2 not a multiple of the tile), the
    residual it adds and the fused single_to_pair logits, by the bf16 rule against the fp32
    oracle; bf16 residual stream or fp32 stream under autocast."""
    print(f"[pair transition bf16 n={n} stream={stream_dtype}]", flush=True)
    sd = W.make_block_weights(28, perturb_affine=True)
    p = sub(sd, "pair_transition.")
    inp = W.make_inputs(n, seed=12)
    blk = primitives.TransitionBlock(128, 4).to(dev)
    blk.load_state_dict(p)
    blk = blk.to(stream_dtype)
    x = inp["pair"].to(dev, stream_dtype).contiguous()
    x0 = x.clone()
    ks = ("single_to_pair_norm.weight", "single_to_pair_norm.bias", "single_to_pair.weight")
    s2p = (sd[ks[0]].to(dev), sd[ks[1]].to(dev), 1e-5, sd[ks[2]].to(dev, torch.bfloat16))  # cast to the GEMM dtype
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        y = blk(x)
        _, logits = blk.forward_residual_(x, s2p=s2p)
        ey = R.transition(x0, to(p, dev, stream_dtype))
        el = R.single_to_pair((x0 + ey).to(stream_dtype), to(sd, dev, stream_dtype))
    ry = R.transition(x0.float().cpu(), p)
    rl = R.single_to_pair(x0.float().cpu() + ry, sd)
    print("  update", assert_bf16_rule(y.cpu(), ey.cpu(), ry, "pair transition bf16"), flush=True)
    print("  residual", assert_bf16_rule(x.cpu(), (x0 + ey).cpu(), x0.float().cpu() + ry, "residual"), flush=True)
    print("  s2p", assert_bf16_rule(logits.cpu(), el.cpu(), rl, "single_to_pair bf16"), flush=True)


@pytest.mark.parametrize("n", [24, 70])
def test_pair_transition_and_fused_single_to_pair_fp32(dev, n):
    sd = W.make_block_weights(25, perturb_affine=True)
    p = sub(sd, "pair_transition.")
    inp = W.make_inputs(n, seed=6)
    blk = primitives.TransitionBlock(128, 4).to(dev)
    blk.load_state_dict(p)
    x = inp["pair"].to(dev).contiguous()
    s2p = (sd["single_to_pair_norm.weight"].to(dev), sd["single_to_pair_norm.bias"].to(dev), 1e-5,
           sd["single_to_pair.weight"].to(dev))  # fmt: skip
    with torch.no_grad():
        y = blk(x)
        _, logits = blk.forward_residual_(x, s2p=s2p)
    ref = R.transition(inp["pair"], p)
    assert_fp32_close(y.cpu(), ref, what="pair transition")
    assert_fp32_close(x.cpu(), inp["pair"] + ref, what="pair transition residual")
    ref_logits = R.single_to_pair(inp["pair"] + ref, sd)
    assert_fp32_close(logits.cpu(), ref_logits, what="fused single_to_pair")


def test_single_attention_and_transition_fp32(dev):
    n = 50
    sd = W.make_block_weights(26, perturb_affine=True)
    inp = W.make_inputs(n, seed=7, pad_last=5)
    pa = sub(sd, "single_attn.")
    sa = attention.SingleAttention(384).to(dev)
    sa.load_state_dict(pa)
    pl = torch.randn(1, 16, n, n, generator=torch.Generator().manual_seed(8))
    st = primitives.TransitionBlock(384, 4).to(dev)
    pt = sub(sd, "single_transition.")
    st.load_state_dict(pt)
    with torch.no_grad():
        got = sa(inp["single"].to(dev), inp["seq_mask"].to(dev), pl.to(dev))
        got_t = st(inp["single"].to(dev))
    ref = R.single_attention(inp["single"], inp["seq_mask"], pl, pa)
    assert_fp32_close(got.cpu(), ref, what="single attention")
    assert_fp32_close(got_t.cpu(), R.transition(inp["single"], pt), what="single transition")


@pytest.mark.parametrize("n,masked", [(37, "all"), (64, "none"), (130, "first")])
def test_single_attention_masking_fp32(dev, n, masked):
    """Key masks: every key masked (uniform attention, the eager rule), none, and a masked first
    key block; N not a multiple of 32 (padding keys) and not of 4 (unaligned pair-logit rows)."""
    sd = W.make_block_weights(27, perturb_affine=True)
    inp = W.make_inputs(n, seed=9)
    seq = torch.ones(1, n)
    if masked == "all":
        seq.zero_()
    elif masked == "first":
        seq[:, :40] = 0
    pa = sub(sd, "single_attn.")
    sa = attention.SingleAttention(384).to(dev)
    sa.load_state_dict(pa)
    pl = 3 * torch.randn(1, 16, n, n, generator=torch.Generator().manual_seed(10))
    with torch.no_grad():
        got = sa(inp["single"].to(dev), seq.to(dev), pl.to(dev))
    ref = R.single_attention(inp["single"], seq, pl, pa)
    assert_fp32_close(got.cpu(), ref, what=f"single attention mask={masked}")


def _block(sd, dev, dtype=torch.float32):
    blk = evoformer.PairFormerBlock(128, 384).to(dev).eval()
    blk.load_state_dict(sd)
    return blk.to(dtype)


def test_block_fp32_matches_reference_golden(dev):
    """The whole block against the reference's own outputs (masked N=24 golden vectors)."""
    g = np.load(os.path.join(GOLDEN, "block_n24_masked.npz"))
    sd = W.make_block_weights(7, perturb_affine=True)
    blk = _block(sd, dev)
    inp = {k: torch.from_numpy(g["in_" + k]).to(dev) for k in ("pair", "single", "pair_mask", "seq_mask")}
    with torch.no_grad():
        pair, single = blk(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"])
    assert_fp32_close(pair.cpu(), torch.from_numpy(g["out_pair"]), what="block pair vs reference")
    assert_fp32_close(single.cpu(), torch.from_numpy(g["out_single"]), what="block single vs reference")


def test_block_fp32_config1(dev):
    """N=64, fp32, weights seed 0, inputs seed 0, full mask."""
    g = np.load(os.path.join(GOLDEN, "block_n64_cfg1.npz"))
    sd = W.make_block_weights(0)
    inp = W.make_inputs(64, seed=0)
    blk = _block(sd, dev)
    with torch.no_grad():
        pair, single = blk(*(inp[k].to(dev) for k in ("pair", "single", "pair_mask", "seq_mask")))
        rp, rs = R.pairformer_block(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], sd)
    assert_fp32_close(pair.cpu(), rp, what="config 1 pair")
    assert_fp32_close(single.cpu(), rs, what="config 1 single")
    assert_fp32_close(single.cpu(), torch.from_numpy(g["out_single"]), what="config 1 single vs reference")
    got = pair.cpu().reshape(-1)[torch.from_numpy(g["pair_sample_idx"])]
    assert rel_l2(got, torch.from_numpy(g["pair_sample_val"])) <= 1e-5


@pytest.mark.parametrize("stream_dtype", [torch.bfloat16, torch.float32])
def test_block_bf16_rule(dev, stream_dtype):
    """bf16 GEMMs, bf16 (bench regime) or fp32 (autocast inference regime) residual stream."""
    n = 80
    sd = W.make_block_weights(27, perturb_affine=True)
    inp = W.make_inputs(n, seed=9, pad_last=8)
    blk = _block(sd, dev, stream_dtype)
    x = [inp[k].to(dev, stream_dtype) if k in ("pair", "single") else inp[k].to(dev) for k in
         ("pair", "single", "pair_mask", "seq_mask")]  # fmt: skip
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        pair, single = blk(*x)
        ep, es = R.pairformer_block(*x, to(sd, dev, stream_dtype))
    rp, rs = R.pairformer_block(*(t.float().cpu() for t in x), sd)
    print("[block bf16 pair]", assert_bf16_rule(pair.cpu(), ep.cpu(), rp, "block pair"), flush=True)
    print("[block bf16 single]", assert_bf16_rule(single.cpu(), es.cpu(), rs, "block single"), flush=True)


def test_block_bf16_batch_items_are_independent(dev):
    """bf16 block on a batch of 2 (ragged N, padding) equals the block on each item alone,
    bit for bit: every persistent kernel indexes batch items inside its flat tile walk
    (tiles straddle the items when N^2 is not a multiple of the tile), so any batch-offset
    mistake changes some position's result."""
    n = 70
    sd = W.make_block_weights(29, perturb_affine=True)
    inp = W.make_inputs(n, seed=10, batch=2, pad_random=5)
    blk = _block(sd, dev, torch.bfloat16)
    x = [inp[k].to(dev, torch.bfloat16) if k in ("pair", "single") else inp[k].to(dev) for k in
         ("pair", "single", "pair_mask", "seq_mask")]  # fmt: skip
    with torch.no_grad():
        pair, single = blk(*x)
        for b in range(2):
            pb, sb = blk(*(t[b : b + 1] for t in x))
            assert torch.equal(pb[0], pair[b]), f"pair, item {b}: max |d| {(pb[0] - pair[b]).abs().max().item()}"
            assert torch.equal(sb[0], single[b]), f"single, item {b}: max |d| {(sb[0] - single[b]).abs().max().item()}"


def test_trunk_two_blocks_fp32(dev):
    blocks = W.make_trunk_weights(31, 2, perturb_affine=True)
    inp = W.make_inputs(32, seed=11, pad_random=3)
    stack = evoformer.PairFormerStack(2).to(dev).eval()
    for blk, sd in zip(stack.blocks, blocks):
        blk.load_state_dict(sd)
    with torch.no_grad():
        pair, single = stack(*(inp[k].to(dev) for k in ("pair", "single", "pair_mask", "seq_mask")))
    rp, rs = R.pairformer_trunk(inp["pair"], inp["single"], inp["pair_mask"], inp["seq_mask"], blocks)
    assert_fp32_close(pair.cpu(), rp, what="trunk pair")
    assert_fp32_close(single.cpu(), rs, what="trunk single")
