"""GPU: the benchmark configurations at their full sizes, against the oracle run on the GPU.

Config 2: one block, N=384, bf16, last 32 tokens padded (masked rows and columns compared too).
Config 3: triangle multiplication out then in, N=1024, bf16, full mask.
Config 4: the 48-block trunk, N=768, bf16, 5 % random padding -- z and s after one block and
          after 48.
Config 5: N=2048 attention: the kernel-level op with pair bias ~ N(0,1) and 10 % of key columns
          masked (the reference kernel tests' inputs, test_evo_attn_robustness.py:231-281), the
          row/column grid-attention modules on sampled lines (rows are independent, so a line
          subset of the oracle is exact), and the single attention with N=2048 pair logits.

bf16 rule (the reference's, tests/triton/test_fused_trimul.py:66-83): relL2(HIP - fp32 oracle)
<= 2 x relL2(eager bf16 - fp32 oracle), with the fp32 oracle evaluated at matmul precision
"highest". Max-abs errors are printed beside it.
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, max_abs, mod, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
ops = mod("ops")
attention = mod("attention")
evoformer = mod("evoformer")
fused = mod("fused")
BF = torch.bfloat16


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


def _report(tag, got, eager, ref):
    e_k, e_s = assert_bf16_rule(got.cpu(), eager.cpu(), ref.cpu(), tag)
    print(f"[{tag}] relL2 hip={e_k:.3e} eager_bf16={e_s:.3e} maxabs hip={max_abs(got, ref):.3e} "
          f"eager_bf16={max_abs(eager, ref):.3e}", flush=True)  # fmt: skip


def _inputs(dev, cfg):
    inp = W.make_inputs(**W.CONFIGS[cfg])
    return {k: v.to(dev) for k, v in inp.items()}


def test_config2_block_n384_bf16_padded(dev):
    print("[config 2] N=384 block bf16, last 32 tokens padded", flush=True)
    sd = W.make_block_weights(1)
    x = _inputs(dev, 2)
    assert x["seq_mask"][0, 352:].sum() == 0 and x["seq_mask"][0, :352].min() == 1
    blk = evoformer.PairFormerBlock(128, 384).to(dev).eval()
    blk.load_state_dict(sd)
    blk = blk.to(BF)
    xb = [x["pair"].to(BF), x["single"].to(BF), x["pair_mask"], x["seq_mask"]]
    with torch.no_grad():
        pair, single = blk(*xb)
        with torch.autocast("cuda", dtype=BF):
            ep, es = R.pairformer_block(*xb, to(sd, dev, BF))
        rp, rs = R.pairformer_block(xb[0].float(), xb[1].float(), x["pair_mask"], x["seq_mask"], to(sd, dev),
                                    row_chunk=128)  # fmt: skip
    assert torch.isfinite(pair).all() and torch.isfinite(single).all()
    _report("config 2 pair", pair, ep, rp)
    _report("config 2 single", single, es, rs)
    # the padded rows/columns follow the eager rule too (fully masked lines average V)
    _report("config 2 pair, padded rows", pair[:, 352:], ep[:, 352:], rp[:, 352:])


def test_config3_trimul_n1024_bf16(dev):
    print("[config 3] N=1024 trimul out then in, bf16", flush=True)
    sd = W.make_block_weights(2)
    x = _inputs(dev, 3)
    zb, mb = x["pair"].to(BF), x["pair_mask"].to(BF)
    mods = []
    for name, cls in (("tri_mul_out.", ops.TriangleMulOutgoing), ("tri_mul_in.", ops.TriangleMulIncoming)):
        m = cls(128).to(dev)
        m.load_state_dict(sub(sd, name))
        mods.append(m.to(BF))
    pout, pin = sub(sd, "tri_mul_out."), sub(sd, "tri_mul_in.")
    with torch.no_grad():
        z1 = zb + mods[0](zb, mb)
        got = z1 + mods[1](z1, mb)
        e1 = zb + R.tri_mul(zb, mb, to(pout, dev, BF), True)
        eager = e1 + R.tri_mul(e1, mb, to(pin, dev, BF), False)
        r1 = zb.float() + R.tri_mul(zb.float(), x["pair_mask"], to(pout, dev), True)
        ref = r1 + R.tri_mul(r1, x["pair_mask"], to(pin, dev), False)
    _report("config 3 outgoing update", z1 - zb, e1 - zb, r1 - zb.float())
    _report("config 3 out+in", got, eager, ref)


def test_config4_trunk48_n768_bf16(dev):
    print("[config 4] N=768 48-block trunk bf16, 5 % padding", flush=True)
    n_blocks = 48
    sds = W.make_trunk_weights(3, n_blocks)
    x = _inputs(dev, 4)
    assert int((x["seq_mask"] == 0).sum()) == 38
    stack = evoformer.PairFormerStack(n_blocks).eval()
    for blk, sd in zip(stack.blocks, sds):
        blk.load_state_dict(sd)
    stack = stack.to(dev).to(BF)
    pm, sm = x["pair_mask"], x["seq_mask"]
    sd_bf = [to(sd, dev, BF) for sd in sds]
    sd_32 = [to(sd, dev) for sd in sds]
    with torch.no_grad():
        p, s = x["pair"].to(BF), x["single"].to(BF)
        ep, es = p, s
        rp, rs = p.float(), s.float()
        for i in range(n_blocks):
            p, s = stack.blocks[i](p, s, pm, sm)
            with torch.autocast("cuda", dtype=BF):
                ep, es = R.pairformer_block(ep, es, pm, sm, sd_bf[i])
            rp, rs = R.pairformer_block(rp, rs, pm, sm, sd_32[i], row_chunk=192)
            if i == 0:
                _report("config 4 pair after 1 block", p, ep, rp)
                _report("config 4 single after 1 block", s, es, rs)
            if (i + 1) % 12 == 0:
                print(f"[config 4] block {i + 1} |z|max={rp.abs().max().item():.1f}", flush=True)
    assert torch.isfinite(p).all() and torch.isfinite(s).all()
    _report("config 4 pair after 48 blocks", p, ep, rp)
    _report("config 4 single after 48 blocks", s, es, rs)
    # The path bench.py times: PairFormerStack.forward runs block i's single half on a
    # second stream beside block i + 1's pair half. It must give the block-by-block result
    # bit for bit (the kernels have no atomics and a static tiling).
    del ep, es, rp, rs
    with torch.no_grad():
        sp, ss = stack(x["pair"].to(BF), x["single"].to(BF), pm, sm)
    torch.cuda.synchronize()
    print("[config 4] two-stream stack vs block by block:", torch.equal(sp, p), torch.equal(ss, s), flush=True)
    assert torch.equal(sp, p), f"pair differs, max {(sp.float() - p.float()).abs().max().item():.3e}"
    assert torch.equal(ss, s), f"single differs, max {(ss.float() - s.float()).abs().max().item():.3e}"


def _evo_inputs_n2048(dev):
    B, S, N, H, D = 1, 2048, 2048, 4, 32
    g = torch.Generator(device=dev).manual_seed(4)
    shape = (B, S, N, H, D)
    Q = (torch.randn(shape, device=dev, generator=g) * D**-0.5).to(BF)
    K = (torch.randn(shape, device=dev, generator=g) * D**-0.5).to(BF)
    V = torch.randn(shape, device=dev, generator=g).to(BF)
    pb = torch.randn((B, 1, H, N, N), device=dev, generator=g)
    cols = torch.randperm(N, generator=torch.Generator().manual_seed(4))[: int(round(0.1 * N))]
    rm = torch.zeros((B, S, 1, 1, N), device=dev)
    rm[..., cols.to(dev)] = -1e9
    return Q, K, V, rm, pb


def _evo_lines_ref(Q, K, V, rm, pb, lines, dtype):
    """Eager attention on a line subset: [B, S, N, H, D] inputs, rows of the fp32/bf16 formula."""
    D = Q.shape[-1]
    q, k, v = (t[:, lines].transpose(-2, -3).to(dtype).contiguous() for t in (Q, K, V))  # [B, L, H, N, D]
    logits = torch.matmul(q, k.transpose(-1, -2).contiguous()) * D**-0.5
    logits = logits.float() + pb + rm[:, lines]
    w = torch.softmax(logits, dim=-1).to(dtype)
    return torch.matmul(w, v).transpose(-2, -3)  # [B, L, N, H, D]


def test_config5_evo_attention_n2048(dev):
    print("[config 5] kernel op N=2048, bias ~ N(0,1), 10 % key columns masked", flush=True)
    Q, K, V, rm, pb = _evo_inputs_n2048(dev)
    with torch.no_grad():
        out = fused._EvoformerAttention.apply(Q, K, V, rm, pb)
    assert out.shape == Q.shape and out.dtype == BF
    lines = torch.tensor([0, 1, 511, 1024, 1777, 2047], device=dev)
    got = out[:, lines]
    eager = _evo_lines_ref(Q, K, V, rm, pb, lines, BF)
    ref = _evo_lines_ref(Q, K, V, rm, pb, lines, torch.float32)
    _report("config 5 evo attention (6 lines)", got, eager, ref)


@pytest.mark.parametrize("transpose", [False, True])
def test_config5_grid_attention_n2048_sampled_lines(dev, transpose):
    print(f"[config 5] GridSelfAttention N=2048 transpose={transpose}", flush=True)
    N = 2048
    sd = W.make_block_weights(4)
    p = sub(sd, "pair_attn_col." if transpose else "pair_attn_row.")
    g = torch.Generator(device=dev).manual_seed(4)
    z = torch.randn((1, N, N, 128), device=dev, generator=g).to(BF)
    keep = torch.ones(N, device=dev)
    keep[torch.randperm(N, generator=torch.Generator().manual_seed(5))[: int(round(0.1 * N))].to(dev)] = 0.0
    # 10 % of key columns masked in the attended frame: no query line is fully masked
    mask = (keep[:, None] * torch.ones(N, device=dev)[None, :]) if transpose else keep[None, :].expand(N, N)
    mask = mask.contiguous()[None]
    m = attention.GridSelfAttention(128, 4, transpose=transpose).to(dev)
    m.load_state_dict(p)
    m = m.to(BF)
    lines = torch.tensor([0, 3, 700, 1500, 2047], device=dev)
    with torch.no_grad():
        out = m(z, mask.to(BF))
        got = out[:, :, lines].transpose(1, 2) if transpose else out[:, lines]
        with torch.autocast("cuda", dtype=BF):
            eager = R.grid_attention(z, mask.to(BF), to(p, dev, BF), transpose, lines=lines)
        ref = R.grid_attention(z.float(), mask, to(p, dev), transpose, lines=lines)
    _report(f"config 5 grid attention transpose={transpose} (5 lines)", got, eager, ref)


def test_config5_single_attention_n2048(dev):
    print("[config 5] SingleAttention N=2048 with pair logits", flush=True)
    N = 2048
    sd = W.make_block_weights(4)
    pa = sub(sd, "single_attn.")
    g = torch.Generator(device=dev).manual_seed(6)
    s = torch.randn((1, N, 384), device=dev, generator=g).to(BF)
    pl = torch.randn((1, 16, N, N), device=dev, generator=g)
    seq = torch.ones((1, N), device=dev)
    seq[0, torch.randperm(N, generator=torch.Generator().manual_seed(7))[:205].to(dev)] = 0.0
    sa = attention.SingleAttention(384).to(dev)
    sa.load_state_dict(pa)
    sa = sa.to(BF)
    with torch.no_grad():
        got = sa(s, seq, pl)
        with torch.autocast("cuda", dtype=BF):
            eager = R.single_attention(s, seq, pl.to(BF), to(pa, dev, BF))
        ref = R.single_attention(s.float(), seq, pl, to(pa, dev))
    _report("config 5 single attention", got, eager, ref)
