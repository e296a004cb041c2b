"""GPU: training-mode semantics of the blocks, and the architectures with deleted branches.

1. The shared-mask dropout-add (``csrc/dropout.hip``) against the oracle: the mask generator bit
   for bit (the oracle's Philox restatement is pinned by the published known-answer vectors in
   ``tests/test_oracle.py``), the fused add and its backward bit for bit, and the applied mask's
   properties (constant along the shared axis, values 0 or 1/(1-p), keep rate 1-p).
2. ``PairFormerBlock`` / ``PairFormerStack`` / ``TemplatePairFormerBlock`` / ``EvoformerBlock`` in
   training mode match the oracle fed the same masks (the masks of the seeds the blocks draw,
   ``kernels.next_dropout_seed``, in the reference's branch order), with and without grad, fp32
   at relL2 and max-abs <= 1e-5; gradients against the oracle differentiated in fp64.
3. Per-block activation checkpointing (``OptimConfig.use_gradient_checkpointing``): a
   checkpointed two-block stack in training mode gives the uncheckpointed outputs and gradients
   bit for bit (the recompute regenerates the same masks), and the blocks do run twice.
4. Blocks without triangle attention and/or the single track (``evoformer.py:226-236``,
   ``:302-321``, ``:353``) against the oracle, and the reference's stage-0 shape (256 pair
   channels in 8 heads, both deleted) loaded from a reference-layout checkpoint, fp32 and the
   bf16 rule.
5. ``SingleAttention`` under grad with a fully masked batch item follows the stock rule
   (uniform weights, the softmax Jacobian there) in the forward and the gradients.
6. A branch module of a scaled block returns the unscaled update from ``forward`` (the
   reference's submodule semantics) and the scaled one from ``branch``.
"""

from __future__ import annotations

import pytest
import torch

from oracle import pairformer_ref as R
from tests._helpers import assert_bf16_rule, assert_fp32_close, mod, rel_l2, sub, to

pytestmark = pytest.mark.gpu
W = mod("weights")
evoformer = mod("evoformer")
kernels = mod("kernels")
config = mod("config")
census = mod("kernel_census")
_lib = mod("_lib")
BF = torch.bfloat16
F32 = torch.float32
STRUCTURAL_ZERO = ("single_to_pair_norm.bias",)
SITES = (("tri_mul_out", True), ("tri_mul_in", True), ("pair_attn_row", True), ("pair_attn_col", False))


@pytest.fixture(autouse=True)
def _highest():
    torch.set_float32_matmul_precision("highest")


# ---------------------------------------------------------------- 1. the kernels
@pytest.mark.parametrize("n,p,seed", [(1, 0.25, 1), (4099, 0.25, (1 << 40) + 3), (100_000, 0.1, 7),
                                      (12_345, 0.5, (1 << 62) + 11)])  # fmt: skip
def test_dropout_mask_matches_oracle(dev, n, p, seed):
    print(f"[dropout mask] n={n} p={p} seed={seed}", flush=True)
    got = torch.empty(n, dtype=F32, device=dev)
    _lib.call("pf_dropout_mask", got.data_ptr(), n, p, seed, _lib.stream_of(got))
    assert torch.equal(got.cpu(), R.dropout_mask(n, p, seed))


@pytest.mark.parametrize("shape", [(2, 37, 41, 128), (1, 5, 33, 64)], ids=["pair", "msa"])
@pytest.mark.parametrize("rowwise", [True, False], ids=["rows", "cols"])
@pytest.mark.parametrize("rdt,xdt", [(F32, F32), (F32, BF), (BF, BF)], ids=["f32", "f32+bf16", "bf16"])
def test_dropout_add_matches_oracle(dev, shape, rowwise, rdt, xdt):
    print(f"[dropout add] shape={shape} rowwise={rowwise} {rdt}/{xdt}", flush=True)
    g = torch.Generator().manual_seed(3)
    res = torch.randn(shape, generator=g).to(rdt)
    x = torch.randn(shape, generator=g).to(xdt)
    seed, p = (5 << 33) + 17, 0.25
    mask = R.shared_dropout_mask(shape, rowwise, p, seed)
    want = R.dropout_add(res, x, mask)
    rd, xd = res.to(dev), x.to(dev)
    assert torch.equal(kernels.dropout_add(rd, xd, p, rowwise, seed).cpu(), want)
    inplace = rd.clone()
    kernels.dropout_add(inplace, xd, p, rowwise, seed, out=inplace)
    assert torch.equal(inplace.cpu(), want)
    assert torch.equal(kernels.dropout_mask(shape, rowwise, p, seed, dev).cpu(), mask)
    # autograd: the residual's cotangent passes through, x's is the cotangent times the mask
    rl, xl = rd.clone().requires_grad_(True), xd.clone().requires_grad_(True)
    out = kernels.DropoutAddFunction.apply(rl, xl, p, rowwise, seed)
    assert torch.equal(out.detach().cpu(), want)
    gout = torch.randn(shape, generator=g).to(rdt)
    out.backward(gout.to(dev))
    assert torch.equal(rl.grad.cpu(), gout)
    assert xl.grad.dtype == xdt
    assert torch.equal(xl.grad.cpu(), (gout.float() * mask).to(xdt))


@pytest.mark.parametrize("rowwise", [True, False], ids=["rows", "cols"])
def test_applied_mask_is_shared_and_scaled(dev, rowwise):
    """With res = 0 and x = 1 the output is the applied mask itself: constant along the shared
    axis, values in {0, 1/(1-p)}, kept at rate 1 - p."""
    shape, p = (2, 64, 96, 128), 0.25
    out = kernels.dropout_add(torch.zeros(shape, device=dev), torch.ones(shape, device=dev), p, rowwise, 99)
    axis = 1 if rowwise else 2
    first = out.select(axis, 0).unsqueeze(axis)
    assert torch.equal(out, first.expand_as(out))
    scale = (torch.tensor(1.0) / (1.0 - torch.tensor(p))).item()  # 1/(1-p) in fp32
    assert set(torch.unique(out).tolist()) == {0.0, scale}
    keep = (first > 0).float().mean().item()
    assert abs(keep - 0.75) < 0.01  # 24576 entries: sd 0.003


# ---------------------------------------------------------------- 2. blocks in training mode
def _inputs(N, seed, c=128, cs=384, fully_masked_single=False):
    g = torch.Generator().manual_seed(seed)
    pair = torch.randn(1, N, N, c, generator=g)
    single = torch.randn(1, N, cs, generator=g)
    pm = (torch.rand(1, N, N, generator=g) > 0.1).float()
    pm[:, :, 0] = 1.0
    pm[:, 0, :] = 1.0
    sm = torch.ones(1, N)
    sm[:, N - 2 :] = 0.0
    gp = torch.randn(1, N, N, c, generator=g)
    gs = torch.randn(1, N, cs, generator=g)
    return pair, single, pm, sm, gp, gs


def _block_masks(shape, p, seed, sites=SITES):
    """The masks a block draws after ``torch.manual_seed(seed)``, one per site, in order."""
    torch.manual_seed(seed)
    return {site: R.shared_dropout_mask(shape, rw, p, kernels.next_dropout_seed()) for site, rw in sites}


def _train_block(sd, dev, p=0.25, **kw):
    blk = evoformer.PairFormerBlock(128, 384, pair_dropout=p, **kw)
    blk.load_state_dict(sd)
    return blk.to(dev).train()


def test_train_block_no_grad_matches_oracle_with_same_masks(dev):
    sd = W.make_block_weights(71, perturb_affine=True)
    blk = _train_block(sd, dev)
    pair, single, pm, sm, _, _ = _inputs(33, 72)
    print("[train block no grad] N=33", flush=True)
    torch.manual_seed(123)
    with torch.no_grad():
        p, s = blk(pair.to(dev), single.to(dev), pm.to(dev), sm.to(dev))
    masks = _block_masks(tuple(pair.shape), 0.25, 123)
    rp, rs = R.pairformer_block(pair, single, pm, sm, sd, dropout=masks)
    e_p, _ = R.pairformer_block(pair, single, pm, sm, sd)
    assert_fp32_close(p.cpu(), rp, what="train block pair")
    assert_fp32_close(s.cpu(), rs, what="train block single")
    assert rel_l2(rp, e_p) > 1e-2  # dropout acts
    # eval mode: no dropout
    with torch.no_grad():
        pe, _ = blk.eval()(pair.to(dev), single.to(dev), pm.to(dev), sm.to(dev))
    assert_fp32_close(pe.cpu(), e_p, what="eval block pair")


def test_train_block_grad_matches_oracle_with_same_masks(dev):
    sd = W.make_block_weights(73, perturb_affine=True)
    blk = _train_block(sd, dev)
    pair, single, pm, sm, gp, gs = _inputs(30, 74)
    print("[train block grad] N=30", flush=True)
    p0, s0 = pair.to(dev).requires_grad_(True), single.to(dev).requires_grad_(True)
    torch.manual_seed(321)
    p, s = blk(p0, s0, pm.to(dev), sm.to(dev))
    ((p * gp.to(dev)).sum() + (s * gs.to(dev)).sum()).backward()
    masks = {k: v.double() for k, v in _block_masks(tuple(pair.shape), 0.25, 321).items()}
    leaves = {k: v.double().clone().requires_grad_(True) for k, v in sd.items()}
    rp0, rs0 = pair.double().requires_grad_(True), single.double().requires_grad_(True)
    rp, rs = R.pairformer_block(rp0, rs0, pm.double(), sm.double(), leaves, dropout=masks)
    ((rp * gp.double()).sum() + (rs * gs.double()).sum()).backward()
    assert_fp32_close(p.detach().cpu(), rp.detach().float(), what="train grad pair")
    assert_fp32_close(s.detach().cpu(), rs.detach().float(), what="train grad single")
    assert_fp32_close(p0.grad.cpu(), rp0.grad.float(), what="train dpair")
    assert_fp32_close(s0.grad.cpu(), rs0.grad.float(), what="train dsingle")
    for k, t in blk.named_parameters():
        if k in STRUCTURAL_ZERO:
            continue
        assert_fp32_close(t.grad.cpu(), leaves[k].grad.float(), what=f"train d{k}")


def test_train_stack_two_streams_matches_oracle(dev):
    """The stack's no-grad path (pair halves on the main stream, single halves on a second)
    in training mode: the masks of block 0 then block 1, as the trunk oracle applies them."""
    sds = W.make_trunk_weights(75, 2, perturb_affine=True)
    stack = evoformer.PairFormerStack(2, 128, 384)
    for blk, sd in zip(stack.blocks, sds):
        blk.load_state_dict(sd)
    stack = stack.to(dev).train()
    pair, single, pm, sm, _, _ = _inputs(26, 76)
    print("[train stack no grad] N=26", flush=True)
    torch.manual_seed(77)
    with torch.no_grad():
        p, s = stack(pair.to(dev), single.to(dev), pm.to(dev), sm.to(dev))
    torch.manual_seed(77)
    drop = [{site: R.shared_dropout_mask(tuple(pair.shape), rw, 0.25, kernels.next_dropout_seed()) for site, rw in SITES}
            for _ in range(2)]  # fmt: skip
    rp, rs = R.pairformer_trunk(pair, single, pm, sm, sds, dropout=drop)
    assert_fp32_close(p.cpu(), rp, what="train stack pair")
    assert_fp32_close(s.cpu(), rs, what="train stack single")


def test_train_template_and_evoformer_blocks_match_oracle(dev):
    sd = W.make_block_weights(78, perturb_affine=True, factor=2)
    tp = {k: v for k, v in sd.items() if k.startswith(("tri_mul_", "pair_attn_", "pair_transition."))}
    tb = evoformer.TemplatePairFormerBlock(128, pair_dropout=0.25)
    tb.load_state_dict(tp)
    tb = tb.to(dev).train()
    pair, _, pm, _, _, _ = _inputs(21, 79)
    print("[train template block] N=21", flush=True)
    torch.manual_seed(5)
    with torch.no_grad():
        got = tb(pair.to(dev), pm.to(dev))
    want = R.template_pairformer_block(pair, pm, tp, dropout=_block_masks(tuple(pair.shape), 0.25, 5))
    assert_fp32_close(got.cpu(), want, what="train template block")

    esd = W.make_evoformer_block_weights(80, perturb_affine=True)
    eb = evoformer.EvoformerBlock(64, 128, msa_dropout=0.15, pair_dropout=0.25)
    eb.load_state_dict(esd)
    eb = eb.to(dev).train()
    g = torch.Generator().manual_seed(81)
    msa = torch.randn(1, 5, 23, 64, generator=g)
    z = torch.randn(1, 23, 23, 128, generator=g)
    mmask = (torch.rand(1, 5, 23, generator=g) > 0.15).float()
    seq = (mmask.max(dim=1).values > 0).float()
    zm = seq[:, :, None] * seq[:, None, :]
    print("[train Evoformer block] S=5 N=23", flush=True)
    torch.manual_seed(6)
    with torch.no_grad():
        gm, gz = eb(msa.to(dev), z.to(dev), mmask.to(dev), zm.to(dev))
    torch.manual_seed(6)
    drop = {"row_attn": R.shared_dropout_mask(tuple(msa.shape), True, 0.15, kernels.next_dropout_seed())}
    drop.update({site: R.shared_dropout_mask(tuple(z.shape), rw, 0.25, kernels.next_dropout_seed()) for site, rw in SITES})
    rm, rz = R.evoformer_block(msa, z, mmask, zm, esd, dropout=drop)
    assert_fp32_close(gm.cpu(), rm, what="train Evoformer msa")
    assert_fp32_close(gz.cpu(), rz, what="train Evoformer pair")


# ---------------------------------------------------------------- 3. checkpointing
def test_checkpointed_stack_equals_uncheckpointed_bit_for_bit(dev):
    sds = W.make_trunk_weights(82, 2, perturb_affine=True)
    pair, single, pm, sm, gp, gs = _inputs(24, 83)
    runs = []
    for ckpt in (False, True):
        stack = evoformer.PairFormerStack(2, 128, 384, optim=config.OptimConfig(use_gradient_checkpointing=ckpt))
        for blk, sd in zip(stack.blocks, sds):
            blk.load_state_dict(sd)
        stack = stack.to(dev).train()
        assert stack.use_gradient_checkpointing == ckpt
        print(f"[checkpointed stack] ckpt={ckpt}", flush=True)
        p0, s0 = pair.to(dev).requires_grad_(True), single.to(dev).requires_grad_(True)
        before = census.snapshot().get("PairFormerBlock", {}).get("hip_block_grad", 0)
        torch.manual_seed(84)
        p, s = stack(p0, s0, pm.to(dev), sm.to(dev))
        ((p * gp.to(dev)).sum() + (s * gs.to(dev)).sum()).backward()
        calls = census.snapshot().get("PairFormerBlock", {}).get("hip_block_grad", 0) - before
        assert calls == (4 if ckpt else 2), calls  # the checkpointed blocks recompute once
        grads = {k: t.grad.clone() for k, t in stack.named_parameters()}
        runs.append((p.detach(), s.detach(), p0.grad, s0.grad, grads))
    (pa, sa, dpa, dsa, ga), (pb, sb, dpb, dsb, gb) = runs
    assert torch.equal(pa, pb) and torch.equal(sa, sb)
    assert torch.equal(dpa, dpb) and torch.equal(dsa, dsb)
    for k in ga:
        assert torch.equal(ga[k], gb[k]), k


# ---------------------------------------------------------------- 4. deleted branches
@pytest.mark.parametrize("attn,single", [(False, True), (True, False), (False, False)],
                         ids=["no-attn", "no-single", "neither"])  # fmt: skip
def test_block_without_branches_fp32(dev, attn, single):
    sd = W.make_block_weights(85, perturb_affine=True, use_triangle_attention=attn, use_single_track=single)
    blk = evoformer.PairFormerBlock(128, 384, use_triangle_attention=attn, use_single_track=single)
    blk.load_state_dict(sd)
    blk = blk.to(dev).eval()
    pair, sgl, pm, sm, gp, gs = _inputs(29, 86)
    print(f"[block without branches] attn={attn} single={single}", flush=True)
    with torch.no_grad():
        p, s = blk(pair.to(dev), sgl.to(dev), pm.to(dev), sm.to(dev))
        stack = evoformer.PairFormerStack(1, 128, 384, use_triangle_attention=attn, use_single_track=single)
        stack.blocks[0].load_state_dict(sd)
        ps, ss = stack.to(dev).eval()(pair.to(dev), sgl.to(dev), pm.to(dev), sm.to(dev))
    rp, rs = R.pairformer_block(pair, sgl, pm, sm, sd, use_triangle_attention=attn, use_single_track=single)
    assert_fp32_close(p.cpu(), rp, what="pair")
    assert torch.equal(ps, p) and torch.equal(ss, s)
    if single:
        assert_fp32_close(s.cpu(), rs, what="single")
    else:
        assert torch.equal(s.cpu(), sgl)
    # under grad, training mode: the sites that remain take dropout
    sites = tuple(x for x in SITES if attn or not x[0].startswith("pair_attn"))
    blk.train()
    p0, s0 = pair.to(dev).requires_grad_(True), sgl.to(dev).requires_grad_(True)
    torch.manual_seed(87)
    p, s = blk(p0, s0, pm.to(dev), sm.to(dev))
    loss = (p * gp.to(dev)).sum() + ((s * gs.to(dev)).sum() if single else 0.0)
    loss.backward()
    masks = {k: v.double() for k, v in _block_masks(tuple(pair.shape), 0.25, 87, sites).items()}
    leaves = {k: v.double().clone().requires_grad_(True) for k, v in sd.items()}
    rp0, rs0 = pair.double().requires_grad_(True), sgl.double().requires_grad_(True)
    rp, rs = R.pairformer_block(rp0, rs0, pm.double(), sm.double(), leaves, dropout=masks,
                                use_triangle_attention=attn, use_single_track=single)  # fmt: skip
    rloss = (rp * gp.double()).sum() + ((rs * gs.double()).sum() if single else 0.0)
    rloss.backward()
    assert_fp32_close(p.detach().cpu(), rp.detach().float(), what="train pair")
    assert_fp32_close(p0.grad.cpu(), rp0.grad.float(), what="dpair")
    for k, t in blk.named_parameters():
        if k not in STRUCTURAL_ZERO:
            assert_fp32_close(t.grad.cpu(), leaves[k].grad.float(), what=f"d{k}")


def _stage0_trunk(tmp_path, dev, dtype):
    from tests.test_checkpoint import write_stage0_checkpoint

    ck = mod("checkpoint")
    path = tmp_path / "stage0.safetensors"
    sd = write_stage0_checkpoint(path)
    trunk, _ = ck.load_trunk(path, device=dev, dtype=dtype)
    blocks = [sub(sd, f"evoformer.trunk_pairformer.{i}.") for i in range(2)]
    return trunk, blocks, sd, path


def test_stage0_shape_trunk_fp32_and_bf16(dev, tmp_path):
    """The reference's stage-0 trunk shape (configs/stage0.yaml:62-71): 256 pair channels in 8
    heads, no triangle attention, no single track, two layers from a reference-layout file."""
    flags = dict(use_triangle_attention=False, use_single_track=False)
    trunk, blocks, _, path = _stage0_trunk(tmp_path, dev, None)
    pair, single, pm, sm, _, _ = _inputs(40, 88, c=256)
    print("[stage0 trunk fp32] N=40 C=256", flush=True)
    with torch.no_grad():
        p, s = trunk(pair.to(dev), single.to(dev), pm.to(dev), sm.to(dev))
    rp, rs = R.pairformer_trunk(pair, single, pm, sm, blocks, **flags)
    assert_fp32_close(p.cpu(), rp, what="stage0 pair")
    assert torch.equal(s.cpu(), single)

    ck = mod("checkpoint")
    tb, _ = ck.load_trunk(path, device=dev, dtype=BF)
    pair, single, pm, sm, _, _ = _inputs(96, 89, c=256)
    pd, sd_, pmd, smd = pair.to(dev), single.to(dev), pm.to(dev), sm.to(dev)
    print("[stage0 trunk bf16] N=96 C=256", flush=True)
    with torch.no_grad():
        p, _ = tb(pd.to(BF), sd_.to(BF), pmd, smd)
        with torch.autocast("cuda", dtype=BF):
            ep, _ = R.pairformer_trunk(pd.to(BF), sd_.to(BF), pmd, smd, [to(b, dev, BF) for b in blocks], **flags)
        rp, _ = R.pairformer_trunk(pd, sd_, pmd, smd, [to(b, dev) for b in blocks], **flags)
    print("  ", assert_bf16_rule(p.cpu(), ep.cpu(), rp.cpu(), "stage0 pair bf16"), flush=True)


def test_evoformer_block_without_triangle_attention(dev):
    esd = W.make_evoformer_block_weights(90, perturb_affine=True, use_triangle_attention=False)
    eb = evoformer.EvoformerBlock(64, 128, use_triangle_attention=False)
    eb.load_state_dict(esd)
    eb = eb.to(dev).eval()
    g = torch.Generator().manual_seed(91)
    msa, z = torch.randn(1, 4, 19, 64, generator=g), torch.randn(1, 19, 19, 128, generator=g)
    mmask = (torch.rand(1, 4, 19, generator=g) > 0.15).float()
    seq = (mmask.max(dim=1).values > 0).float()
    zm = seq[:, :, None] * seq[:, None, :]
    print("[Evoformer block without attention]", flush=True)
    with torch.no_grad():
        gm, gz = eb(msa.to(dev), z.to(dev), mmask.to(dev), zm.to(dev))
    rm, rz = R.evoformer_block(msa, z, mmask, zm, esd, use_triangle_attention=False)
    assert_fp32_close(gm.cpu(), rm, what="msa")
    assert_fp32_close(gz.cpu(), rz, what="pair")


# ---------------------------------------------------------------- 5. single attention, masked item
def test_single_attention_fully_masked_item_under_grad(dev):
    """Batch item 1 has every key masked: the stock path's -1e9-shifted logits round to one
    value, so it attends uniformly (mean of V) and its gradients are the uniform softmax's
    Jacobian; the HIP forward and backward follow that rule (fp32, against fp64 autograd)."""
    sd = W.make_block_weights(92, perturb_affine=True)
    p = sub(sd, "single_attn.")
    m = mod("attention").SingleAttention(384)
    m.load_state_dict(p)
    m = m.to(dev)
    g = torch.Generator().manual_seed(93)
    B, N = 2, 37
    x = torch.randn(B, N, 384, generator=g)
    pl = torch.randn(B, 16, N, N, generator=g)
    mask = torch.ones(B, N)
    mask[0, -5:] = 0.0
    mask[1] = 0.0
    dy = torch.randn(B, N, 384, generator=g)
    print("[single attention, fully masked item, grad]", flush=True)
    xd, pld = x.to(dev).requires_grad_(True), pl.to(dev).requires_grad_(True)
    y = m(xd, mask.to(dev), pld)
    (y * dy.to(dev)).sum().backward()
    leaves = {k: v.double().clone().requires_grad_(True) for k, v in p.items()}
    xr, plr = x.double().requires_grad_(True), pl.double().requires_grad_(True)
    yr = R.single_attention(xr, mask.double(), plr, leaves)
    (yr * dy.double()).sum().backward()
    assert_fp32_close(y.detach().cpu(), yr.detach().float(), what="y")
    assert float(yr.detach()[1].abs().max()) > 0  # the masked item is not zero
    assert_fp32_close(xd.grad.cpu(), xr.grad.float(), what="dx")
    assert_fp32_close(pld.grad.cpu(), plr.grad.float(), what="dpair_logits")
    assert float(plr.grad[1].abs().max()) > 0  # and its gradients are not either
    for k, t in m.named_parameters():
        assert_fp32_close(t.grad.cpu(), leaves[k].grad.float(), what=f"d{k}")


# ---------------------------------------------------------------- 6. scaled blocks' submodules
def test_scaled_block_submodules_return_unscaled_updates(dev):
    sd = W.make_block_weights(94, perturb_affine=True)
    blk = evoformer.PairFormerBlock(128, 384, residual_out_scale=0.5, pair_transition_residual_gain=0.8)
    blk.load_state_dict(sd)
    blk = blk.to(dev).eval()
    pair, single, pm, sm, _, _ = _inputs(27, 95)
    z, mask = pair.to(dev), pm.to(dev)
    print("[scaled block submodules]", flush=True)
    for grad in (False, True):
        with torch.set_grad_enabled(grad):
            u_out = blk.tri_mul_out(z, mask)
            u_row = blk.pair_attn_row(z, mask)
            u_pt = blk.pair_transition(z)
            b_out = blk.tri_mul_out.branch(z, mask)
            b_pt = blk.pair_transition.branch(z)
        assert_fp32_close(u_out.detach().cpu(), R.tri_mul(pair, pm, sub(sd, "tri_mul_out."), True), what="tri_mul_out")
        assert_fp32_close(u_row.detach().cpu(), R.grid_attention(pair, pm, sub(sd, "pair_attn_row."), False),
                          what="pair_attn_row")  # fmt: skip
        assert_fp32_close(u_pt.detach().cpu(), R.transition(pair, sub(sd, "pair_transition.")), what="transition")
        assert_fp32_close(b_out.detach().cpu(), 0.5 * u_out.detach().cpu(), what="scaled tri_mul_out")
        assert_fp32_close(b_pt.detach().cpu(), 0.4 * u_pt.detach().cpu(), what="scaled transition")
